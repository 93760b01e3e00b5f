"""Seeded synthetic inputs for the MLA decode path.

The reference draws Q* and C from ``torch.randn`` after ``torch.manual_seed(42)``
(mla.py:42, :107, :110), so its values depend on torch's RNG implementation
and on the order of draws. Here inputs come from numpy's PCG64 generator with
an explicit seed per array, so the same seed gives the same values on this
host, on the GPU box and in the C oracle. Values are N(0, 1) rounded to the
requested storage type (fp16 inputs are exactly representable, so fp32 copies
of them feed the fp32 oracle without any further rounding).
"""
from __future__ import annotations

import numpy as np

HEAD_DIM_K = 576
HEAD_DIM_V = 512


def normal(shape, seed: int, dtype=np.float16) -> np.ndarray:
    """N(0, 1) samples of the given shape from PCG64(seed), rounded to dtype."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal(size=shape, dtype=np.float32).astype(dtype)


def decode_inputs(num_heads: int, seq_length: int, seed: int = 42,
                  dtype=np.float16):
    """Q* [num_heads, 576] and C [seq_length, 576] for one decode step."""
    q = normal((num_heads, HEAD_DIM_K), seed, dtype)
    c = normal((seq_length, HEAD_DIM_K), seed + 1, dtype)
    return q, c


def batched_seqlens(batch: int, lo: int = 512, hi: int = 16384,
                    seed: int = 42) -> np.ndarray:
    """N_b drawn uniformly from [lo, hi] (inclusive) by seed."""
    rng = np.random.Generator(np.random.PCG64(seed + 1000))
    return rng.integers(lo, hi, size=batch, endpoint=True).astype(np.int64)


def batched_inputs(num_heads: int, seqlens, seed: int = 42, dtype=np.float16):
    """Q* [B, num_heads, 576], packed C [sum N_b, 576] and cu_seqlens [B + 1]
    (int32) for a batch of independent sequences."""
    seqlens = np.asarray(seqlens, dtype=np.int64)
    batch = seqlens.shape[0]
    cu = np.zeros(batch + 1, dtype=np.int32)
    cu[1:] = np.cumsum(seqlens)
    q = normal((batch, num_heads, HEAD_DIM_K), seed, dtype)
    c = normal((int(cu[-1]), HEAD_DIM_K), seed + 1, dtype)
    return q, c, cu
