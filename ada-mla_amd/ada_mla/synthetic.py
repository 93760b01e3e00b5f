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


def paged_inputs(num_heads: int, seqlens, page_size: int, seed: int = 42, dtype=np.float16,
                 spare_pages: int = 3, spare_columns: int = 2):
    """A paged cache holding the same logical data as batched_inputs(num_heads,
    seqlens, seed, dtype): Q* [B, num_heads, 576], kv_pages
    [num_pages, page_size, 576], block_table [B, max_pages + spare_columns]
    (int32; every sequence's pages are a random permutation of the pool, the
    spare columns and pages are filled with values no sequence reads),
    cu_seqlens [B + 1] (int32), and the packed cache itself."""
    q, c, cu = batched_inputs(num_heads, seqlens, seed, dtype)
    seqlens = np.diff(cu.astype(np.int64))
    need = [-(-int(n) // page_size) for n in seqlens]
    n_pages = sum(need) + spare_pages
    rng = np.random.Generator(np.random.PCG64(seed + 2000))
    perm = rng.permutation(n_pages)
    kv = normal((n_pages, page_size, HEAD_DIM_K), seed + 3, dtype)  # unread rows keep random data
    cols = max(need + [1]) + spare_columns
    bt = np.full((len(seqlens), cols), n_pages + 7, dtype=np.int32)  # out-of-range: never read
    k = 0
    for b, n in enumerate(seqlens):
        for j in range(need[b]):
            page = int(perm[k])
            k += 1
            bt[b, j] = page
            rows = c[cu[b] + j * page_size: cu[b] + min((j + 1) * page_size, int(n))]
            kv[page, :rows.shape[0]] = rows
    return q, kv, bt, cu, c
