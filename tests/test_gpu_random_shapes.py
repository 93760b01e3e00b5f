"""GPU parity over seeded random shapes: head counts that are any multiple of
16 up to 256, lengths up to 20000, requested or planned split counts, ragged
batches with empty sequences, and the fp16, bf16 and fp8 caches, all through
the C ABI against the float64 closed form (mla.py:44-47) of each sequence on
the values the kernel read. The fixed shape sweeps elsewhere pin the block
and split edges; these cases reach the planner's other head tiles and chunk
counts. Bars: fp16 and fp8 atol = rtol = 1e-2 with mean relative error
< 5e-3; bf16 the same atol / rtol with mean relative error < 1e-2 (8
significant bits).
"""
import numpy as np
import pytest
import torch

from ada_mla import capi
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu

N_CASES = 36


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    for i in range(N_CASES):
        kind = ["fp16", "bf16", "fp8"][i % 3]
        n_h = 16 * int(rng.integers(1, 17))
        batched = bool(rng.integers(0, 2))
        if batched:
            b = int(rng.integers(1, 7))
            lens = [int(x) for x in rng.integers(0, 6000, size=b)]
            if rng.integers(0, 3) == 0:
                lens[int(rng.integers(0, b))] = 0
        else:
            lens = [int(rng.integers(1, 20001))]
        splits = 0 if rng.integers(0, 2) else int(rng.integers(1, 300))
        out.append((i, kind, n_h, lens, batched, splits))
    return out


def _check(got, want, rel_bar, what):
    assert np.isfinite(got).all(), what
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2, err_msg=what)
    rel = np.abs(got - want).mean() / max(np.abs(want).mean(), 1e-30)
    assert rel < rel_bar, f"{what}: mean relative error {rel:.3e}"


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}-{c[1]}-h{c[2]}-{'b' if c[4] else 's'}{len(c[3])}")
def test_random_shape(case):
    i, kind, n_h, lens, batched, splits = case
    print(f"random case {i}: {kind} n_h={n_h} lens={lens} batched={batched} splits={splits}", flush=True)
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(1000 + i)
    total = sum(lens)
    b = len(lens)
    q32 = rng.standard_normal((b, n_h, 576), dtype=np.float32)
    c32 = rng.standard_normal((max(total, 1), 576), dtype=np.float32)[:total]
    if kind == "fp8":
        scale = 0.5
        q = torch.from_numpy(q32).half().to(dev)
        c = torch.from_numpy(c32 / np.float32(scale)).to(torch.float8_e4m3fn).to(dev)
        c_vals = c.float().cpu().numpy().astype(np.float64) * scale
    else:
        dt = torch.float16 if kind == "fp16" else torch.bfloat16
        q = torch.from_numpy(q32).to(dt).to(dev)
        c = torch.from_numpy(c32).to(dt).to(dev)
        c_vals = c.float().cpu().numpy().astype(np.float64)
    q_vals = q.float().cpu().numpy().astype(np.float64)
    if batched:
        cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
        if kind == "fp16":
            out = capi.decode_split_batched_fp16(q, c, cu, num_splits=splits)
        elif kind == "bf16":
            out = capi.decode_split_batched_bf16(q, c, cu, num_splits=splits)
        else:
            out = capi.decode_split_batched_fp8(q, c, scale, cu, num_splits=splits)
    else:
        if kind == "fp16":
            out = capi.decode_split_fp16(q[0], c, num_splits=splits)
        elif kind == "bf16":
            out = capi.decode_split_bf16(q[0], c, num_splits=splits)
        else:
            out = capi.decode_split_fp8(q[0], c, scale, num_splits=splits)
        out = out[None]
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().astype(np.float64)
    rel_bar = 1e-2 if kind == "bf16" else 5e-3
    lo = 0
    for s, n in enumerate(lens):
        what = f"case {i} sequence {s} (N={n})"
        if n == 0:
            assert not got[s].any(), what + ": an empty sequence gives zeros"
        else:
            _check(got[s], O.closed_form(q_vals[s], c_vals[lo:lo + n]), rel_bar, what)
        lo += n
