"""One-launch decode: a single-sequence 16-bit call whose plan has one split
runs only the split kernel, which writes the output itself (no partials, no
combine). Checked against the float64 oracle to the fp16 contract
(atol = rtol = 1e-2, mean relative error < 5e-3) and against the two-launch
path on the same plan (MLA_FLAG_TWO_LAUNCHES: the same split kernel writing a
partial, then combine_kernel), which differs from it by the combine's fp32
rescale of the one partial and its rounding to fp16.
"""
import numpy as np
import pytest
import torch

from ada_mla import capi, synthetic
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu

F16_TOL = 1e-2
F16_REL_MEAN = 5e-3
ONE_PARTIAL_TOL = 2e-3  # one partial through the combine: one more fp16 rounding


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda:0"))


def _check16(got, ref, what=""):
    assert np.isfinite(got).all(), what
    np.testing.assert_allclose(got, ref, atol=F16_TOL, rtol=F16_TOL, err_msg=what)
    rel = np.abs(got - ref).mean() / max(np.abs(ref).mean(), 1e-30)
    assert rel < F16_REL_MEAN, f"{what}: mean relative error {rel:.3e}"


def _fp16(q, c, **kw):
    out = capi.decode_split_fp16(_t(q), _t(c), **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("n_h,n,splits", [(128, 1, 0), (128, 31, 0), (128, 32, 0), (128, 33, 0), (128, 128, 0),
                                          (16, 100, 0), (64, 200, 0), (48, 77, 0), (1024, 40, 0), (128, 4096, 1),
                                          (16, 3000, 1)])
def test_one_launch_vs_oracle_and_two_launches(n_h, n, splits):
    lib = capi.load()
    print(f"one launch n_h={n_h} N={n} splits={splits}", flush=True)
    assert lib.mla_decode_split_launches(n_h, n, splits, 0) == 1
    q, c = synthetic.decode_inputs(n_h, n, seed=900 + n_h + n)
    one = _fp16(q, c, num_splits=splits)
    two = _fp16(q, c, num_splits=splits, flags=capi.FLAG_TWO_LAUNCHES)
    _check16(one, O.closed_form(q, c), f"one launch n_h={n_h} N={n}")
    assert np.abs(one - two).max() <= ONE_PARTIAL_TOL


def test_one_launch_single_token_is_exact():
    # one token: softmax weight 1, the output is that row's C_N exactly
    q, c = synthetic.decode_inputs(128, 1, seed=931)
    assert np.array_equal(_fp16(q, c), np.repeat(c[:, :512].astype(np.float32), 128, axis=0))


def test_one_launch_fp32_partials_flag():
    # the partial precision flag does not apply: no partials are stored
    q, c = synthetic.decode_inputs(128, 100, seed=932)
    a = _fp16(q, c)
    b = _fp16(q, c, flags=capi.FLAG_FP32_PARTIALS)
    assert np.array_equal(a, b)


def test_one_launch_one_hot_coverage():
    # every token of the single split reaches the output: a dominant logit on
    # token j gives C_N[j]
    n_h, n = 16, 150
    q, c = synthetic.decode_inputs(n_h, n, seed=933)
    for j in (0, 31, 32, 77, 149):
        qj = (np.tile(c[j], (n_h, 1)).astype(np.float32) * 8.0).astype(np.float16)
        got = _fp16(qj, c)
        _check16(got, O.closed_form(qj, c), f"one-hot token {j}")


def test_bf16_and_fp8_one_launch():
    import ada_mla
    for n_h, n in [(128, 100), (16, 1), (64, 200)]:
        q, c = synthetic.decode_inputs(n_h, n, seed=1010 + n)
        qb = _t(q.astype(np.float32)).to(torch.bfloat16)
        cb = _t(c.astype(np.float32)).to(torch.bfloat16)
        got = ada_mla.mla_decode_split(qb, cb).float().cpu().numpy()
        ref = O.closed_form(qb.float().cpu().numpy(), cb.float().cpu().numpy())
        np.testing.assert_allclose(got, ref, atol=F16_TOL, rtol=F16_TOL)
        scale = 0.5
        c8 = (_t(c).float() / scale).to(torch.float8_e4m3fn)
        got8 = ada_mla.mla_decode_split(_t(q), c8, cache_scale=scale).float().cpu().numpy()
        ref8 = O.closed_form(q, c8.float().cpu().numpy().astype(np.float64) * scale)
        _check16(got8, ref8, f"fp8 n_h={n_h} N={n}")
