"""GPU parity of the projections around the decode (mla_absorb_query_*,
mla_project_output_*) against the float64 oracle, and of the whole decode step
of an MLA block (absorb -> batched decode -> project) against attention
computed without weight absorption (oracle.block_unabsorbed). The reference
has no code for these projections (README.md:64-110 gives the math), so the
oracle is textbook GEMM plus the absorption identity, itself pinned on the CPU
(tests/test_oracle.py).

Tolerances: fp16 atol = rtol = 1e-2 (products of up to 16384 terms
accumulated in fp32, rounded to fp16 once per GEMM); bf16 atol = rtol = 3e-2
(8 significant bits per stored intermediate).
"""
import numpy as np
import pytest
import torch

from ada_mla import capi, synthetic
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale, dtype):
    t = torch.from_numpy(synthetic.normal(shape, seed, np.float32) * np.float32(scale)).to(dtype)
    return t.cuda(), t.double().numpy()


@pytest.mark.parametrize("dtype,tol", [(torch.float16, 1e-2), (torch.bfloat16, 3e-2)])
@pytest.mark.parametrize("b,n_h", [(1, 16), (5, 128), (32, 16), (70, 32), (2, 1), (3, 3)])
def test_absorb_query(dtype, tol, b, n_h):
    print(f"absorb {dtype} B={b} n_h={n_h}", flush=True)
    qn, qn_d = _rand((b, n_h, 128), 1, 1.0, dtype)
    qr, qr_d = _rand((b, n_h, 64), 2, 1.0, dtype)
    w, w_d = _rand((n_h, 128, 512), 3, 128 ** -0.5, dtype)
    got = capi.absorb_query(qn, qr, w)
    torch.cuda.synchronize()
    got = got.double().cpu().numpy()
    want = O.absorb_query(qn_d, qr_d, w_d)
    np.testing.assert_allclose(got, want, atol=tol, rtol=tol)
    # the rope columns are copied exactly
    assert np.array_equal(got[:, :, 512:], qr_d)


@pytest.mark.parametrize("dtype,tol", [(torch.float16, 1e-2), (torch.bfloat16, 3e-2)])
# The W_O kernel cuts its (64-column unit, K-chunk) steps into equal ranges,
# one per workgroup; on a 256-CU MI355X: (32, 128, 5120), the block workload,
# splits units between 3-4 workgroups; (33, 16, 1000) one unit over 8 (two
# row groups); (256, 16, 8192) and (5, 1, 256) keep every unit in one
# workgroup (direct stores, no reduction); n_h = 1 and 3 end K in a
# 128-column chunk, (4, 3, 1000) with that chunk in a split unit.
@pytest.mark.parametrize("b,n_h,d_model", [(1, 16, 256), (4, 128, 5120), (33, 16, 1000), (70, 32, 512),
                                           (32, 128, 5120), (256, 16, 8192), (5, 1, 256), (4, 3, 1000)])
def test_project_output(dtype, tol, b, n_h, d_model):
    print(f"project {dtype} B={b} n_h={n_h} d_model={d_model}", flush=True)
    o, o_d = _rand((b, n_h, 512), 4, 1.0, dtype)
    wuv, wuv_d = _rand((n_h, 128, 512), 5, 512 ** -0.5, dtype)
    wo, wo_d = _rand((d_model, n_h * 128), 6, (n_h * 128) ** -0.5, dtype)
    got = capi.project_output(o, wuv, wo)
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.double().cpu().numpy(), O.project_output(o_d, wuv_d, wo_d), atol=tol, rtol=tol)


@pytest.mark.parametrize("n_h", [16, 128])
def test_decode_block_equals_unabsorbed_attention(n_h):
    # absorb -> batched decode -> project, against per-head attention with
    # explicit keys C_N W_UK[h]^T and values C_N W_UV[h]^T
    print(f"block n_h={n_h}", flush=True)
    import ada_mla
    dt = torch.float16
    seqlens = np.array([300, 0, 1, 2048])
    q32, c32, cu = synthetic.batched_inputs(n_h, seqlens, seed=13, dtype=np.float32)
    c = torch.from_numpy(c32).to(dt)
    qn, qn_d = _rand((4, n_h, 128), 7, 1.0, dt)
    qr, qr_d = _rand((4, n_h, 64), 8, 1.0, dt)
    wuk, wuk_d = _rand((n_h, 128, 512), 9, 128 ** -0.5, dt)
    wuv, wuv_d = _rand((n_h, 128, 512), 10, 512 ** -0.5, dt)
    wo, wo_d = _rand((1024, n_h * 128), 11, (n_h * 128) ** -0.5, dt)
    q_star = ada_mla.mla_absorb_query(qn, qr, wuk)
    o_star = ada_mla.mla_decode_split_batched(q_star, c.cuda(), torch.from_numpy(cu).cuda())
    out = ada_mla.mla_project_output(o_star, wuv, wo)
    torch.cuda.synchronize()
    want = O.block_unabsorbed(qn_d, qr_d, c.double().numpy(), cu, wuk_d, wuv_d, wo_d)
    got = out.double().cpu().numpy()
    assert not got[1].any()  # the empty sequence
    np.testing.assert_allclose(got, want, atol=1e-2, rtol=1e-2)
    rel = np.abs(got - want).mean() / np.abs(want).mean()
    assert rel < 1e-2, rel
