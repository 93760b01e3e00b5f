"""GPU parity of the bf16 KV-cache path (mla_decode_split_bf16 and
mla_decode_split_batched_bf16) against the float64 closed form on the same
bf16-valued inputs. The reference has no bf16 path (README.md:405-408 lists it
as future work), so the closed form is the oracle here.

Tolerance: atol = rtol = 1e-2 as for fp16, and a mean relative error below
1e-2: bf16 keeps 8 significant bits, so the output's own rounding is about
2e-3 relative, and P and the split partials are bf16 as well.
"""
import numpy as np
import pytest
import torch

from ada_mla import capi, synthetic
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2
REL_MEAN = 1e-2


def _bf16_inputs(n_h, n, seed):
    """bf16 tensors on the GPU and their exact float64 values."""
    q = torch.from_numpy(synthetic.normal((n_h, 576), seed, np.float32)).to(torch.bfloat16)
    c = torch.from_numpy(synthetic.normal((n, 576), seed + 1, np.float32)).to(torch.bfloat16)
    return q.cuda(), c.cuda(), q.double().numpy(), c.double().numpy()


def _run(q, c, **kw):
    out = capi.decode_split_bf16(q, c, **kw)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    return out.double().cpu().numpy()


def _check(got, ref, what=""):
    assert np.isfinite(got).all(), what
    np.testing.assert_allclose(got, ref, atol=TOL, rtol=TOL, err_msg=what)
    rel = np.abs(got - ref).mean() / max(np.abs(ref).mean(), 1e-30)
    assert rel < REL_MEAN, f"{what}: mean relative error {rel:.3e}"


@pytest.mark.parametrize("n_h", [16, 32, 48, 128])
@pytest.mark.parametrize("n", [1, 17, 33, 100, 1000, 4097])
def test_bf16_shapes(n_h, n):
    print(f"bf16 n_h={n_h} N={n}", flush=True)
    q, c, qd, cd = _bf16_inputs(n_h, n, seed=300 + n)
    _check(_run(q, c), O.closed_form(qd, cd), f"n_h={n_h} N={n}")


@pytest.mark.parametrize("n_h,n", [(128, 4096), (128, 65536), (16, 32768)])
def test_bf16_benchmark_shapes(n_h, n):
    print(f"bf16 config n_h={n_h} N={n}", flush=True)
    q, c, qd, cd = _bf16_inputs(n_h, n, seed=42)
    _check(_run(q, c), O.closed_form(qd, cd), f"n_h={n_h} N={n}")


def test_bf16_split_count_invariance():
    q, c, qd, cd = _bf16_inputs(128, 3000, seed=31)
    ref = O.closed_form(qd, cd)
    for s in [1, 3, 16, 1000]:
        print(f"bf16 splits={s}", flush=True)
        _check(_run(q, c, num_splits=s), ref, f"splits={s}")


def test_bf16_single_token_is_exact():
    q, c, _, cd = _bf16_inputs(32, 1, seed=3)
    assert np.array_equal(_run(q, c), np.repeat(cd[:, :512], 32, axis=0))


def test_bf16_values_beyond_fp16_range():
    # bf16 keeps fp32's exponent range: a cache scaled by 2^20 (far beyond
    # fp16's 65504) must come back scaled by 2^20 -- the bf16 partials hold it
    q, c, qd, cd = _bf16_inputs(16, 500, seed=17)
    scale = 2.0 ** 20
    cs = (c.float() * scale).to(torch.bfloat16)
    qs = (q.float() / scale).to(torch.bfloat16)  # keeps the logits of the unscaled case
    got = _run(qs, cs)
    _check(got / scale, O.closed_form(qs.double().cpu().numpy(), cs.double().cpu().numpy()) / scale,
           "scaled by 2^20")


def test_bf16_batched_many_items_with_empty():
    # 24 sequences x 128 heads: more combine items than resident waves, so
    # each combine wave merges several tiles of a sequence
    seqlens = np.random.default_rng(8).integers(2, 600, size=24)
    seqlens[::5] = 0
    seqlens[2] = 1
    q32, c32, cu = synthetic.batched_inputs(128, seqlens, seed=10, dtype=np.float32)
    q = torch.from_numpy(q32).to(torch.bfloat16)
    c = torch.from_numpy(c32).to(torch.bfloat16)
    out = capi.decode_split_batched_bf16(q.cuda(), c.cuda(), torch.from_numpy(cu).cuda(), num_splits=9)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    ref = O.closed_form_batched(q.double().numpy(), c.double().numpy(), cu)
    for b in range(len(seqlens)):
        if seqlens[b] == 0:
            assert not got[b].any()
        else:
            _check(got[b], ref[b], f"seq {b}")


@pytest.mark.parametrize("splits", [0, 3])
def test_bf16_batched_ragged_with_empty(splits):
    seqlens = np.array([5, 0, 17, 1, 300, 64, 0, 1000, 33])
    q32, c32, cu = synthetic.batched_inputs(128, seqlens, seed=9, dtype=np.float32)
    q = torch.from_numpy(q32).to(torch.bfloat16)
    c = torch.from_numpy(c32).to(torch.bfloat16)
    out = capi.decode_split_batched_bf16(q.cuda(), c.cuda(), torch.from_numpy(cu).cuda(), num_splits=splits)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    ref = O.closed_form_batched(q.double().numpy(), c.double().numpy(), cu)
    for b in range(len(seqlens)):
        if seqlens[b] == 0:
            assert not got[b].any()
        else:
            _check(got[b], ref[b], f"seq {b}")


@pytest.mark.parametrize("n_h,splits", [(32, 1), (128, 2)])
def test_bf16_batched_chunks_spanning_many_pieces(n_h, splits):
    # chunks over three or more sequences: pieces of >= 4 blocks load their
    # successor's Q* and first blocks during their last steps
    seqlens = np.array([130, 200, 0, 150, 300, 129, 40, 260, 140, 0, 500, 97, 1000, 33, 160, 128, 1, 255])
    q32, c32, cu = synthetic.batched_inputs(n_h, seqlens, seed=22, dtype=np.float32)
    q = torch.from_numpy(q32).to(torch.bfloat16)
    c = torch.from_numpy(c32).to(torch.bfloat16)
    out = capi.decode_split_batched_bf16(q.cuda(), c.cuda(), torch.from_numpy(cu).cuda(), num_splits=splits)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    ref = O.closed_form_batched(q.double().numpy(), c.double().numpy(), cu)
    for b in range(len(seqlens)):
        if seqlens[b] == 0:
            assert not got[b].any()
        else:
            _check(got[b], ref[b], f"seq {b}")


def test_bf16_extension_dispatch():
    import ada_mla
    q, c, _, _ = _bf16_inputs(128, 1500, seed=13)
    a = ada_mla.mla_decode_split(q, c)
    b = capi.decode_split_bf16(q, c)
    torch.cuda.synchronize()
    assert a.dtype == torch.bfloat16 and torch.equal(a, b)
    cu = torch.tensor([0, 700, 1500], dtype=torch.int32, device="cuda")
    qb = torch.stack([q, q])
    got = ada_mla.mla_decode_split_batched(qb, c, cu)
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16 and got.shape == (2, 128, 512)
    one = capi.decode_split_bf16(q.contiguous(), c[700:].contiguous())
    torch.cuda.synchronize()
    assert (got[1].float() - one.float()).abs().max().item() < 2e-2
