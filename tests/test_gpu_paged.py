"""GPU parity of the paged-KV decode (mla_decode_paged_fp16 / _bf16, and the
extension's mla_decode_paged) against the closed form on the gathered
sequences, and against the packed batched entry on the same logical data.
The reference has no paged cache; the oracle is closed_form_paged (the
per-sequence closed form after gathering rows through the block table).

Pages are random permutations of a pool with spare pages; block-table
columns past a sequence's pages hold out-of-range ids that must never be
read. Tolerances as for the packed paths: fp16 atol = rtol = 1e-2 with mean
relative error < 5e-3; bf16 atol = rtol = 1e-2 with mean relative error < 1e-2.
"""
import numpy as np
import pytest
import torch

from ada_mla import capi, synthetic
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _check(got, ref, rel_bar, what=""):
    assert np.isfinite(got).all(), what
    np.testing.assert_allclose(got, ref, atol=TOL, rtol=TOL, err_msg=what)
    rel = np.abs(got - ref).mean() / max(np.abs(ref).mean(), 1e-30)
    assert rel < rel_bar, f"{what}: mean relative error {rel:.3e}"


def _paged(n_h, seqlens, page, seed, dtype=torch.float16, splits=0):
    q, kv, bt, cu, c = synthetic.paged_inputs(n_h, seqlens, page, seed=seed, dtype=np.float32)
    qt = torch.from_numpy(q).to(dtype).cuda()
    kvt = torch.from_numpy(kv).to(dtype).cuda()
    out = capi.decode_paged(qt, kvt, torch.from_numpy(bt).cuda(), torch.from_numpy(cu).cuda(),
                            int(cu[-1]), num_splits=splits)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    # the oracle sees exactly the values the kernel read
    qd = qt.double().cpu().numpy()
    kvd = kvt.double().cpu().numpy()
    return out.double().cpu().numpy(), O.closed_form_paged(qd, kvd, bt, cu), seqlens


def _check_all(got, ref, seqlens, rel_bar, what):
    for b, n in enumerate(seqlens):
        if n == 0:
            assert not got[b].any(), f"{what} seq {b} (empty)"
        else:
            _check(got[b], ref[b], rel_bar, f"{what} seq {b} N={n}")


EDGE = [5, 0, 31, 32, 33, 1, 63, 64, 65, 127, 128, 129, 300, 1000]


@pytest.mark.parametrize("page", [32, 64, 128, 256])
@pytest.mark.parametrize("splits", [0, 1, 7, 100])
def test_paged_fp16_edges(page, splits):
    print(f"paged fp16 page={page} splits={splits}", flush=True)
    got, ref, n = _paged(128, EDGE, page, seed=page + splits, splits=splits)
    _check_all(got, ref, n, 5e-3, f"page={page} splits={splits}")


@pytest.mark.parametrize("n_h", [16, 32, 48])
def test_paged_head_counts(n_h):
    print(f"paged n_h={n_h}", flush=True)
    got, ref, n = _paged(n_h, [700, 3, 64, 2000], 64, seed=n_h, splits=5)
    _check_all(got, ref, n, 5e-3, f"n_h={n_h}")


@pytest.mark.parametrize("page", [32, 64])
def test_paged_bf16(page):
    print(f"paged bf16 page={page}", flush=True)
    got, ref, n = _paged(128, EDGE, page, seed=77, dtype=torch.bfloat16, splits=7)
    _check_all(got, ref, n, 1e-2, f"bf16 page={page}")


@pytest.mark.parametrize("page,dtype", [(32, torch.float16), (256, torch.float16), (64, torch.bfloat16)])
def test_paged_long_sequences(page, dtype):
    # long sequences at 128 heads: the planner takes 64-head tiles, whose O
    # waves feed the ring and read the block table a step ahead
    seqlens = [9000, 0, 15000, 33, 12000, 1, 8000, 16000]
    print(f"paged long page={page} {dtype}", flush=True)
    got, ref, n = _paged(128, seqlens, page, seed=page, dtype=dtype)
    _check_all(got, ref, n, 5e-3 if dtype == torch.float16 else 1e-2, f"long page={page}")


# chunks spanning three or more sequences, with pieces that load their
# successor's Q* and first blocks (>= 4 blocks) and pieces that do not
MANY_PIECES = [130, 200, 0, 150, 300, 129, 40, 260, 140, 0, 500, 97, 1000, 33, 160, 128, 1, 255]


@pytest.mark.parametrize("n_h", [16, 128])
@pytest.mark.parametrize("page", [32, 64])
@pytest.mark.parametrize("splits,dtype", [(1, torch.float16), (2, torch.float16), (3, torch.bfloat16)])
def test_paged_chunks_spanning_many_pieces(n_h, page, splits, dtype):
    print(f"paged many pieces n_h={n_h} page={page} splits={splits} {dtype}", flush=True)
    got, ref, lens = _paged(n_h, np.array(MANY_PIECES), page, seed=23, dtype=dtype, splits=splits)
    _check_all(got, ref, lens, 5e-3 if dtype == torch.float16 else 1e-2, f"paged many pieces {dtype}")


def test_paged_config5_shape():
    seqlens = synthetic.batched_seqlens(32, seed=42)
    print(f"paged config 5 total={int(seqlens.sum())}", flush=True)
    got, ref, n = _paged(128, seqlens, 64, seed=42)
    _check_all(got, ref, n, 5e-3, "config 5 paged")


def test_paged_equals_packed_batched():
    # the same logical data through both layouts: block origins differ (the
    # paged kernel starts blocks at page-aligned tokens), so the results agree
    # to rounding, not bitwise
    seqlens = [900, 0, 33, 4100, 64]
    q, kv, bt, cu, c = synthetic.paged_inputs(128, seqlens, 64, seed=5)
    qt, kvt, ct = (torch.from_numpy(a).cuda() for a in (q, kv, c))
    cut = torch.from_numpy(cu).cuda()
    for splits in (0, 3, 40):
        a = capi.decode_paged(qt, kvt, torch.from_numpy(bt).cuda(), cut, int(cu[-1]), num_splits=splits)
        b = capi.decode_split_batched_fp16(qt, ct, cut, num_splits=splits)
        torch.cuda.synchronize()
        assert (a.float() - b.float()).abs().max().item() < 2e-3, splits


def test_paged_all_empty_and_extension():
    import ada_mla
    q = torch.randn(3, 16, 576, dtype=torch.float16, device="cuda")
    kv = torch.randn(2, 32, 576, dtype=torch.float16, device="cuda")
    bt = torch.zeros(3, 1, dtype=torch.int32, device="cuda")
    cu = torch.zeros(4, dtype=torch.int32, device="cuda")
    out = ada_mla.mla_decode_paged(q, kv, bt, cu)
    torch.cuda.synchronize()
    assert out.shape == (3, 16, 512) and not out.any()
    # extension == C ABI, with total_tokens read from the device or given
    qn, kvn, btn, cun, _ = synthetic.paged_inputs(32, [100, 257], 32, seed=8)
    qt, kvt = torch.from_numpy(qn).cuda(), torch.from_numpy(kvn).cuda()
    btt, cut = torch.from_numpy(btn).cuda(), torch.from_numpy(cun).cuda()
    a = ada_mla.mla_decode_paged(qt, kvt, btt, cut)
    b = ada_mla.mla_decode_paged(qt, kvt, btt, cut, total_tokens=int(cun[-1]))
    c = capi.decode_paged(qt, kvt, btt, cut, int(cun[-1]))
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)


def test_paged_bad_page_ids_stay_in_bounds():
    # ids outside [0, num_pages) are clamped: the result is meaningless, but
    # the call completes and leaves finite values (no access outside the cache)
    q = torch.randn(1, 16, 576, dtype=torch.float16, device="cuda")
    kv = torch.randn(4, 32, 576, dtype=torch.float16, device="cuda")
    bt = torch.tensor([[-5, 1 << 30, 2]], dtype=torch.int32, device="cuda")
    cu = torch.tensor([0, 90], dtype=torch.int32, device="cuda")
    out = capi.decode_paged(q, kv, bt, cu, 90)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
