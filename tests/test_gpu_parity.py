"""GPU parity of the HIP decode path against the CPU oracle, through the C ABI
(ada_mla.capi -> libmla_mi355x.so) unless a test says otherwise.

Tolerances (from the decode contract): fp16 outputs atol = rtol = 1e-2 against
the float64 closed form on the same (fp16-valued) inputs; the fp32 path
atol = rtol = 1e-4. Because |O*| is small at long N (about 0.02 at N = 65536),
every fp16 case also has to meet a tighter mean relative error
(mean |diff| / mean |ref|, the reference's `rel` metric, mla.py:118) of 5e-3,
and token coverage is checked exactly by one-hot sweeps.
"""
import math

import numpy as np
import pytest
import torch

from ada_mla import capi, synthetic
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu

F16_TOL = 1e-2
F32_TOL = 1e-4
F16_REL_MEAN = 5e-3


def _dev():
    return torch.device("cuda:0")


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(_dev())


def _fp16(q, c, **kw):
    out = capi.decode_split_fp16(_t(q), _t(c), **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _fp32(q, c, **kw):
    out = capi.decode_fused_fp32(_t(q), _t(c), **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check16(got, ref, what=""):
    assert np.isfinite(got).all(), what
    np.testing.assert_allclose(got, ref, atol=F16_TOL, rtol=F16_TOL, err_msg=what)
    rel = np.abs(got - ref).mean() / max(np.abs(ref).mean(), 1e-30)
    assert rel < F16_REL_MEAN, f"{what}: mean relative error {rel:.3e}"


def _check32(got, ref, what=""):
    assert np.isfinite(got).all(), what
    np.testing.assert_allclose(got, ref, atol=F32_TOL, rtol=F32_TOL, err_msg=what)


# ------------------------------------------------------------ golden vectors

def test_golden_fp16(golden):
    for name, case in golden.items():
        print(f"golden fp16 {name}", flush=True)
        _check16(_fp16(case["q"], case["c"]), case["contract"], name)


def test_golden_fp32(golden):
    for name, case in golden.items():
        print(f"golden fp32 {name}", flush=True)
        q = case["q"].astype(np.float32)
        c = case["c"].astype(np.float32)
        _check32(_fp32(q, c), case["contract"], name)


# --------------------------------------------------------- shapes and edges

@pytest.mark.parametrize("n_h", [16, 32, 48, 128])
@pytest.mark.parametrize("n", [1, 15, 16, 17, 31, 33, 63, 64, 65, 100, 257, 1000, 4097])
def test_fp16_shapes(n_h, n):
    print(f"fp16 n_h={n_h} N={n}", flush=True)
    q, c = synthetic.decode_inputs(n_h, n, seed=100 + n)
    _check16(_fp16(q, c), O.closed_form(q, c), f"n_h={n_h} N={n}")


@pytest.mark.parametrize("n_h", [16, 128])
@pytest.mark.parametrize("n", [1, 15, 17, 100, 1024, 3000])
def test_fp32_shapes(n_h, n):
    print(f"fp32 n_h={n_h} N={n}", flush=True)
    q, c = synthetic.decode_inputs(n_h, n, seed=200 + n)
    q, c = q.astype(np.float32), c.astype(np.float32)
    _check32(_fp32(q, c), O.closed_form(q, c), f"n_h={n_h} N={n}")


@pytest.mark.parametrize("n_h,n", [(128, 16384), (128, 20001), (32, 65536 + 7), (64, 32768 + 5), (48, 20000)])
def test_fp32_long_sequences(n_h, n):
    # long sequences: the fp32 plan takes 32-head workgroups where n_h allows
    # (two 16-head sub-tiles per wave), 16-head ones at n_h = 48
    print(f"fp32 n_h={n_h} N={n}", flush=True)
    q, c = synthetic.decode_inputs(n_h, n, seed=300 + n)
    q, c = q.astype(np.float32), c.astype(np.float32)
    _check32(_fp32(q, c), O.closed_form(q, c), f"n_h={n_h} N={n}")


@pytest.mark.parametrize("n_h", [32, 128])
def test_fp32_split_count_invariance(n_h):
    # requested split counts walk the fp32 kernel through both head tiles
    # (32 heads once a chunk holds >= 192 tokens: 1, 2, 3, 7 splits here),
    # one-block pieces (200 splits: 16-token chunks, the S and O roles each
    # idle for one of the two steps) and a ragged last block (N = 3001)
    q, c = synthetic.decode_inputs(n_h, 3001, seed=33)
    q, c = q.astype(np.float32), c.astype(np.float32)
    ref = O.closed_form(q, c)
    outs = []
    for s in [1, 2, 3, 7, 16, 64, 200]:
        print(f"fp32 n_h={n_h} splits={s}", flush=True)
        outs.append(_fp32(q, c, num_splits=s))
        _check32(outs[-1], ref, f"n_h={n_h} splits={s}")
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() < 1e-5


@pytest.mark.parametrize("n_h", [1024, 4096])
@pytest.mark.parametrize("n", [1, 200])
def test_many_heads(n_h, n):
    # up to the largest head count the entry points accept (4096): 64 head
    # tiles of 64 heads, more combine items than resident waves
    print(f"many heads n_h={n_h} N={n}", flush=True)
    q, c = synthetic.decode_inputs(n_h, n, seed=400 + n)
    ref = O.closed_form(q, c)
    _check16(_fp16(q, c), ref, f"fp16 n_h={n_h} N={n}")
    q32, c32 = q.astype(np.float32), c.astype(np.float32)
    _check32(_fp32(q32, c32), O.closed_form(q32, c32), f"fp32 n_h={n_h} N={n}")


def test_many_heads_batched():
    lens = [130, 0, 1]
    q, c, cu = synthetic.batched_inputs(4096, lens, seed=9)
    out = capi.decode_split_batched_fp16(_t(q), _t(c), torch.from_numpy(cu).cuda())
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    _check16(got, O.closed_form_batched(q, c, cu), "batched n_h=4096")
    assert (got[1] == 0).all()


def test_fp32_matches_c_restatement_of_reference_cpu_kernel():
    q, c = synthetic.decode_inputs(128, 1024, seed=7, dtype=np.float32)
    _check32(_fp32(q, c), O.naive_cpu(q, c), "vs naive_cpu")


def test_transpose_read_equals_scalar_read():
    # the two ways of reading C_N^T feed identical MFMA operands
    # (the scalar read is built for the two-launch path only)
    for n_h, n in [(16, 200), (128, 1000), (32, 77)]:
        q, c = synthetic.decode_inputs(n_h, n, seed=n)
        a = _fp16(q, c, flags=capi.FLAG_TWO_LAUNCHES)
        b = _fp16(q, c, flags=capi.FLAG_SCALAR_TRANSPOSE)
        assert np.array_equal(a, b), (n_h, n)


@pytest.mark.parametrize("n_h", [16, 128])
def test_split_count_invariance(n_h):
    q, c = synthetic.decode_inputs(n_h, 3000, seed=31)
    ref = O.closed_form(q, c)
    outs = []
    for s in [1, 2, 3, 7, 16, 64, 1000]:
        print(f"splits={s}", flush=True)
        outs.append(_fp16(q, c, num_splits=s))
        _check16(outs[-1], ref, f"splits={s}")
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() < 2e-3


@pytest.mark.parametrize("n_h,n,splits", [(128, 4096, 0), (128, 1000, 8), (16, 3000, 0), (32, 777, 5)])
def test_one_hot_token_coverage(n_h, n, splits):
    # make token j dominant for every head: the output must be C_N[j]; j runs
    # over block, chunk and sequence boundaries so no token can be skipped
    rng = np.random.default_rng(5)
    c = (rng.standard_normal((n, 576)) * 0.1).astype(np.float16)
    cand = sorted({0, 1, 15, 16, 31, 32, 33, 63, 64, n // 2, n - 2, n - 1} | set(range(0, n, max(1, n // 17))))
    for j in [k for k in cand if 0 <= k < n]:
        q = np.repeat((c[j:j + 1].astype(np.float32) * 400.0).astype(np.float16), n_h, axis=0)
        got = _fp16(q, c, num_splits=splits)
        want = np.repeat(c[j:j + 1, :512].astype(np.float32), n_h, axis=0)
        np.testing.assert_allclose(got, want, atol=2e-3, rtol=0, err_msg=f"token {j}")


def test_single_token_is_exact():
    q, c = synthetic.decode_inputs(128, 1, seed=3)
    got = _fp16(q, c)
    assert np.array_equal(got, np.repeat(c[:, :512].astype(np.float32), 128, axis=0))


def test_equal_rows_and_zero_query():
    _, c1 = synthetic.decode_inputs(16, 1, seed=4)
    c = np.repeat(c1, 500, axis=0)
    q, _ = synthetic.decode_inputs(16, 1, seed=5)
    np.testing.assert_allclose(_fp16(q, c), np.repeat(c1[:, :512].astype(np.float32), 16, 0), atol=1e-3, rtol=0)
    _, c = synthetic.decode_inputs(16, 700, seed=6)
    q0 = np.zeros((16, 576), np.float16)
    _check16(_fp16(q0, c), O.closed_form(q0, c), "q = 0")


def test_large_and_very_negative_logits():
    q, c = synthetic.decode_inputs(32, 2000, seed=8)
    big = (q.astype(np.float32) * 6).astype(np.float16)  # logits ~ +-40: sharp softmax
    _check16(_fp16(big, c), O.closed_form(big, c), "sharp")
    # every logit far below zero (the reference's max init ~ 0 underflows here)
    c_pos = np.abs(c)
    neg = -np.full((32, 576), 0.5, np.float16)
    _check16(_fp16(neg, c_pos), O.closed_form(neg, c_pos), "all logits << 0")


# -------------------------------------------------------- benchmark configs

def test_config2_n4096():
    q, c = synthetic.decode_inputs(128, 4096, seed=42)
    _check16(_fp16(q, c), O.closed_form(q, c), "config 2")


def test_config3_n65536():
    q, c = synthetic.decode_inputs(128, 65536, seed=42)
    _check16(_fp16(q, c), O.closed_form(q, c), "config 3")


def test_config4_nh16_n32768():
    q, c = synthetic.decode_inputs(16, 32768, seed=42)
    _check16(_fp16(q, c), O.closed_form(q, c), "config 4")


def test_config1_fp32_n1024():
    q, c = synthetic.decode_inputs(128, 1024, seed=42, dtype=np.float32)
    _check32(_fp32(q, c), O.closed_form(q, c), "config 1")


# ------------------------------------------------------------------ batched

def _batched(q, c, cu, **kw):
    out = capi.decode_split_batched_fp16(_t(q), _t(c), _t(cu), **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("splits", [0, 1, 3, 50])
def test_batched_ragged_with_empty(splits):
    seqlens = np.array([5, 0, 17, 1, 300, 64, 0, 1000, 33])
    q, c, cu = synthetic.batched_inputs(128, seqlens, seed=9)
    got = _batched(q, c, cu, num_splits=splits)
    ref = O.closed_form_batched(q, c, cu)
    for b in range(len(seqlens)):
        if seqlens[b] == 0:
            assert not got[b].any()
        else:
            _check16(got[b], ref[b], f"seq {b}")


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp8"])
@pytest.mark.parametrize("n,splits", [(100, 0), (100, 1), (3000, 1), (3000, 0)])
def test_batched_single_sequence(dtype, n, splits):
    # a batch of one sequence: one-split plans once took the one-launch path,
    # which does not take cu_seqlens, and the call failed with nothing computed
    print(f"batched B=1 {dtype} N={n} splits={splits}", flush=True)
    q, c, cu = synthetic.batched_inputs(128, np.array([n]), seed=31 + n)
    if dtype == "fp8":
        c8 = torch.from_numpy(c.astype(np.float32) * np.float32(2.0)).to(torch.float8_e4m3fn)
        cd = c8.float().double().numpy() * 0.5
        out = capi.decode_split_batched_fp8(_t(q), c8.to(_dev()), 0.5, _t(cu), num_splits=splits)
        ref = O.closed_form_batched(q, cd, cu)
    elif dtype == "bf16":
        qb, cb = torch.from_numpy(q.astype(np.float32)).bfloat16(), torch.from_numpy(c.astype(np.float32)).bfloat16()
        out = capi.decode_split_batched_bf16(qb.to(_dev()), cb.to(_dev()), _t(cu), num_splits=splits)
        ref = O.closed_form_batched(qb.double().numpy(), cb.double().numpy(), cu)
    else:
        out = capi.decode_split_batched_fp16(_t(q), _t(c), _t(cu), num_splits=splits)
        ref = O.closed_form_batched(q, c, cu)
    torch.cuda.synchronize()
    _check16(out.float().cpu().numpy()[0], ref[0], f"B=1 {dtype} N={n} splits={splits}")


def test_batched_all_empty():
    q, _, _ = synthetic.batched_inputs(16, np.array([1, 1]), seed=1)
    cu = np.zeros(3, np.int32)
    got = _batched(q, np.zeros((0, 576), np.float16), cu)
    assert not got.any()


def test_config5_batched():
    seqlens = synthetic.batched_seqlens(32, seed=42)
    q, c, cu = synthetic.batched_inputs(128, seqlens, seed=42)
    got = _batched(q, c, cu)
    for b in range(32):
        lo, hi = cu[b], cu[b + 1]
        _check16(got[b], O.closed_form(q[b], c[lo:hi]), f"config 5 seq {b} N={hi - lo}")


def test_config5_lengths_at_16_heads():
    # config 5's lengths with 16 heads (a tensor-parallel share of 128): the
    # planner's plan is stream-bound and takes every CU, 256 chunks over 32
    # sequences, so many chunks hold two or three pieces
    seqlens = synthetic.batched_seqlens(32, seed=42)
    q, c, cu = synthetic.batched_inputs(16, seqlens, seed=43)
    got = _batched(q, c, cu)
    ref = O.closed_form_batched(q, c, cu)
    for b in range(32):
        _check16(got[b], ref[b], f"16 heads, config 5 seq {b} N={cu[b + 1] - cu[b]}")


@pytest.mark.parametrize("n_h,batch,splits", [(128, 24, 0), (128, 24, 7), (128, 24, 200), (16, 160, 0), (48, 48, 13)])
def test_batched_many_items_with_empty(n_h, batch, splits):
    # more (16 x 16 tile, sequence) items than the combine keeps resident
    # (4096): each combine wave merges several tiles of one sequence
    rng = np.random.default_rng(31 + n_h + splits)
    seqlens = rng.integers(2, 700, size=batch)
    seqlens[::7] = 0
    seqlens[3::11] = 1
    seqlens[5] = 2500
    q, c, cu = synthetic.batched_inputs(n_h, seqlens, seed=5)
    got = _batched(q, c, cu, num_splits=splits)
    ref = O.closed_form_batched(q, c, cu)
    for b in range(batch):
        if seqlens[b] == 0:
            assert not got[b].any(), f"empty seq {b}"
        else:
            _check16(got[b], ref[b], f"seq {b} N={seqlens[b]}")


# Chunks that span three or more sequences (pieces). A piece of at least 4
# blocks (128 tokens) with a successor loads the successor's Q* and first
# blocks into the ring slots it frees in its last steps; shorter pieces leave
# their successor to load its own; both kinds follow each other here, with
# empty sequences between. Requested split counts fix the chunk length
# (ceil(ceil(total / splits) / 32) * 32 tokens), so the test checks that it
# covers what it claims.
MANY_PIECES = np.array([130, 200, 0, 150, 300, 129, 40, 260, 140, 0, 500, 97, 1000, 33, 160, 128, 1, 255])


# Piece costs the planner may charge per sequence start (virtual tokens, by
# head tile); chunks cut the virtual length (token t of sequence b at
# t + cost (b + 1)) into equal parts.
PIECE_COSTS = (192, 224, 288)


def _chunk_bounds(seqlens, splits, cost):
    """Real token ranges of the chunks of a requested split count: a
    restatement of the planner's chunking and the kernel's virtual bounds."""
    cu = np.concatenate([[0], np.cumsum(seqlens)])
    total_v = int(cu[-1]) + cost * len(seqlens)
    chunk = -(-(-(-total_v // splits)) // 32) * 32

    def real(x):  # first real token at or after virtual position x
        for b in range(len(seqlens)):
            if cu[b + 1] + cost * (b + 1) > x:
                return max(int(cu[b]), x - cost * (b + 1))
        return int(cu[-1])
    return [(real(v), real(v + chunk)) for v in range(0, total_v, chunk)]


def _max_pieces_per_chunk(seqlens, splits):
    cu = np.concatenate([[0], np.cumsum(seqlens)])
    most = []
    for cost in PIECE_COSTS:
        m = 0
        for lo, hi in _chunk_bounds(seqlens, splits, cost):
            m = max(m, sum(1 for b in range(len(seqlens)) if max(cu[b], lo) < min(cu[b + 1], hi)))
        most.append(m)
    return min(most)


@pytest.mark.parametrize("n_h", [16, 32, 64, 128])
@pytest.mark.parametrize("splits", [1, 2, 3])
def test_batched_chunks_spanning_many_pieces(n_h, splits):
    assert _max_pieces_per_chunk(MANY_PIECES, splits) >= 3
    print(f"many pieces n_h={n_h} splits={splits}", flush=True)
    q, c, cu = synthetic.batched_inputs(n_h, MANY_PIECES, seed=21)
    got = _batched(q, c, cu, num_splits=splits)
    ref = O.closed_form_batched(q, c, cu)
    for b, n in enumerate(MANY_PIECES):
        if n == 0:
            assert not got[b].any(), f"empty seq {b}"
        else:
            _check16(got[b], ref[b], f"seq {b} N={n}")


@pytest.mark.parametrize("case,splits", [("gaps", 40), ("gaps", 0), ("wide", 0), ("wide", 150), ("wide", 7)])
def test_batched_virtual_chunks(case, splits):
    # Chunks cut a batch's virtual length, in which every sequence start adds
    # the planner's piece cost. "gaps": short sequences among empty ones with
    # many requested splits, so that some chunks fall between sequences and
    # hold no tokens; "wide": more than 64 sequences (the sequence search
    # runs over cu_seqlens in passes of 64), ragged, with empty ones.
    if case == "gaps":
        seqlens = np.array([5, 0, 0, 0, 7, 3, 0, 40, 0, 1])
        assert all(any(lo >= hi for lo, hi in _chunk_bounds(seqlens, 40, c)) for c in PIECE_COSTS)
    else:
        rng = np.random.default_rng(77)
        seqlens = rng.integers(1, 600, size=150)
        seqlens[::9] = 0
        seqlens[70] = 3000
    print(f"virtual chunks {case} splits={splits}", flush=True)
    q, c, cu = synthetic.batched_inputs(32, seqlens, seed=13)
    got = _batched(q, c, cu, num_splits=splits)
    ref = O.closed_form_batched(q, c, cu)
    for b, n in enumerate(seqlens):
        if n == 0:
            assert not got[b].any(), f"empty seq {b}"
        else:
            _check16(got[b], ref[b], f"seq {b} N={n}")


def test_batched_equals_single_sequence_calls():
    seqlens = np.array([700, 129, 2048])
    q, c, cu = synthetic.batched_inputs(128, seqlens, seed=12)
    got = _batched(q, c, cu)
    for b in range(3):
        single = _fp16(q[b], c[cu[b]:cu[b + 1]])
        assert np.abs(got[b] - single).max() < 2e-3


# ------------------------------------------------- extension and runtime

def test_extension_matches_capi_and_dispatches_dtype():
    import ada_mla
    q, c = synthetic.decode_inputs(128, 1500, seed=13)
    qt, ct = _t(q), _t(c)
    a = ada_mla.mla_decode_split(qt, ct)
    b = capi.decode_split_fp16(qt, ct)
    torch.cuda.synchronize()
    assert a.dtype == torch.float16 and a.shape == (128, 512)
    assert torch.equal(a, b)
    f = ada_mla.mla_decode_fused(qt.float(), ct.float())
    torch.cuda.synchronize()
    assert f.dtype == torch.float32
    _check32(f.cpu().numpy(), O.closed_form(q, c), "fused fp32")
    # reference mla_decode_split on fp32 returned uninitialised memory; here it computes
    g = ada_mla.mla_decode_split(qt.float(), ct.float())
    assert torch.equal(g, f)


def test_extension_non_contiguous_inputs():
    import ada_mla
    q, c = synthetic.decode_inputs(32, 300, seed=14)
    qt = _t(np.ascontiguousarray(q.T)).t()  # a transposed view
    ct = _t(np.concatenate([c, c], axis=1))[:, :576]
    assert not qt.is_contiguous() and not ct.is_contiguous()
    got = ada_mla.mla_decode_split(qt, ct).float().cpu().numpy()
    _check16(got, O.closed_form(q, c), "non-contiguous")


def test_extension_batched():
    import ada_mla
    seqlens = np.array([100, 0, 3000])
    q, c, cu = synthetic.batched_inputs(128, seqlens, seed=15)
    got = ada_mla.mla_decode_split_batched(_t(q), _t(c), _t(cu)).float().cpu().numpy()
    ref = O.closed_form_batched(q, c, cu)
    _check16(got[0], ref[0])
    _check16(got[2], ref[2])
    assert not got[1].any()


def test_extension_gpu_argument_errors():
    import ada_mla
    q = torch.zeros(128, 576, dtype=torch.float16, device=_dev())
    with pytest.raises(RuntimeError, match="GPU tensors"):
        ada_mla.mla_decode_split(q, torch.zeros(10, 576, dtype=torch.float16))


def test_runs_on_current_nondefault_stream():
    import ada_mla
    q, c = synthetic.decode_inputs(128, 2000, seed=16)
    qt, ct = _t(q), _t(c)
    ref = ada_mla.mla_decode_split(qt, ct)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = ada_mla.mla_decode_split(qt, ct)
    s.synchronize()
    assert torch.equal(out, ref)


def test_repeat_determinism():
    q, c = synthetic.decode_inputs(128, 5000, seed=17)
    qt, ct = _t(q), _t(c)
    outs = [capi.decode_split_fp16(qt, ct) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    f = [capi.decode_fused_fp32(qt.float(), ct.float()) for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(f[0], f[1])


# ------------------------------------------- fp32 partials (MLA_FLAG_FP32_PARTIALS)

@pytest.mark.parametrize("n_h,n", [(16, 1), (16, 1000), (128, 33), (128, 4096), (48, 2500)])
def test_fp32_partials(n_h, n):
    print(f"fp32 partials n_h={n_h} N={n}", flush=True)
    q, c = synthetic.decode_inputs(n_h, n, seed=400 + n)
    got = _fp16(q, c, flags=capi.FLAG_FP32_PARTIALS)
    _check16(got, O.closed_form(q, c), f"n_h={n_h} N={n}")
    # the partial precision only moves the output by fp16-partial rounding
    assert np.abs(got - _fp16(q, c)).max() < 2e-3


def test_config3_n65536_fp32_partials():
    # BASELINE config 3 names fp32 partials
    q, c = synthetic.decode_inputs(128, 65536, seed=42)
    _check16(_fp16(q, c, flags=capi.FLAG_FP32_PARTIALS), O.closed_form(q, c), "config 3, fp32 partials")


# ------------------------------------------ quarter-tile combine (few items)
# With fewer (16 x 16 tile, sequence) items than CUs the combine merges
# quarter tiles (16 heads x 4 dims): lane (j, h) takes slots 4 i + j, so a slot
# count that is not a multiple of 4 leaves lanes without a slot, and more
# than 16 waves x 16 slots take a second load batch per wave.

@pytest.mark.parametrize("n_h,n,splits,flags", [
    (16, 32768, 600, 0), (16, 32768, 600, 4), (16, 5000, 3, 0), (16, 70, 2, 0),
    (32, 5000, 0, 0), (48, 1000, 77, 0), (64, 4096, 6, 4), (64, 20000, 0, 0)])
def test_quarter_combine(n_h, n, splits, flags):
    print(f"quarter combine n_h={n_h} N={n} splits={splits} flags={flags}", flush=True)
    q, c = synthetic.decode_inputs(n_h, n, seed=700 + n_h + splits)
    _check16(_fp16(q, c, num_splits=splits, flags=flags), O.closed_form(q, c),
             f"n_h={n_h} N={n} splits={splits} flags={flags}")


@pytest.mark.parametrize("n_h,n,flags", [(16, 65536, 0), (16, 65536 + 3, 4), (32, 65536, 0), (32, 131072 + 9, 4)])
def test_few_heads_long_sequences_planner_plans(n_h, n, flags):
    # the planner's own plans where few heads stream C: every CU busy (256
    # chunks at n_h = 16; 128 chunks of two 16-head tiles or 256 of one
    # 32-head tile at n_h = 32)
    lib = capi.load()
    splits = lib.mla_decode_split_num_splits(n_h, n, 0, flags)
    tile = lib.mla_decode_split_head_tile(n_h, n, 0, flags)
    print(f"few heads n_h={n_h} N={n} flags={flags}: {splits} splits, {tile}-head tiles", flush=True)
    assert splits * (n_h // tile) >= 128
    q, c = synthetic.decode_inputs(n_h, n, seed=900 + n_h)
    _check16(_fp16(q, c, flags=flags), O.closed_form(q, c), f"n_h={n_h} N={n} flags={flags}")


@pytest.mark.parametrize("n_h,n,splits", [(16, 3000, 0), (16, 3000, 300), (32, 777, 5)])
def test_quarter_combine_fp32(n_h, n, splits):
    print(f"quarter combine fp32 n_h={n_h} N={n} splits={splits}", flush=True)
    q, c = synthetic.decode_inputs(n_h, n, seed=800 + n, dtype=np.float32)
    _check32(_fp32(q, c, num_splits=splits), O.closed_form(q, c), f"n_h={n_h} N={n} splits={splits}")


@pytest.mark.parametrize("splits", [0, 3, 50, 400])
def test_quarter_combine_batched_ragged_with_empty(splits):
    print(f"quarter combine batched splits={splits}", flush=True)
    seqlens = np.array([5, 0, 17, 1000, 300, 64, 0])  # 7 x 32 tiles at 16 heads: 224 items
    q, c, cu = synthetic.batched_inputs(16, seqlens, seed=19)
    got = _batched(q, c, cu, num_splits=splits)
    ref = O.closed_form_batched(q, c, cu)
    for b in range(len(seqlens)):
        if seqlens[b] == 0:
            assert not got[b].any(), f"empty seq {b}"
        else:
            _check16(got[b], ref[b], f"seq {b} splits={splits}")


@pytest.mark.parametrize("flags", [0, 4])
def test_two_phase_api_equals_single_call(flags):
    # the two phases are the two-launch call's launches
    lib = capi.load()
    q, c = synthetic.decode_inputs(128, 3000, seed=21)
    qt, ct = _t(q), _t(c)
    one = capi.decode_split_fp16(qt, ct, flags=flags | capi.FLAG_TWO_LAUNCHES)
    out = torch.empty_like(one)
    ws_bytes = lib.mla_decode_split_workspace_size(128, 3000, 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=qt.device)
    s = capi._stream(qt)
    assert lib.mla_decode_split_fp16_partials(qt.data_ptr(), ct.data_ptr(), ws.data_ptr(), ws_bytes,
                                              128, 3000, 0, flags, s) == 0
    assert lib.mla_decode_split_fp16_combine(ws.data_ptr(), ws_bytes, out.data_ptr(), 128, 3000, 0, flags, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(one, out)


@pytest.mark.parametrize("splits", [0, 7])
def test_batched_two_phase_api_equals_single_call(splits):
    # mla_decode_split_batched_fp16_partials then _combine are the batched
    # call's two launches: bitwise equal output, empty sequences included
    lib = capi.load()
    seqlens = np.array([700, 0, 33, 4100, 1, 0, 2500])
    q, c, cu = synthetic.batched_inputs(128, seqlens, seed=12)
    qt, ct, cut = _t(q), _t(c), _t(cu)
    B, n_h, total = len(seqlens), 128, int(seqlens.sum())
    one = capi.decode_split_batched_fp16(qt, ct, cut, num_splits=splits)
    out = torch.full_like(one, float("nan"))
    ws_bytes = lib.mla_decode_split_batched_workspace_size(B, n_h, total, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=qt.device)
    s = capi._stream(qt)
    assert lib.mla_decode_split_batched_fp16_partials(qt.data_ptr(), ct.data_ptr(), cut.data_ptr(), ws.data_ptr(),
                                                      ws_bytes, B, n_h, total, splits, s) == 0
    assert lib.mla_decode_split_batched_fp16_combine(ws.data_ptr(), ws_bytes, cut.data_ptr(), out.data_ptr(), B,
                                                     n_h, total, splits, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(one, out)
    ref = O.closed_form_batched(q, c, cu)
    got = out.float().cpu().numpy()
    for b in range(B):
        np.testing.assert_allclose(got[b], ref[b], atol=1e-2, rtol=1e-2, err_msg=f"sequence {b}")
