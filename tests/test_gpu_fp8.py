"""GPU parity of the fp8 KV-cache path (mla_decode_split_fp8 and
mla_decode_split_batched_fp8): the cache is stored as OCP fp8 E4M3FN holding
C / scale, the query and output are fp16. The oracle is the float64 closed
form on the dequantised cache (fp8 value x scale) and the fp16 query; there is
no reference fp8 path (README.md:408 lists it as future work).

Tolerance as for fp16: atol = rtol = 1e-2 and mean relative error < 5e-3 --
the dequantisation itself is exact (every E4M3 value is an fp16 value), so
only the kernel's own rounding remains: fp16 P, fp16 partials and output,
and, with 32- or 64-head tiles, Q* held as two fp8 parts (about 8
significant bits, each head scaled by a power of two) for the first product.
"""
import numpy as np
import pytest
import torch

from ada_mla import capi, synthetic
from oracle import mla_oracle as O

pytestmark = pytest.mark.gpu


def _fp8_inputs(n_h, n, seed, scale):
    q = synthetic.normal((n_h, 576), seed, np.float16)
    c32 = synthetic.normal((n, 576), seed + 1, np.float32)
    c8 = torch.from_numpy(c32 / np.float32(scale)).to(torch.float8_e4m3fn)
    c_deq = c8.float().double().numpy() * scale
    return q, c8, c_deq


def _check(got, ref, what, scale=1.0):
    # scale: the cache's dequantisation scale when the data are not of
    # order one (the absolute tolerance is for unit-scale values)
    assert np.isfinite(got).all(), what
    np.testing.assert_allclose(got, ref, atol=1e-2 * scale, rtol=1e-2, err_msg=what)
    rel = np.abs(got - ref).mean() / max(np.abs(ref).mean(), 1e-30)
    assert rel < 5e-3, f"{what}: mean relative error {rel:.3e}"


@pytest.mark.parametrize("n_h", [16, 32, 128])
@pytest.mark.parametrize("n", [1, 17, 33, 100, 1000, 4097])
def test_fp8_shapes(n_h, n):
    print(f"fp8 n_h={n_h} N={n}", flush=True)
    q, c8, cd = _fp8_inputs(n_h, n, seed=500 + n, scale=0.25)
    out = capi.decode_split_fp8(torch.from_numpy(q).cuda(), c8.cuda(), 0.25)
    torch.cuda.synchronize()
    _check(out.double().cpu().numpy(), O.closed_form(q, cd), f"n_h={n_h} N={n}")


@pytest.mark.parametrize("n_h,n,scale", [(128, 4096, 1.0), (128, 65536, 0.03125), (16, 32768, 3.0)])
def test_fp8_benchmark_shapes(n_h, n, scale):
    print(f"fp8 config n_h={n_h} N={n} scale={scale}", flush=True)
    q, c8, cd = _fp8_inputs(n_h, n, seed=42, scale=scale)
    out = capi.decode_split_fp8(torch.from_numpy(q).cuda(), c8.cuda(), scale)
    torch.cuda.synchronize()
    _check(out.double().cpu().numpy(), O.closed_form(q, cd), f"n_h={n_h} N={n}")


def test_fp8_split_invariance_and_single_token():
    q, c8, cd = _fp8_inputs(32, 3000, seed=3, scale=0.5)
    ref = O.closed_form(q, cd)
    for s in (1, 3, 40):
        out = capi.decode_split_fp8(torch.from_numpy(q).cuda(), c8.cuda(), 0.5, num_splits=s)
        torch.cuda.synchronize()
        _check(out.double().cpu().numpy(), ref, f"splits={s}")
    q1, c1, cd1 = _fp8_inputs(16, 1, seed=4, scale=2.0)
    out = capi.decode_split_fp8(torch.from_numpy(q1).cuda(), c1.cuda(), 2.0)
    torch.cuda.synchronize()
    # one token: the output is that token's dequantised C_N row, rounded to fp16
    want = np.repeat(cd1[:, :512], 16, axis=0).astype(np.float16).astype(np.float64)
    assert np.array_equal(out.double().cpu().numpy(), want)


@pytest.mark.parametrize("n_h", [32, 128])
@pytest.mark.parametrize("q_scale,c_scale", [(2.0 ** 4, 2.0 ** -4), (2.0 ** -8, 2.0 ** 8), (2.0 ** 10, 2.0 ** -6)])
def test_fp8_query_dynamic_range(n_h, q_scale, c_scale):
    # With 32- or 64-head tiles the first product runs on fp8 MFMAs, with
    # each head's Q* row scaled by a power of two and split into two fp8
    # operands. Rows of different magnitudes (per-head factors 2^-2 .. 2^2,
    # times q_scale, offset by the cache scale so that the logits stay of
    # order one), entries far outside fp8's range either way, and an
    # all-zero row (uniform weights) must all come out right. The plans are
    # a 64-head tile (128 heads, N = 65536) and a 32-head tile (32 heads,
    # 200 splits of N = 20000).
    n, splits = (65536, 0) if n_h == 128 else (20000, 200)
    assert capi.load().mla_decode_split_head_tile(n_h, n, splits, capi.FLAG_FP8_CACHE) == (64 if n_h == 128 else 32)
    print(f"fp8 dynamic range n_h={n_h} q_scale={q_scale}", flush=True)
    q = synthetic.normal((n_h, 576), 77, np.float32)
    q = q * (2.0 ** np.linspace(-2.0, 2.0, n_h))[:, None] * q_scale
    q[3] = 0.0
    q16 = q.astype(np.float16)
    c8 = torch.from_numpy(synthetic.normal((n, 576), 78, np.float32)).to(torch.float8_e4m3fn)
    cd = c8.float().double().numpy() * c_scale
    out = capi.decode_split_fp8(torch.from_numpy(q16).cuda(), c8.cuda(), c_scale, num_splits=splits)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    ref = O.closed_form(q16, cd)
    _check(got, ref, f"n_h={n_h} q_scale={q_scale}", scale=max(1.0, c_scale))
    # the zero row: every token weighs the same
    np.testing.assert_allclose(got[3], cd[:, :512].mean(axis=0), atol=1e-3 * c_scale, rtol=1e-2)


@pytest.mark.parametrize("n_h", [128, 32])
def test_fp8_query_near_fp16_max(n_h):
    # Heads whose largest |q| lies in [2^15, 65504]: rounded to the split's 4
    # significant bits such an entry can become 65536, beyond fp16, so these
    # heads form the second fp8 part at half scale. Rows scaled to maxima of
    # 65504, 64000, 63488, 40000 and 32768 (and, for contrast, 30000), with a
    # cache scale that keeps the logits of order one.
    n, splits = (65536, 0) if n_h == 128 else (20000, 200)
    assert capi.load().mla_decode_split_head_tile(n_h, n, splits, capi.FLAG_FP8_CACHE) == (64 if n_h == 128 else 32)
    print(f"fp8 query near fp16 max n_h={n_h}", flush=True)
    q = synthetic.normal((n_h, 576), 91, np.float32)
    tops = np.array([65504.0, 64000.0, 63488.0, 40000.0, 32768.0, 30000.0])
    amax = tops[np.arange(n_h) % len(tops)]
    q = q / np.abs(q).max(axis=1, keepdims=True) * amax[:, None]
    q16 = q.astype(np.float16)
    assert np.isfinite(q16).all() and np.abs(q16).max() == 65504.0
    c_scale = 2.0 ** -13
    c8 = torch.from_numpy(synthetic.normal((n, 576), 92, np.float32)).to(torch.float8_e4m3fn)
    cd = c8.float().double().numpy() * c_scale
    out = capi.decode_split_fp8(torch.from_numpy(q16).cuda(), c8.cuda(), c_scale, num_splits=splits)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    _check(got, O.closed_form(q16, cd), f"n_h={n_h} near fp16 max", scale=c_scale)


def test_fp8_batched_with_empty():
    seqlens = np.array([5, 0, 17, 1, 300, 64, 0, 1000, 33])
    q, _, cu = synthetic.batched_inputs(128, seqlens, seed=9)
    c32 = synthetic.normal((int(cu[-1]), 576), 10, np.float32)
    c8 = torch.from_numpy(c32 / np.float32(0.5)).to(torch.float8_e4m3fn)
    cd = c8.float().double().numpy() * 0.5
    out = capi.decode_split_batched_fp8(torch.from_numpy(q).cuda(), c8.cuda(), 0.5, torch.from_numpy(cu).cuda(),
                                        num_splits=7)
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    ref = O.closed_form_batched(q, cd, cu)
    for b in range(len(seqlens)):
        if seqlens[b] == 0:
            assert not got[b].any()
        else:
            _check(got[b], ref[b], f"seq {b}")


@pytest.mark.parametrize("n_h,n,tile", [(16, 65536 + 5, 16), (32, 131072, 32)])
def test_fp8_few_heads_long_sequences(n_h, n, tile):
    # the fp8 plans of their own: with few heads about every CU takes a chunk
    # (228 chunks of 16 heads at N = 65541, where a chunk rounds up to 9
    # blocks; 256 of one 32-head tile, whose first product runs on fp8 MFMAs)
    lib = capi.load()
    assert lib.mla_decode_split_num_splits(n_h, n, 0, capi.FLAG_FP8_CACHE) > 200
    assert lib.mla_decode_split_head_tile(n_h, n, 0, capi.FLAG_FP8_CACHE) == tile
    print(f"fp8 few heads n_h={n_h} N={n}", flush=True)
    q, c8, cd = _fp8_inputs(n_h, n, seed=60 + n_h, scale=0.5)
    out = capi.decode_split_fp8(torch.from_numpy(q).cuda(), c8.cuda(), 0.5)
    torch.cuda.synchronize()
    _check(out.double().cpu().numpy(), O.closed_form(q, cd), f"n_h={n_h} N={n}")


@pytest.mark.parametrize("n_h,n,tile", [(96, 20000, 32), (192, 40000, 64), (64, 30000, 32)])
def test_fp8_several_head_tiles(n_h, n, tile):
    # fp8 first product on three head tiles of 32 or 64 heads per chunk
    # (the Q* split of each tile in its own workgroups)
    assert capi.load().mla_decode_split_head_tile(n_h, n, 0, capi.FLAG_FP8_CACHE) == tile
    print(f"fp8 n_h={n_h} N={n} head tile {tile}", flush=True)
    q, c8, cd = _fp8_inputs(n_h, n, seed=90 + n_h, scale=0.5)
    out = capi.decode_split_fp8(torch.from_numpy(q).cuda(), c8.cuda(), 0.5)
    torch.cuda.synchronize()
    _check(out.double().cpu().numpy(), O.closed_form(q, cd), f"n_h={n_h} N={n}")


def test_fp8_config5_batched():
    # BASELINE config 5's shape with an fp8 cache: 64-head tiles whose chunks
    # hold pieces of up to three sequences, each piece splitting its own Q*
    # into fp8 parts after the piece-start barrier
    print("fp8 config 5", flush=True)
    seqlens = synthetic.batched_seqlens(32, seed=42)
    q, _, cu = synthetic.batched_inputs(128, seqlens, seed=42)
    c8 = torch.from_numpy(synthetic.normal((int(cu[-1]), 576), 43, np.float32)).to(torch.float8_e4m3fn)
    cd = c8.float().double().numpy()
    out = capi.decode_split_batched_fp8(torch.from_numpy(q).cuda(), c8.cuda(), 1.0, torch.from_numpy(cu).cuda())
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    for b in range(32):
        lo, hi = cu[b], cu[b + 1]
        _check(got[b], O.closed_form(q[b], cd[lo:hi]), f"config 5 seq {b} N={hi - lo}")


def test_fp8_batched_many_items_with_empty():
    # 24 sequences x 128 heads: the combine merges several tiles per wave
    seqlens = np.random.default_rng(6).integers(2, 600, size=24)
    seqlens[1::6] = 0
    q, _, cu = synthetic.batched_inputs(128, seqlens, seed=11)
    c32 = synthetic.normal((int(cu[-1]), 576), 12, np.float32)
    c8 = torch.from_numpy(c32 / np.float32(1.5)).to(torch.float8_e4m3fn)
    cd = c8.float().double().numpy() * 1.5
    out = capi.decode_split_batched_fp8(torch.from_numpy(q).cuda(), c8.cuda(), 1.5, torch.from_numpy(cu).cuda())
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    ref = O.closed_form_batched(q, cd, cu)
    for b in range(len(seqlens)):
        if seqlens[b] == 0:
            assert not got[b].any()
        else:
            _check(got[b], ref[b], f"seq {b}")


def test_fp8_extension_equals_c_abi():
    # ada_mla.mla_decode_split / _batched with a float8_e4m3fn cache run the
    # same kernels as the C ABI entries: results are bitwise equal
    import ada_mla
    q, c8, cd = _fp8_inputs(128, 2500, seed=21, scale=0.125)
    qt, ct = torch.from_numpy(q).cuda(), c8.cuda()
    a = ada_mla.mla_decode_split(qt, ct, cache_scale=0.125)
    b = capi.decode_split_fp8(qt, ct, 0.125)
    torch.cuda.synchronize()
    assert a.dtype == torch.float16 and torch.equal(a, b)
    _check(a.double().cpu().numpy(), O.closed_form(q, cd), "extension")
    seqlens = np.array([40, 0, 2000])
    qb, _, cu = synthetic.batched_inputs(16, seqlens, seed=22)
    cb = torch.from_numpy(synthetic.normal((int(cu[-1]), 576), 23, np.float32)).to(torch.float8_e4m3fn).cuda()
    qbt, cut = torch.from_numpy(qb).cuda(), torch.from_numpy(cu).cuda()
    a = ada_mla.mla_decode_split_batched(qbt, cb, cut, num_splits=5, cache_scale=2.0)
    b = capi.decode_split_batched_fp8(qbt, cb, 2.0, cut, num_splits=5)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
