"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
every function include/mla_mi355x.h declares, its argument validation
returns the documented codes without launching anything, workspace sizes
follow the split plan, and the torch extension rejects bad inputs. No
compute call is made here (no GPU)."""
import ctypes
import subprocess

import numpy as np
import pytest
import torch

from ada_mla import capi


def test_library_exports_every_declared_function():
    lib = capi.load()
    declared = capi.declared_functions()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(lib, name), name
    # and the dynamic symbol table agrees
    syms = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True,
                          text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in syms.splitlines() if ln.strip()}
    assert set(declared) <= exported


def test_abi_version_and_status_strings():
    lib = capi.load()
    assert lib.mla_abi_version() == 2
    assert lib.mla_status_string(0) == b"success"
    assert b"workspace" in lib.mla_status_string(3)
    assert lib.mla_status_string(99) == b"unknown status"


def test_workspace_size_one_split():
    lib = capi.load()
    # one split: 128 heads x 512 partial O + 2 x 128 fp32 (256-byte aligned); the
    # 16-bit path's size covers fp32 partials (MLA_FLAG_FP32_PARTIALS) too
    assert lib.mla_decode_split_workspace_size(128, 4096, 1) == 128 * 512 * 4 + 2 * 512
    assert lib.mla_decode_fused_workspace_size(16, 100, 1) == 16 * 512 * 4 + 2 * 256


def test_workspace_size_rejects_bad_sizes():
    lib = capi.load()
    assert lib.mla_decode_split_workspace_size(24, 4096, 0) == 0
    assert lib.mla_decode_split_workspace_size(0, 4096, 0) == 0
    assert lib.mla_decode_split_workspace_size(128, 0, 0) == 0
    assert lib.mla_decode_split_batched_workspace_size(0, 128, 100, 0) == 0
    assert lib.mla_decode_split_batched_workspace_size(4, 128, 0, 0) > 0  # all-empty batch is valid


def test_workspace_grows_with_splits_and_batch():
    lib = capi.load()
    a = lib.mla_decode_split_workspace_size(128, 65536, 8)
    b = lib.mla_decode_split_workspace_size(128, 65536, 64)
    assert b == 8 * (a - 2 * 4096) + 2 * 32768
    # batched: slots = splits + batch - 1
    s = lib.mla_decode_split_batched_workspace_size(32, 128, 270000, 64)
    assert s == (64 + 31) * 128 * 512 * 4 + 2 * ((64 + 31) * 128 * 4)


def test_split_count_is_clamped_to_blocks():
    lib = capi.load()
    # 40 tokens cannot be cut into more than 2 blocks of 32 (128 heads -> 32-head tiles)
    assert lib.mla_decode_split_workspace_size(128, 40, 1000) == lib.mla_decode_split_workspace_size(128, 40, 2)


FAKE = 0x10000  # never dereferenced: every call below returns before any launch, or (without a GPU) fails at it


@pytest.mark.parametrize("args,code", [
    ((None, FAKE, FAKE, FAKE, 1 << 30, 128, 64, 0, None), capi.STATUS_INVALID_VALUE),
    ((FAKE, FAKE, FAKE, FAKE, 1 << 30, 24, 64, 0, None), capi.STATUS_INVALID_VALUE),
    ((FAKE, FAKE, FAKE, FAKE, 1 << 30, 128, 0, 0, None), capi.STATUS_INVALID_VALUE),
    ((FAKE + 2, FAKE, FAKE, FAKE, 1 << 30, 128, 64, 0, None), capi.STATUS_MISALIGNED),
    ((FAKE, FAKE, FAKE, FAKE + 8, 1 << 30, 128, 64, 0, None), capi.STATUS_MISALIGNED),
    ((FAKE, FAKE, FAKE, FAKE, 16, 128, 64, 0, None), capi.STATUS_WORKSPACE_TOO_SMALL),
])
def test_split_fp16_argument_errors(args, code):
    assert capi.load().mla_decode_split_fp16(*args) == code
    # the bf16 entry takes the same arguments and validates them the same way
    assert capi.load().mla_decode_split_bf16(*args) == code


def test_noalloc_argument_errors():
    lib = capi.load()
    f = lib.mla_decode_split_fp16_noalloc
    assert f(FAKE, FAKE, FAKE, 24, 64, 0, None) == capi.STATUS_INVALID_VALUE
    assert f(FAKE, FAKE, FAKE, 128, 0, 0, None) == capi.STATUS_INVALID_VALUE
    # partials of 4096 heads x 256 splits (~1 GB) exceed the 32 MiB scratch: rejected
    # before the scratch is looked up or anything launched
    assert f(FAKE, FAKE, FAKE, 4096, 65536, 256, None) == capi.STATUS_SCRATCH_EXCEEDED
    assert b"scratch" in lib.mla_status_string(capi.STATUS_SCRATCH_EXCEEDED)
    # every plan the planner picks by itself for 128 heads fits (16 MiB + m, l at most)
    for n in (1, 4096, 65536, 1 << 20):
        splits = lib.mla_decode_split_num_splits(128, n, 0, 0)
        assert splits * 128 * 512 * 2 < capi.NOALLOC_SCRATCH_BYTES


def test_fused_fp32_rejects_head_dim():
    lib = capi.load()
    assert lib.mla_decode_fused_fp32(FAKE, FAKE, FAKE, FAKE, 1 << 30, 128, 512, 64, 0, None) == \
        capi.STATUS_INVALID_VALUE
    assert lib.mla_decode_fused_fp32(FAKE, FAKE, FAKE, FAKE, 16, 128, 576, 64, 0, None) == \
        capi.STATUS_WORKSPACE_TOO_SMALL


@pytest.mark.parametrize("fn", ["mla_decode_split_batched_fp16", "mla_decode_split_batched_bf16"])
def test_batched_argument_errors(fn):
    lib = capi.load()
    f = getattr(lib, fn)
    assert f(FAKE, FAKE, None, FAKE, FAKE, 1 << 30, 4, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 30, 0, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 16, 4, 128, 100, 0, None) == capi.STATUS_WORKSPACE_TOO_SMALL


def test_batched_two_phase_argument_errors():
    lib = capi.load()
    p, c = lib.mla_decode_split_batched_fp16_partials, lib.mla_decode_split_batched_fp16_combine
    # no cu_seqlens, no workspace, batch 0, a head count that is not a multiple of 16
    assert p(FAKE, FAKE, None, FAKE, 1 << 30, 4, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert p(FAKE, FAKE, FAKE, None, 1 << 30, 4, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert p(FAKE, FAKE, FAKE, FAKE, 1 << 30, 0, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert p(FAKE, FAKE, FAKE, FAKE, 1 << 30, 4, 24, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert p(FAKE, FAKE, FAKE, FAKE, 16, 4, 128, 100, 0, None) == capi.STATUS_WORKSPACE_TOO_SMALL
    assert c(FAKE, 1 << 30, None, FAKE, 4, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert c(FAKE, 1 << 30, FAKE, None, 4, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert c(FAKE, 16, FAKE, FAKE, 4, 128, 100, 0, None) == capi.STATUS_WORKSPACE_TOO_SMALL


# --------------------------------------------------------- torch extension

def _ext():
    import ada_mla
    return ada_mla


def test_extension_surface():
    m = _ext()
    assert m.HEAD_DIM_K == 576 and m.HEAD_DIM_C == 512 and m.HEAD_DIM_ROPE == 64
    for fn in ("mla_decode_split", "mla_decode_fused", "mla_decode_split_batched"):
        assert callable(getattr(m, fn))


@pytest.mark.parametrize("q,c,msg", [
    (torch.zeros(128, 576, dtype=torch.float16), torch.zeros(64, 576, dtype=torch.float32), "same dtype"),
    (torch.zeros(128, 576, dtype=torch.float64), torch.zeros(64, 576, dtype=torch.float64),
     "float16, bfloat16 or float32"),
    (torch.zeros(128, 576, dtype=torch.float16), torch.zeros(64, 577, dtype=torch.float16), "cache must be"),
    (torch.zeros(128, 576, dtype=torch.float16), torch.zeros(0, 576, dtype=torch.float16), "at least one token"),
    (torch.zeros(128, 512, dtype=torch.float16), torch.zeros(64, 576, dtype=torch.float16), "query must be"),
    (torch.zeros(24, 576, dtype=torch.float16), torch.zeros(64, 576, dtype=torch.float16), "multiple of 16"),
    (torch.zeros(128, 576, dtype=torch.float16), torch.zeros(64, 576, dtype=torch.float16), "GPU tensors"),
])
def test_extension_rejects_bad_inputs(q, c, msg):
    m = _ext()
    for fn in (m.mla_decode_split, m.mla_decode_fused):
        with pytest.raises(RuntimeError, match=msg):
            fn(q, c)


def test_batched_extension_rejects_bad_inputs():
    m = _ext()
    q = torch.zeros(2, 128, 576, dtype=torch.float16)
    c = torch.zeros(10, 576, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="batch \\+ 1"):
        m.mla_decode_split_batched(q, c, torch.zeros(2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="int32"):
        m.mla_decode_split_batched(q, c, torch.zeros(3, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="GPU tensors"):
        m.mla_decode_split_batched(q, c, torch.zeros(3, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="both bfloat16"):
        m.mla_decode_split_batched(q.bfloat16(), c, torch.zeros(3, dtype=torch.int32))


def test_fp8_extension_rejects_bad_inputs():
    m = _ext()
    q = torch.zeros(128, 576, dtype=torch.float16)
    c8 = torch.zeros(64, 576, dtype=torch.float8_e4m3fn)
    # fp8 caches pair with a float16 query only
    with pytest.raises(RuntimeError, match="same dtype"):
        m.mla_decode_split(q.bfloat16(), c8)
    with pytest.raises(RuntimeError, match="cache_scale"):
        m.mla_decode_split(q, c8, cache_scale=0.0)
    with pytest.raises(RuntimeError, match="cache_scale"):
        m.mla_decode_split(q, c8, cache_scale=float("inf"))
    with pytest.raises(RuntimeError, match="go through mla_decode_split"):
        m.mla_decode_fused(q, c8)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        m.mla_decode_split(q, c8, cache_scale=0.5)
    qb = torch.zeros(2, 128, 576, dtype=torch.float16)
    cu = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="cache_scale"):
        m.mla_decode_split_batched(qb, c8, cu, cache_scale=-1.0)
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        m.mla_decode_split_batched(qb.bfloat16(), c8, cu)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        m.mla_decode_split_batched(qb, c8, cu, cache_scale=0.5)


@pytest.mark.parametrize("fn", ["mla_decode_paged_fp16", "mla_decode_paged_bf16"])
def test_paged_argument_errors(fn):
    lib = capi.load()
    f = getattr(lib, fn)
    ok = dict(q=FAKE, kv=FAKE, bt=FAKE, cu=FAKE, out=FAKE, ws=FAKE, wsb=1 << 30, batch=4, nh=128, total=100,
              page=64, pages=10, stride=4, splits=0)

    def call(**kw):
        a = {**ok, **kw}
        return f(a["q"], a["kv"], a["bt"], a["cu"], a["out"], a["ws"], a["wsb"], a["batch"], a["nh"], a["total"],
                 a["page"], a["pages"], a["stride"], a["splits"], None)
    for bad in (dict(bt=None), dict(cu=None), dict(page=16), dict(page=96), dict(page=0), dict(pages=0),
                dict(stride=0), dict(nh=24), dict(batch=0), dict(total=-1)):
        assert call(**bad) == capi.STATUS_INVALID_VALUE, bad
    assert call(kv=FAKE + 4) == capi.STATUS_MISALIGNED
    assert call(wsb=16) == capi.STATUS_WORKSPACE_TOO_SMALL


def test_paged_workspace_size():
    lib = capi.load()
    assert lib.mla_decode_paged_workspace_size(0, 128, 100, 0) == 0
    assert lib.mla_decode_paged_workspace_size(4, 24, 100, 0) == 0
    # one split: fp16 partial O for (1 chunk + 3 extra sequences) slots
    assert lib.mla_decode_paged_workspace_size(4, 128, 100, 1) == 4 * 128 * 512 * 2 + 2 * 4 * 128 * 4


def test_paged_extension_rejects_bad_inputs():
    m = _ext()
    q = torch.zeros(2, 128, 576, dtype=torch.float16)
    kv = torch.zeros(4, 64, 576, dtype=torch.float16)
    bt = torch.zeros(2, 3, dtype=torch.int32)
    cu = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="power of two"):
        m.mla_decode_paged(q, torch.zeros(4, 48, 576, dtype=torch.float16), bt, cu)
    with pytest.raises(RuntimeError, match="block_table must be"):
        m.mla_decode_paged(q, kv, bt.long(), cu)
    with pytest.raises(RuntimeError, match="batch rows"):
        m.mla_decode_paged(q, kv, bt[:1], cu)
    with pytest.raises(RuntimeError, match="kv_cache must both be float16 or both bfloat16"):
        m.mla_decode_paged(q, kv.bfloat16(), bt, cu)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        m.mla_decode_paged(q, kv, bt, cu)


def test_plan_cache_returns_the_same_plans():
    # plans are cached per host thread (16 entries): more distinct argument
    # sets than entries, asked twice in different orders, give the same answers
    lib = capi.load()
    args = [(nh, n, s) for nh in (16, 32, 128) for n in (1, 100, 4096, 65536) for s in (0, 3, 64)]
    first = {a: (lib.mla_decode_split_num_splits(*a, 0), lib.mla_decode_split_workspace_size(*a)) for a in args}
    for a in reversed(args):
        assert (lib.mla_decode_split_num_splits(*a, 0), lib.mla_decode_split_workspace_size(*a)) == first[a], a
    # the flag is part of the key
    assert lib.mla_decode_split_num_splits(128, 65536, 0, 0) != lib.mla_decode_split_num_splits(128, 65536, 0, 4)


def test_single_launch_choice():
    # a whole single-sequence call whose plan has one split is one launch;
    # the flags that select the two-launch path are honoured
    lib = capi.load()
    f = lib.mla_decode_split_launches
    for n_h, n in [(128, 1), (128, 32), (128, 128), (16, 100), (64, 200)]:
        assert lib.mla_decode_split_num_splits(n_h, n, 0, 0) == 1, (n_h, n)
        assert f(n_h, n, 0, 0) == 1, (n_h, n)
        assert f(n_h, n, 0, capi.FLAG_TWO_LAUNCHES) == 2
        assert f(n_h, n, 0, capi.FLAG_SCALAR_TRANSPOSE) == 2
    for n_h, n in [(128, 4096), (16, 32768), (128, 65536)]:
        assert f(n_h, n, 0, 0) == 2
    assert f(128, 4096, 1, 0) == 1  # a requested single split
    assert f(24, 100, 0, 0) == 0 and f(128, 0, 0, 0) == 0


def test_head_tile_query():
    # the plan's heads per workgroup: 64 at long N, 16 at N = 4096 (eight
    # tiles fill the CUs), 32 when a requested split count leaves room; 0 for
    # invalid sizes
    lib = capi.load()
    f = lib.mla_decode_split_head_tile
    assert f(128, 65536, 0, 0) == 64
    assert f(128, 4096, 0, 0) == 16
    assert f(32, 20000, 200, 0) == 32
    assert f(16, 32768, 0, 0) == 16
    assert f(24, 100, 0, 0) == 0 and f(128, 0, 0, 0) == 0


def test_few_head_long_sequences_stream_with_at_least_half_the_cus():
    # With few heads C streams from HBM at the chip's rate only when enough
    # chunks are in flight: the planner charges each block the HBM time of
    # every chunk streaming at once, so at long N it keeps at least 128 of
    # the 256 CUs busy (a floor over the whole call once chose 108-114
    # chunks there, 12-18% slower on MI355X; once its blocks wait on HBM a plan
    # takes every CU), and at N = 16384 stays at 128 chunks, where more splits
    # cost more in partials than they save.
    lib = capi.load()
    splits, tile = lib.mla_decode_split_num_splits, lib.mla_decode_split_head_tile
    for n_h in (16, 32):
        for n in (65536, 131072, 262144):
            for flags in (0, capi.FLAG_FP32_PARTIALS):
                workgroups = splits(n_h, n, 0, flags) * (n_h // tile(n_h, n, 0, flags))
                assert 128 <= workgroups <= 256, (n_h, n, flags, workgroups)
    assert splits(16, 16384, 0, 0) == 128


def test_fp8_cache_plan_query():
    # MLA_FLAG_FP8_CACHE asks the plan queries for the fp8-cache entries'
    # plan: their cache streams half the bytes, so with few heads more chunks
    # pay before C binds the block time (n_h = 16, N = 32768: 256 chunks, 5%
    # faster on MI355X than the 16-bit plan's 128); with 128 heads the two
    # plans are the same
    lib = capi.load()
    splits, tile = lib.mla_decode_split_num_splits, lib.mla_decode_split_head_tile
    f8 = capi.FLAG_FP8_CACHE
    assert splits(16, 32768, 0, f8) == 256 and splits(16, 32768, 0, 0) == 128
    for n in (4096, 65536):
        assert (splits(128, n, 0, f8), tile(128, n, 0, f8)) == (splits(128, n, 0, 0), tile(128, n, 0, 0))
    # the fp8 entries keep fp16 partials: the fp32-partials flag does not change their plan
    assert splits(128, 65536, 0, f8 | capi.FLAG_FP32_PARTIALS) == splits(128, 65536, 0, f8)


def test_block_projection_argument_errors():
    lib = capi.load()
    for fn in ("mla_absorb_query_fp16", "mla_absorb_query_bf16"):
        f = getattr(lib, fn)
        assert f(None, FAKE, FAKE, FAKE, 1, 16, None) == capi.STATUS_INVALID_VALUE
        assert f(FAKE, FAKE, FAKE, FAKE, 0, 16, None) == capi.STATUS_INVALID_VALUE
        assert f(FAKE, FAKE + 2, FAKE, FAKE, 1, 16, None) == capi.STATUS_MISALIGNED
    for fn in ("mla_project_output_fp16", "mla_project_output_bf16"):
        f = getattr(lib, fn)
        assert f(FAKE, FAKE, None, FAKE, FAKE, 1 << 20, 1, 16, 64, None) == capi.STATUS_INVALID_VALUE
        assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, 1, 16, 0, None) == capi.STATUS_INVALID_VALUE
        assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 16, 1, 16, 64, None) == capi.STATUS_WORKSPACE_TOO_SMALL
    # per-head values of B x n_h x 128 in the input dtype, 256-byte aligned
    def a256(n):
        return (n + 255) // 256 * 256
    # the values, then two fp32 tiles of 32 x 64 per workgroup of the W_O kernel: 16 column blocks x
    # 8 K-chunks = 128 steps, one per workgroup
    assert lib.mla_project_output_workspace_size(3, 16, 1000) == a256(3 * 16 * 128 * 2) + 2 * 128 * 32 * 64 * 4
    # at most 512 workgroups: 80 x 64 = 5120 steps
    assert lib.mla_project_output_workspace_size(32, 128, 5120) == 32 * 128 * 128 * 2 + 2 * 512 * 32 * 64 * 4
    assert lib.mla_project_output_workspace_size(0, 16, 1000) == 0
    assert lib.mla_project_output_workspace_size(3, 16, 0) == 0


def test_block_extension_rejects_bad_inputs():
    m = _ext()
    h = torch.float16
    with pytest.raises(RuntimeError, match="q_rope must be"):
        m.mla_absorb_query(torch.zeros(2, 16, 128, dtype=h), torch.zeros(2, 16, 32, dtype=h),
                           torch.zeros(16, 128, 512, dtype=h))
    with pytest.raises(RuntimeError, match="w_uk must be"):
        m.mla_absorb_query(torch.zeros(2, 16, 128, dtype=h), torch.zeros(2, 16, 64, dtype=h),
                           torch.zeros(16, 512, 128, dtype=h))
    with pytest.raises(RuntimeError, match="w_o must be"):
        m.mla_project_output(torch.zeros(2, 16, 512, dtype=h), torch.zeros(16, 128, 512, dtype=h),
                             torch.zeros(64, 100, dtype=h))
    with pytest.raises(RuntimeError, match="GPU tensor"):
        m.mla_project_output(torch.zeros(2, 16, 512, dtype=h), torch.zeros(16, 128, 512, dtype=h),
                             torch.zeros(64, 16 * 128, dtype=h))


def test_fp8_argument_errors():
    lib = capi.load()
    f = lib.mla_decode_split_fp8
    for bad_scale in (0.0, -1.0, float("inf"), float("nan")):
        assert f(FAKE, FAKE, bad_scale, FAKE, FAKE, 1 << 30, 128, 64, 0, None) == capi.STATUS_INVALID_VALUE
    assert f(FAKE, FAKE, 1.0, FAKE, FAKE, 1 << 30, 24, 64, 0, None) == capi.STATUS_INVALID_VALUE
    assert f(FAKE, FAKE + 8, 1.0, FAKE, FAKE, 1 << 30, 128, 64, 0, None) == capi.STATUS_MISALIGNED
    assert f(FAKE, FAKE, 1.0, FAKE, FAKE, 16, 128, 64, 0, None) == capi.STATUS_WORKSPACE_TOO_SMALL
    g = lib.mla_decode_split_batched_fp8
    assert g(FAKE, FAKE, 1.0, None, FAKE, FAKE, 1 << 30, 4, 128, 100, 0, None) == capi.STATUS_INVALID_VALUE
    assert lib.mla_decode_split_fp8_workspace_size(0, 128, 10, 0) == 0
    assert lib.mla_decode_split_fp8_workspace_size(1, 128, 10, 0) > 0


@pytest.mark.parametrize("fn", ["mla_decode_split_batched_fp16", "mla_decode_split_batched_bf16",
                                "mla_decode_split_batched_fp8"])
@pytest.mark.parametrize("splits", [0, 1])
def test_batched_single_sequence_reaches_the_launch(fn, splits):
    # A batch of one sequence with a one-split plan once took the one-launch
    # path, which rejects cu_seqlens before launching (hipErrorInvalidValue).
    # Here, with no GPU, the call must get as far as the launch itself, which
    # then fails for want of a device. With a GPU present the launch would run
    # on the never-dereferenced FAKE pointers, so the test only runs without
    # one (the GPU parity of this case is test_gpu_parity.py's
    # test_batched_single_sequence).
    if torch.cuda.device_count() > 0:
        pytest.skip("launch-reaching CPU check: needs a machine without a GPU")
    lib = capi.load()
    f = getattr(lib, fn)
    args = (FAKE, FAKE) + ((1.0,) if fn.endswith("fp8") else ()) + (FAKE, FAKE, FAKE, 1 << 30, 1, 128, 100, splits, None)
    assert f(*args) == capi.STATUS_HIP_ERROR
    assert lib.mla_last_hip_error() != 1  # not hipErrorInvalidValue from the plan/launch mismatch


@pytest.mark.parametrize("n", [1, 100, 1000, 4097, 65536])
def test_fp8_workspace_size_covers_the_single_sequence_entry(n):
    # mla_decode_split_fp8_workspace_size serves both fp8 entries; with batch 1
    # it must also cover the single-sequence entry's plan, which (no
    # cu_seqlens) may cut the sequence differently from a batch of one.
    # Without a GPU a call with enough workspace fails only at the launch.
    if torch.cuda.device_count() > 0:
        pytest.skip("launch-reaching CPU check: needs a machine without a GPU")
    lib = capi.load()
    ws = lib.mla_decode_split_fp8_workspace_size(1, 128, n, 0)
    for flagless_splits in (0, 3):
        ws_s = lib.mla_decode_split_fp8_workspace_size(1, 128, n, flagless_splits)
        st = lib.mla_decode_split_fp8(FAKE, FAKE, 1.0, FAKE, FAKE, ws_s, 128, n, flagless_splits, None)
        assert st == capi.STATUS_HIP_ERROR, (n, flagless_splits, st)
        st = lib.mla_decode_split_batched_fp8(FAKE, FAKE, 1.0, FAKE, FAKE, FAKE, ws_s, 1, 128, n, flagless_splits,
                                              None)
        assert st == capi.STATUS_HIP_ERROR, (n, flagless_splits, st)
    assert ws > 0
