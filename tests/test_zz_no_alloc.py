"""The allocation-free entry point mla_decode_split_fp16_noalloc, through the C
ABI: the split partials live in the library's per-GPU scratch array instead
of a caller workspace. It launches the same kernels with the same plan as
mla_decode_split_fp16, so its output must equal that entry point's bitwise,
on consecutive calls (the second smaller than the first, so it runs on what
the first left in the scratch), and it must reject plans whose partials do
not fit the scratch.
"""
import ctypes

import numpy as np
import pytest
import torch

from ada_mla import capi, synthetic

pytestmark = pytest.mark.gpu


def _noalloc(q, c, num_splits=0, out=None):
    lib = capi.load()
    n_h, n = q.shape[0], c.shape[0]
    if out is None:
        out = torch.empty((n_h, capi.HEAD_DIM_V), dtype=torch.float16, device=q.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
    st = lib.mla_decode_split_fp16_noalloc(q.data_ptr(), c.data_ptr(), out.data_ptr(), n_h, n, num_splits, stream)
    return st, out


@pytest.mark.parametrize("first,second", [((128, 4096), (128, 1000)), ((128, 65536), (16, 33)),
                                          ((64, 20000), (32, 4097))])
def test_noalloc_matches_workspace_entry_on_consecutive_calls(first, second):
    dev = torch.device("cuda:0")
    for seed, (n_h, n) in enumerate((first, second)):
        print(f"noalloc case n_h={n_h} N={n}", flush=True)
        q, c = synthetic.decode_inputs(n_h, n, seed=11 + seed)
        qd, cd = torch.from_numpy(q).to(dev), torch.from_numpy(c).to(dev)
        st, got = _noalloc(qd, cd)
        assert st == capi.STATUS_SUCCESS, capi.load().mla_status_string(st)
        ref = capi.decode_split_fp16(qd, cd)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"n_h={n_h} N={n}: max diff {(got.float() - ref.float()).abs().max()}"


def test_noalloc_requested_splits():
    dev = torch.device("cuda:0")
    q, c = synthetic.decode_inputs(128, 3000, seed=5)
    qd, cd = torch.from_numpy(q).to(dev), torch.from_numpy(c).to(dev)
    st, got = _noalloc(qd, cd, num_splits=7)
    assert st == capi.STATUS_SUCCESS
    ref = capi.decode_split_fp16(qd, cd, num_splits=7)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    # The rejection of plans whose partials exceed the scratch is a host-side check,
    # tested on the CPU with pointers that are never dereferenced
    # (tests/test_boundary_cpu.py): no call here claims sizes its buffers do not have.
