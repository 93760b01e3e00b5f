"""ctypes binding of the C ABI in include/mla_mi355x.h (libmla_mi355x.so).

This is the binding a Python caller without the torch extension would add;
the parity tests call the kernels through it. torch is used only for device
memory and the current stream: tensors are passed as raw device pointers.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmla_mi355x.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "mla_mi355x.h")

HEAD_DIM_K = 576
HEAD_DIM_V = 512
STATUS_SUCCESS = 0
STATUS_INVALID_VALUE = 1
STATUS_MISALIGNED = 2
STATUS_WORKSPACE_TOO_SMALL = 3
STATUS_HIP_ERROR = 4
STATUS_SCRATCH_EXCEEDED = 5
NOALLOC_SCRATCH_BYTES = 32 << 20
FLAG_SCALAR_TRANSPOSE = 1
FLAG_FP32_PARTIALS = 4
FLAG_FP8_CACHE = 16  # plan queries: the fp8-cache entries' plan
FLAG_TWO_LAUNCHES = 8

_vp, _i, _u, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint, ctypes.c_size_t
_SIGNATURES = {
    "mla_abi_version": (_i, []),
    "mla_status_string": (ctypes.c_char_p, [_i]),
    "mla_last_hip_error": (_i, []),
    "mla_decode_split_num_splits": (_i, [_i, _i, _i, _u]),
    "mla_decode_split_head_tile": (_i, [_i, _i, _i, _u]),
    "mla_decode_split_launches": (_i, [_i, _i, _i, _u]),
    "mla_decode_split_workspace_size": (_sz, [_i, _i, _i]),
    "mla_decode_split_fp16": (_i, [_vp, _vp, _vp, _vp, _sz, _i, _i, _i, _vp]),
    "mla_decode_split_fp16_ex": (_i, [_vp, _vp, _vp, _vp, _sz, _i, _i, _i, _u, _vp]),
    "mla_decode_split_fp16_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "mla_decode_split_fp16_partials": (_i, [_vp, _vp, _vp, _sz, _i, _i, _i, _u, _vp]),
    "mla_decode_split_fp16_combine": (_i, [_vp, _sz, _vp, _i, _i, _i, _u, _vp]),
    "mla_decode_fused_workspace_size": (_sz, [_i, _i, _i]),
    "mla_decode_fused_fp32": (_i, [_vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "mla_decode_split_batched_workspace_size": (_sz, [_i, _i, _i, _i]),
    "mla_decode_split_batched_fp16": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "mla_decode_split_batched_fp16_partials": (_i, [_vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "mla_decode_split_batched_fp16_combine": (_i, [_vp, _sz, _vp, _vp, _i, _i, _i, _i, _vp]),
    "mla_decode_split_bf16": (_i, [_vp, _vp, _vp, _vp, _sz, _i, _i, _i, _vp]),
    "mla_decode_split_batched_bf16": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "mla_decode_paged_workspace_size": (_sz, [_i, _i, _i, _i]),
    "mla_project_output_workspace_size": (_sz, [_i, _i, _i]),
    "mla_decode_split_fp8_workspace_size": (_sz, [_i, _i, _i, _i]),
    "mla_decode_split_fp8": (_i, [_vp, _vp, ctypes.c_float, _vp, _vp, _sz, _i, _i, _i, _vp]),
    "mla_decode_split_batched_fp8": (_i, [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "mla_absorb_query_fp16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp]),
    "mla_absorb_query_bf16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp]),
    "mla_project_output_fp16": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _vp]),
    "mla_project_output_bf16": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _vp]),
    "mla_decode_paged_fp16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "mla_decode_paged_bf16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _i, _vp]),
}

_lib = None


class MlaError(RuntimeError):
    def __init__(self, fn: str, status: int):
        lib = load()
        msg = lib.mla_status_string(status).decode()
        if status == STATUS_HIP_ERROR:
            msg += f" (hipError_t {lib.mla_last_hip_error()})"
        super().__init__(f"{fn}: {msg}")
        self.status = status


def load():
    """Load libmla_mi355x.so (after torch, so that the library binds to the
    HIP runtime torch already loaded). Raises if the library is not built."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built (run python ada-mla_amd/build.py)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _lib = lib
    return _lib


def declared_functions() -> list[str]:
    """Function names declared in include/mla_mi355x.h."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mla_[a-z0-9_]+)\s*\(", text)))


def _stream(t):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _check(fn: str, st: int):
    if st != STATUS_SUCCESS:
        raise MlaError(fn, st)


def decode_split_fp16(q, c, num_splits: int = 0, flags: int = 0, out=None):
    """fp16 decode through mla_decode_split_fp16_ex: q [n_h, 576], c [N, 576]."""
    import torch
    lib = load()
    assert q.dtype == torch.float16 and c.dtype == torch.float16
    assert q.is_contiguous() and c.is_contiguous() and q.shape[1] == HEAD_DIM_K and c.shape[1] == HEAD_DIM_K
    n_h, n = q.shape[0], c.shape[0]
    if out is None:
        out = torch.empty((n_h, HEAD_DIM_V), dtype=torch.float16, device=q.device)
    ws_bytes = lib.mla_decode_split_workspace_size(n_h, n, num_splits)
    if ws_bytes == 0:
        raise MlaError("mla_decode_split_workspace_size", STATUS_INVALID_VALUE)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    _check("mla_decode_split_fp16_ex",
           lib.mla_decode_split_fp16_ex(q.data_ptr(), c.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                        ws_bytes, n_h, n, num_splits, flags, _stream(q)))
    return out


def decode_fused_fp32(q, c, num_splits: int = 0, out=None):
    """fp32 decode through mla_decode_fused_fp32."""
    import torch
    lib = load()
    assert q.dtype == torch.float32 and c.dtype == torch.float32
    assert q.is_contiguous() and c.is_contiguous()
    n_h, n = q.shape[0], c.shape[0]
    if out is None:
        out = torch.empty((n_h, HEAD_DIM_V), dtype=torch.float32, device=q.device)
    ws_bytes = lib.mla_decode_fused_workspace_size(n_h, n, num_splits)
    if ws_bytes == 0:
        raise MlaError("mla_decode_fused_workspace_size", STATUS_INVALID_VALUE)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    _check("mla_decode_fused_fp32",
           lib.mla_decode_fused_fp32(q.data_ptr(), c.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
                                     n_h, q.shape[1], n, num_splits, _stream(q)))
    return out


def decode_split_bf16(q, c, num_splits: int = 0, out=None):
    """bf16 decode through mla_decode_split_bf16: q [n_h, 576], c [N, 576]."""
    import torch
    lib = load()
    assert q.dtype == torch.bfloat16 and c.dtype == torch.bfloat16
    assert q.is_contiguous() and c.is_contiguous() and q.shape[1] == HEAD_DIM_K and c.shape[1] == HEAD_DIM_K
    n_h, n = q.shape[0], c.shape[0]
    if out is None:
        out = torch.empty((n_h, HEAD_DIM_V), dtype=torch.bfloat16, device=q.device)
    ws_bytes = lib.mla_decode_split_workspace_size(n_h, n, num_splits)
    if ws_bytes == 0:
        raise MlaError("mla_decode_split_workspace_size", STATUS_INVALID_VALUE)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    _check("mla_decode_split_bf16",
           lib.mla_decode_split_bf16(q.data_ptr(), c.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                     ws_bytes, n_h, n, num_splits, _stream(q)))
    return out


def decode_split_batched_bf16(q, c, cu_seqlens, num_splits: int = 0, out=None):
    """Batched bf16 decode (mla_decode_split_batched_bf16); shapes as decode_split_batched_fp16."""
    return _decode_batched(q, c, cu_seqlens, num_splits, out, "mla_decode_split_batched_bf16")


def decode_split_batched_fp16(q, c, cu_seqlens, num_splits: int = 0, out=None):
    """Batched fp16 decode: q [B, n_h, 576], c [sum N, 576], cu_seqlens [B+1] int32 (device)."""
    return _decode_batched(q, c, cu_seqlens, num_splits, out, "mla_decode_split_batched_fp16")


def _decode_batched(q, c, cu_seqlens, num_splits, out, fn):
    import torch
    lib = load()
    dt = torch.bfloat16 if fn.endswith("bf16") else torch.float16
    assert q.dtype == dt and c.dtype == dt and cu_seqlens.dtype == torch.int32
    assert q.is_contiguous() and c.is_contiguous() and cu_seqlens.is_contiguous()
    b, n_h = q.shape[0], q.shape[1]
    total = c.shape[0]
    if out is None:
        out = torch.empty((b, n_h, HEAD_DIM_V), dtype=dt, device=q.device)
    ws_bytes = lib.mla_decode_split_batched_workspace_size(b, n_h, total, num_splits)
    if ws_bytes == 0:
        raise MlaError("mla_decode_split_batched_workspace_size", STATUS_INVALID_VALUE)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    _check(fn, getattr(lib, fn)(q.data_ptr(), c.data_ptr() if total else None, cu_seqlens.data_ptr(),
                                out.data_ptr(), ws.data_ptr(), ws_bytes, b, n_h, total, num_splits,
                                _stream(q)))
    return out


def decode_paged(q, kv_cache, block_table, cu_seqlens, total_tokens: int, num_splits: int = 0, out=None):
    """Paged-KV decode (mla_decode_paged_fp16 / _bf16 by q's dtype): q [B, n_h, 576],
    kv_cache [num_pages, page_size, 576], block_table [B, max_pages] int32,
    cu_seqlens [B+1] int32 (device), total_tokens = cu_seqlens[B] (host)."""
    import torch
    lib = load()
    assert q.dtype in (torch.float16, torch.bfloat16) and kv_cache.dtype == q.dtype
    assert block_table.dtype == torch.int32 and cu_seqlens.dtype == torch.int32
    assert q.is_contiguous() and kv_cache.is_contiguous() and block_table.is_contiguous()
    b, n_h = q.shape[0], q.shape[1]
    num_pages, page_size = kv_cache.shape[0], kv_cache.shape[1]
    if out is None:
        out = torch.empty((b, n_h, HEAD_DIM_V), dtype=q.dtype, device=q.device)
    ws_bytes = lib.mla_decode_paged_workspace_size(b, n_h, total_tokens, num_splits)
    if ws_bytes == 0:
        raise MlaError("mla_decode_paged_workspace_size", STATUS_INVALID_VALUE)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    fn = "mla_decode_paged_fp16" if q.dtype == torch.float16 else "mla_decode_paged_bf16"
    _check(fn, getattr(lib, fn)(q.data_ptr(), kv_cache.data_ptr(), block_table.data_ptr(), cu_seqlens.data_ptr(),
                                out.data_ptr(), ws.data_ptr(), ws_bytes, b, n_h, total_tokens, page_size,
                                num_pages, block_table.shape[1], num_splits, _stream(q)))
    return out


def _suffix(t):
    import torch
    return {torch.float16: "fp16", torch.bfloat16: "bf16"}[t.dtype]


def absorb_query(q_nope, q_rope, w_uk, out=None):
    """Q* [B, n_h, 576] = [q_nope W_UK[h], q_rope] (mla_absorb_query_*): q_nope [B, n_h, 128],
    q_rope [B, n_h, 64], w_uk [n_h, 128, 512]."""
    import torch
    lib = load()
    b, n_h = q_nope.shape[0], q_nope.shape[1]
    assert q_nope.shape == (b, n_h, 128) and q_rope.shape == (b, n_h, 64) and w_uk.shape == (n_h, 128, 512)
    assert q_rope.dtype == q_nope.dtype == w_uk.dtype
    assert q_nope.is_contiguous() and q_rope.is_contiguous() and w_uk.is_contiguous()
    if out is None:
        out = torch.empty((b, n_h, HEAD_DIM_K), dtype=q_nope.dtype, device=q_nope.device)
    fn = "mla_absorb_query_" + _suffix(q_nope)
    _check(fn, getattr(lib, fn)(q_nope.data_ptr(), q_rope.data_ptr(), w_uk.data_ptr(), out.data_ptr(), b, n_h,
                                _stream(q_nope)))
    return out


def project_output(o_star, w_uv, w_o, out=None):
    """out [B, d_model] = concat_h(O*[:, h] W_UV[h]^T) W_O^T (mla_project_output_*): o_star
    [B, n_h, 512], w_uv [n_h, 128, 512], w_o [d_model, n_h * 128]."""
    import torch
    lib = load()
    b, n_h = o_star.shape[0], o_star.shape[1]
    d_model = w_o.shape[0]
    assert o_star.shape == (b, n_h, 512) and w_uv.shape == (n_h, 128, 512) and w_o.shape == (d_model, n_h * 128)
    assert o_star.dtype == w_uv.dtype == w_o.dtype
    assert o_star.is_contiguous() and w_uv.is_contiguous() and w_o.is_contiguous()
    if out is None:
        out = torch.empty((b, d_model), dtype=o_star.dtype, device=o_star.device)
    ws_bytes = lib.mla_project_output_workspace_size(b, n_h, d_model)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=o_star.device)
    fn = "mla_project_output_" + _suffix(o_star)
    _check(fn, getattr(lib, fn)(o_star.data_ptr(), w_uv.data_ptr(), w_o.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                ws_bytes, b, n_h, d_model, _stream(o_star)))
    return out


def decode_split_fp8(q, c_fp8, c_scale: float, num_splits: int = 0, out=None):
    """fp8-cache decode (mla_decode_split_fp8): q [n_h, 576] fp16, c_fp8 [N, 576] torch.float8_e4m3fn
    (or uint8 bytes) holding C / c_scale -> [n_h, 512] fp16."""
    import torch
    lib = load()
    assert q.dtype == torch.float16 and c_fp8.element_size() == 1
    assert q.is_contiguous() and c_fp8.is_contiguous() and q.shape[1] == HEAD_DIM_K and c_fp8.shape[1] == HEAD_DIM_K
    n_h, n = q.shape[0], c_fp8.shape[0]
    if out is None:
        out = torch.empty((n_h, HEAD_DIM_V), dtype=torch.float16, device=q.device)
    ws_bytes = lib.mla_decode_split_fp8_workspace_size(1, n_h, n, num_splits)
    if ws_bytes == 0:
        raise MlaError("mla_decode_split_fp8_workspace_size", STATUS_INVALID_VALUE)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    _check("mla_decode_split_fp8", lib.mla_decode_split_fp8(q.data_ptr(), c_fp8.data_ptr(), float(c_scale), out.data_ptr(),
                                                            ws.data_ptr(), ws_bytes, n_h, n, num_splits, _stream(q)))
    return out


def decode_split_batched_fp8(q, c_fp8, c_scale: float, cu_seqlens, num_splits: int = 0, out=None):
    """Batched fp8-cache decode (mla_decode_split_batched_fp8); shapes as decode_split_batched_fp16."""
    import torch
    lib = load()
    assert q.dtype == torch.float16 and c_fp8.element_size() == 1 and cu_seqlens.dtype == torch.int32
    b, n_h, total = q.shape[0], q.shape[1], c_fp8.shape[0]
    if out is None:
        out = torch.empty((b, n_h, HEAD_DIM_V), dtype=torch.float16, device=q.device)
    ws_bytes = lib.mla_decode_split_fp8_workspace_size(b, n_h, total, num_splits)
    if ws_bytes == 0:
        raise MlaError("mla_decode_split_fp8_workspace_size", STATUS_INVALID_VALUE)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    _check("mla_decode_split_batched_fp8",
           lib.mla_decode_split_batched_fp8(q.data_ptr(), c_fp8.data_ptr() if total else None, float(c_scale),
                                            cu_seqlens.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes, b, n_h,
                                            total, num_splits, _stream(q)))
    return out
