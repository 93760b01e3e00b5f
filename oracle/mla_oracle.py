"""CPU oracle for the weight-absorbed MLA decode path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker (or the timed CPU baseline). The product path (``ada_mla``) never
imports it and fails loudly when its HIP library is missing.

Contents, each restating a reference function:

``closed_form``          mla_decode_torch (mla.py:44-47):
                         softmax(q @ c.T / sqrt(192)) @ c[:, :512], in float64.
``sdpa_math``            mla_decode_sdpa with the MATH backend (mla.py:49-66):
                         key = c, value = c[:, :512], scale 1/sqrt(192); the
                         math backend scales q and k by sqrt(scale) each before
                         the product, restated the same way.
``closed_form_batched``  the batched decode (no reference counterpart: the
                         reference has no batch dimension, csrc/mla_api.cpp:67-69)
                         = closed_form applied per sequence of a packed cache.
``gather_paged`` /
``closed_form_paged``    the paged-KV decode (no reference counterpart): the
                         logical rows of every sequence gathered from the pages
                         its block-table row names, then closed_form_batched.
``absorb_query`` /
``project_output`` /
``block_unabsorbed``     the projections around the decode (no reference code;
                         the math is README.md:64-110): the absorbed query
                         [q_nope W_UK[h], q_rope], the value and output
                         projections, and the same attention computed without
                         absorption (keys C_N W_UK[h]^T and values C_N W_UV[h]^T
                         per head), which the absorbed path must equal.
``split_partials`` /
``lse_merge``            the split-KV partial results and the combine of
                         mla_decode_combine (csrc/mla_decode_splitk_fwd.cuh:894-939),
                         in float64 with the running max started at -inf
                         instead of the smallest fp16 denormal.
``naive_cpu``            ctypes binding of oracle/mla_naive_cpu.c, the C
                         restatement of run_mla_decode_cpu
                         (csrc/mla_decode_naive_fp32_cpu.cpp:5-61).
``reference_cpu``        ctypes binding of the reference's own run_mla_decode_cpu,
                         compiled from its source into oracle/_ref by
                         oracle/Makefile (absent where /root/reference was not).

Pinning (tests/test_oracle.py): ``naive_cpu`` in the reference's own form is
bit-identical to ``reference_cpu`` and to the committed golden vectors
written by it; ``closed_form`` agrees with the reference kernel through the
exact identity 1/sqrt(192) = sqrt(3)/sqrt(576); the closed form is checked
against textbook special cases (N = 1, equal rows, q = 0, a dominant logit,
token permutation, brute force on tiny shapes); ``lse_merge`` against the
unsplit closed form for every split point on small inputs.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

HEAD_DIM_C = 512   # mla.py:31
HEAD_DIM_ROPE = 64  # mla.py:32
HEAD_DIM_K = HEAD_DIM_C + HEAD_DIM_ROPE  # mla.py:33 (576)
HEAD_DIM = 128     # mla.py:30; the softmax scale uses HEAD_DIM + HEAD_DIM_ROPE
SCALE = 1.0 / math.sqrt(HEAD_DIM + HEAD_DIM_ROPE)  # mla.py:46: 1/sqrt(192)
REF_CPU_DIVISOR = math.sqrt(HEAD_DIM_K)            # cpu.cpp:24: sqrt(576)

_HERE = os.path.dirname(os.path.abspath(__file__))
_ORACLE_LIB = os.path.join(_HERE, "liboracle_mla.so")
_REF_LIB = os.path.join(_HERE, "_ref", "libref_mla_cpu.so")


def _softmax_rows(x: np.ndarray) -> np.ndarray:
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def closed_form(q, c, scale: float = SCALE, dv: int = HEAD_DIM_C) -> np.ndarray:
    """softmax(scale * q c^T) c[:, :dv] in float64 (mla.py:44-47)."""
    q = np.asarray(q, dtype=np.float64)
    c = np.asarray(c, dtype=np.float64)
    if q.ndim != 2 or c.ndim != 2 or q.shape[1] != c.shape[1] or c.shape[0] < 1:
        raise ValueError("closed_form: q [n_h, d], c [N>=1, d] expected")
    p = _softmax_rows((q @ c.T) * scale)
    return p @ c[:, :dv]


def sdpa_math(q, c, scale: float = SCALE, dv: int = HEAD_DIM_C) -> np.ndarray:
    """SDPA math-backend form of mla.py:49-62 (key = c, value = c[:, :512]):
    q and k are each multiplied by sqrt(scale) before the product."""
    q = np.asarray(q, dtype=np.float64)
    c = np.asarray(c, dtype=np.float64)
    s = math.sqrt(scale)
    p = _softmax_rows((q * s) @ (c * s).T)
    return p @ c[:, :dv]


def closed_form_batched(q, c_packed, cu_seqlens, scale: float = SCALE,
                        dv: int = HEAD_DIM_C) -> np.ndarray:
    """Per-sequence closed form over a packed cache: q [B, n_h, d], c_packed
    [sum N_b, d], cu_seqlens [B + 1]. An empty sequence yields zeros."""
    q = np.asarray(q, dtype=np.float64)
    c_packed = np.asarray(c_packed, dtype=np.float64)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    B = q.shape[0]
    out = np.zeros((B, q.shape[1], dv), dtype=np.float64)
    for b in range(B):
        lo, hi = int(cu[b]), int(cu[b + 1])
        if hi > lo:
            out[b] = closed_form(q[b], c_packed[lo:hi], scale, dv)
    return out


def gather_paged(kv_pages, block_table, cu_seqlens) -> np.ndarray:
    """Packed cache [sum N_b, d] of a paged one: token l of sequence b is row
    l % page_size of page block_table[b, l // page_size] of kv_pages
    [num_pages, page_size, d]."""
    kv = np.asarray(kv_pages)
    bt = np.asarray(block_table, dtype=np.int64)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    page = kv.shape[1]
    rows = []
    for b in range(bt.shape[0]):
        n = int(cu[b + 1] - cu[b])
        l = np.arange(n)
        rows.append(kv[bt[b, l // page], l % page])
    return np.concatenate(rows, axis=0) if rows else kv[:0, 0]


def closed_form_paged(q, kv_pages, block_table, cu_seqlens, scale: float = SCALE,
                      dv: int = HEAD_DIM_C) -> np.ndarray:
    """closed_form_batched over the sequences of a paged cache."""
    return closed_form_batched(q, gather_paged(kv_pages, block_table, cu_seqlens), cu_seqlens, scale, dv)


def absorb_query(q_nope, q_rope, w_uk) -> np.ndarray:
    """Q* [B, n_h, 576]: Q*[b, h, :512] = q_nope[b, h] @ w_uk[h] (w_uk [n_h, 128, 512]),
    Q*[b, h, 512:] = q_rope[b, h] -- q*_i = c^Q W^UQ_i (W^UK_i)^T of README.md:76-80
    without the scale, which the decode applies."""
    q_nope = np.asarray(q_nope, dtype=np.float64)
    w_uk = np.asarray(w_uk, dtype=np.float64)
    nope = np.einsum("bhk,hkd->bhd", q_nope, w_uk)
    return np.concatenate([nope, np.asarray(q_rope, dtype=np.float64)], axis=2)


def project_output(o_star, w_uv, w_o) -> np.ndarray:
    """out [B, d_model] = concat_h(o_star[:, h] @ w_uv[h]^T) @ w_o^T (README.md:84-85)."""
    o_star = np.asarray(o_star, dtype=np.float64)
    o = np.einsum("bhd,hkd->bhk", o_star, np.asarray(w_uv, dtype=np.float64))
    return o.reshape(o.shape[0], -1) @ np.asarray(w_o, dtype=np.float64).T


def block_unabsorbed(q_nope, q_rope, c_packed, cu_seqlens, w_uk, w_uv, w_o,
                     scale: float = SCALE) -> np.ndarray:
    """The decode step of an MLA block without weight absorption: per head,
    keys [C_N W_UK[h]^T, C_R] and values C_N W_UV[h]^T, softmax attention with
    the query [q_nope, q_rope], then the output projection. Equal to
    project_output(closed_form_batched(absorb_query(...)), ...) in exact
    arithmetic (README.md:68-80)."""
    q_nope = np.asarray(q_nope, dtype=np.float64)
    q_rope = np.asarray(q_rope, dtype=np.float64)
    c = np.asarray(c_packed, dtype=np.float64)
    w_uk = np.asarray(w_uk, dtype=np.float64)
    w_uv = np.asarray(w_uv, dtype=np.float64)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    B, n_h = q_nope.shape[0], q_nope.shape[1]
    o = np.zeros((B, n_h, w_uv.shape[1]))
    for b in range(B):
        cb = c[cu[b]:cu[b + 1]]
        if cb.shape[0] == 0:
            continue
        for h in range(n_h):
            k = np.concatenate([cb[:, :HEAD_DIM_C] @ w_uk[h].T, cb[:, HEAD_DIM_C:]], axis=1)
            v = cb[:, :HEAD_DIM_C] @ w_uv[h].T
            q = np.concatenate([q_nope[b, h], q_rope[b, h]])
            p = _softmax_rows((q @ k.T)[None, :] * scale)[0]
            o[b, h] = p @ v
    return o.reshape(B, -1) @ np.asarray(w_o, dtype=np.float64).T


def split_partials(q, c, bounds, scale: float = SCALE, dv: int = HEAD_DIM_C):
    """Unnormalised per-split results (O_s, m_s, l_s) for token ranges
    [bounds[s], bounds[s+1]): m_s = max logit, l_s = sum exp(logit - m_s),
    O_s = sum exp(logit - m_s) c[:, :dv]. This is what each split CTA of
    mla_decode_splitk_mma_fp16 stores (csrc/mla_decode_splitk_fwd.cuh:880-891),
    here in float64 with natural-log units."""
    q = np.asarray(q, dtype=np.float64)
    c = np.asarray(c, dtype=np.float64)
    outs, ms, ls = [], [], []
    for s in range(len(bounds) - 1):
        lo, hi = bounds[s], bounds[s + 1]
        if hi <= lo:
            outs.append(np.zeros((q.shape[0], dv)))
            ms.append(np.full(q.shape[0], -np.inf))
            ls.append(np.zeros(q.shape[0]))
            continue
        logits = (q @ c[lo:hi].T) * scale
        m = logits.max(axis=1)
        e = np.exp(logits - m[:, None])
        outs.append(e @ c[lo:hi, :dv])
        ms.append(m)
        ls.append(e.sum(axis=1))
    return np.stack(outs), np.stack(ms), np.stack(ls)


def lse_merge(o_parts, m_parts, l_parts) -> np.ndarray:
    """Combine of mla_decode_combine (csrc/mla_decode_splitk_fwd.cuh:894-939):
    m = max_s m_s; l = sum_s l_s e^(m_s - m); O = sum_s O_s e^(m_s - m) / l.
    The running max starts at -inf (the reference starts at the smallest fp16
    denormal, :916); splits with m_s = -inf (no tokens) contribute nothing."""
    o_parts = np.asarray(o_parts, dtype=np.float64)
    m_parts = np.asarray(m_parts, dtype=np.float64)
    l_parts = np.asarray(l_parts, dtype=np.float64)
    m = np.max(m_parts, axis=0)
    w = np.where(np.isneginf(m_parts), 0.0, np.exp(m_parts - m[None, :]))
    l = (l_parts * w).sum(axis=0)
    o = (o_parts * w[:, :, None]).sum(axis=0)
    return o / l[:, None]


def _load(path: str):
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    return lib


_oracle_lib = None


def naive_cpu(q, c, divisor: float = 1.0 / SCALE, dv: int = HEAD_DIM_C) -> np.ndarray:
    """C restatement of run_mla_decode_cpu (cpu.cpp:5-61) on float32 inputs.
    divisor = sqrt(576), dv = 576 is the reference's own form; the default is
    the decode contract (1/scale = sqrt(192), dv = 512)."""
    global _oracle_lib
    if _oracle_lib is None:
        _oracle_lib = _load(_ORACLE_LIB)
        if _oracle_lib is None:
            raise RuntimeError(f"{_ORACLE_LIB} not built (run make -C oracle)")
        f = _oracle_lib.oracle_mla_decode_cpu
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                      ctypes.c_double]
    q = np.ascontiguousarray(q, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.float32)
    n_h, d = q.shape
    n = c.shape[0]
    if c.shape[1] != d or dv > d:
        raise ValueError("naive_cpu: shape mismatch")
    out = np.empty((n_h, dv), dtype=np.float32)
    rc = _oracle_lib.oracle_mla_decode_cpu(q.ctypes.data, c.ctypes.data,
                                           out.ctypes.data, n_h, d, n, dv,
                                           float(divisor))
    if rc != 0:
        raise RuntimeError(f"oracle_mla_decode_cpu failed: {rc}")
    return out


_ref_lib = None


def reference_cpu_available() -> bool:
    return os.path.exists(_REF_LIB)


def reference_cpu(q, c) -> np.ndarray:
    """The reference's own run_mla_decode_cpu (scale 1/sqrt(576), all 576
    output columns), compiled from its source into oracle/_ref."""
    global _ref_lib
    if _ref_lib is None:
        _ref_lib = _load(_REF_LIB)
        if _ref_lib is None:
            raise RuntimeError(f"{_REF_LIB} not built (make -C oracle ref)")
        f = _ref_lib.ref_run_mla_decode_cpu
        f.restype = None
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                      ctypes.c_int, ctypes.c_int, ctypes.c_int]
    q = np.ascontiguousarray(q, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.float32)
    n_h, d = q.shape
    out = np.empty((n_h, d), dtype=np.float32)
    _ref_lib.ref_run_mla_decode_cpu(q.ctypes.data, c.ctypes.data,
                                    out.ctypes.data, n_h, d, c.shape[0])
    return out
