"""ada_mla -- MI355X (gfx950) MLA decode, a drop-in for the fused path of the
reference's ``ada_mla`` extension module (csrc/mla_api.cpp:115-120).

    import ada_mla
    out = ada_mla.mla_decode_split(q, c)   # fp16: q [n_h, 576], c [N, 576] -> [n_h, 512]
    out = ada_mla.mla_decode_fused(q, c)   # fp32 (the reference's --fp32 path)
    out = ada_mla.mla_decode_split_batched(q, c_packed, cu_seqlens)  # [B, n_h, 512]
    out = ada_mla.mla_decode_paged(q, kv_pages, block_table, cu_seqlens)  # paged KV cache
    q = ada_mla.mla_absorb_query(q_nope, q_rope, w_uk)     # the projections around
    y = ada_mla.mla_project_output(o_star, w_uv, w_o)      # the decode (MLA block)

The functions live in the compiled extension ``ada_mla._C`` (built by
ada-mla_amd/build.py), which calls the HIP library through its C ABI
(include/mla_mi355x.h). They are resolved on first use; if the extension is
missing, that use raises ImportError -- there is no fallback path.
"""
from __future__ import annotations

import importlib

__all__ = ["mla_decode_split", "mla_decode_fused", "mla_decode_split_batched", "mla_decode_paged",
           "mla_absorb_query", "mla_project_output", "HEAD_DIM_C", "HEAD_DIM_ROPE", "HEAD_DIM_K", "extension"]

_EXPORTS = {"mla_decode_split", "mla_decode_fused", "mla_decode_split_batched", "mla_decode_paged",
            "mla_absorb_query", "mla_project_output", "HEAD_DIM_C", "HEAD_DIM_ROPE", "HEAD_DIM_K"}


def extension():
    """The compiled extension module; raises ImportError if it is not built."""
    import torch  # noqa: F401  -- load torch's HIP runtime before the extension's
    try:
        return importlib.import_module(__name__ + "._C")
    except ImportError as e:  # pragma: no cover - exercised only without a build
        raise ImportError(
            "ada_mla: the HIP extension ada_mla._C is not built "
            "(run `python ada-mla_amd/build.py`); there is no CPU fallback") from e


def __getattr__(name):
    if name in _EXPORTS:
        return getattr(extension(), name)
    raise AttributeError(f"module 'ada_mla' has no attribute {name!r}")
