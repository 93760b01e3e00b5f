// PyTorch extension `ada_mla._C`: the Python surface of the reference's
// extension module `ada_mla` (csrc/mla_api.cpp:115-120), with the same
// function names and (query, cache) -> out contract, implemented over the
// C ABI in include/mla_mi355x.h.
//
// Differences from the reference, all on inputs it mishandled:
//  * inputs are validated (device, dtype, rank, 576 columns, num_heads a
//    multiple of 16, N >= 1) and made contiguous; errors raise instead of
//    being printf'd (reference TODOs csrc/mla_api.cpp:8, :18, :91).
//  * kernels run on torch's current HIP stream of the input's device, not
//    the legacy default stream.
//  * mla_decode_split accepts fp32 as well (the reference's fp32 split
//    launcher is an empty stub, csrc/mla_decode_splitk_fwd_sm89.cu:8-24, and
//    returned uninitialised memory); mla_decode_fused accepts fp16 as well
//    (the reference read any dtype as float*, csrc/mla_api.cpp:46-48).
//  * an optional num_splits keyword (default: chosen from N and the CU count).
//  * bf16 query/cache are accepted by mla_decode_split, mla_decode_fused and
//    mla_decode_split_batched (bf16 MFMAs; the reference lists bf16 as
//    future work, README.md:405-408).
//  * mla_decode_split and mla_decode_split_batched also take a float8_e4m3fn
//    cache with a float16 query: the cache holds C / cache_scale (keyword
//    cache_scale, default 1) and is read at one byte per value (fp8 is
//    future work in the reference too, README.md:408).
#include <torch/extension.h>

#include <cmath>

#include <c10/hip/HIPStream.h>

#include "mla_mi355x.h"

namespace {

void check_status(int st, const char *fn)
{
    TORCH_CHECK(st == MLA_STATUS_SUCCESS, fn, ": ", mla_status_string(st),
                st == MLA_STATUS_HIP_ERROR ? " (hipError_t " + std::to_string(mla_last_hip_error()) + ")"
                                           : std::string());
}

// Shape and dtype are checked before the device so that every argument error
// is reported the same way whatever the tensors' device.
bool is_fp8_cache(const at::Tensor &query, const at::Tensor &cache)
{
    return cache.scalar_type() == at::kFloat8_e4m3fn && query.scalar_type() == at::kHalf;
}

void check_cache_scale(double cache_scale, const char *fn)
{
    TORCH_CHECK(std::isfinite(cache_scale) && cache_scale > 0, fn, ": cache_scale must be finite and > 0, got ",
                cache_scale);
}

void check_pair(const at::Tensor &query, const at::Tensor &cache, const char *fn)
{
    TORCH_CHECK(query.scalar_type() == cache.scalar_type() || is_fp8_cache(query, cache), fn,
                ": query and cache must have the same dtype (or a float16 query with a float8_e4m3fn cache)");
    TORCH_CHECK(query.scalar_type() == at::kHalf || query.scalar_type() == at::kBFloat16 ||
                    query.scalar_type() == at::kFloat,
                fn, ": dtype must be float16, bfloat16 or float32, got ", query.scalar_type());
    TORCH_CHECK(cache.dim() == 2 && cache.size(1) == MLA_HEAD_DIM_K, fn, ": cache must be [N, ",
                MLA_HEAD_DIM_K, "], got ", cache.sizes());
    TORCH_CHECK(cache.size(0) >= 1, fn, ": cache must hold at least one token");
    TORCH_CHECK(cache.size(0) <= INT32_MAX, fn, ": too many tokens");
    TORCH_CHECK(query.dim() == 2 && query.size(1) == MLA_HEAD_DIM_K, fn,
                ": query must be [num_heads, ", MLA_HEAD_DIM_K, "], got ", query.sizes());
    TORCH_CHECK(query.size(0) > 0 && query.size(0) % 16 == 0 && query.size(0) <= 4096, fn,
                ": num_heads must be a positive multiple of 16 (<= 4096), got ", query.size(0));
    TORCH_CHECK(query.is_cuda() && cache.is_cuda(), fn, ": query and cache must be GPU tensors");
    TORCH_CHECK(query.device() == cache.device(), fn, ": query and cache must be on the same device");
}

void check_heads(int64_t num_heads, const char *fn)
{
    TORCH_CHECK(num_heads > 0 && num_heads % 16 == 0 && num_heads <= 4096, fn,
                ": num_heads must be a positive multiple of 16 (<= 4096), got ", num_heads);
}

void *stream_of(const at::Tensor &t)
{
    return static_cast<void *>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

at::Tensor workspace(size_t bytes, const at::Tensor &like)
{
    return at::empty({static_cast<int64_t>(bytes)}, like.options().dtype(at::kByte));
}

// Single sequence, dispatch on dtype.
at::Tensor decode_single(const at::Tensor &query_in, const at::Tensor &cache_in, int64_t num_splits,
                         double cache_scale, const char *fn)
{
    const bool fp8 = is_fp8_cache(query_in, cache_in);
    if (fp8)
        check_cache_scale(cache_scale, fn);
    check_pair(query_in, cache_in, fn);
    const at::OptionalDeviceGuard guard(query_in.device());
    const at::Tensor query = query_in.contiguous();
    const at::Tensor cache = cache_in.contiguous();
    const int nh = static_cast<int>(query.size(0));
    const int n = static_cast<int>(cache.size(0));
    const int splits = static_cast<int>(num_splits);
    at::Tensor out = at::empty({nh, MLA_HEAD_DIM_V}, query.options());
    int st;
    if (fp8) {
        const size_t ws_bytes = mla_decode_split_fp8_workspace_size(1, nh, n, splits);
        TORCH_CHECK(ws_bytes > 0, fn, ": unsupported sizes");
        at::Tensor ws = workspace(ws_bytes, query);
        st = mla_decode_split_fp8(query.data_ptr(), cache.data_ptr(), static_cast<float>(cache_scale),
                                  out.data_ptr(), ws.data_ptr(), ws_bytes, nh, n, splits, stream_of(query));
    } else if (query.scalar_type() != at::kFloat) {
        const size_t ws_bytes = mla_decode_split_workspace_size(nh, n, splits);
        TORCH_CHECK(ws_bytes > 0, fn, ": unsupported sizes");
        at::Tensor ws = workspace(ws_bytes, query);
        auto f = query.scalar_type() == at::kHalf ? mla_decode_split_fp16 : mla_decode_split_bf16;
        st = f(query.data_ptr(), cache.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes, nh, n, splits,
               stream_of(query));
    } else {
        const size_t ws_bytes = mla_decode_fused_workspace_size(nh, n, splits);
        TORCH_CHECK(ws_bytes > 0, fn, ": unsupported sizes");
        at::Tensor ws = workspace(ws_bytes, query);
        st = mla_decode_fused_fp32(query.data_ptr<float>(), cache.data_ptr<float>(), out.data_ptr<float>(),
                                   ws.data_ptr(), ws_bytes, nh, MLA_HEAD_DIM_K, n, splits,
                                   stream_of(query));
    }
    check_status(st, fn);
    return out;
}

// Reference: mla_decode_split (csrc/mla_api.cpp:86-113), the fp16 `-k fused`
// path of mla.py (mla.py:177-179).
at::Tensor mla_decode_split(const at::Tensor &query, const at::Tensor &cache, int64_t num_splits,
                            double cache_scale)
{
    return decode_single(query, cache, num_splits, cache_scale, "mla_decode_split");
}

// Reference: mla_decode_fused (csrc/mla_api.cpp:34-54), the `-k fused --fp32`
// path of mla.py (mla.py:174-176).
at::Tensor mla_decode_fused(const at::Tensor &query, const at::Tensor &cache, int64_t num_splits)
{
    TORCH_CHECK(cache.scalar_type() != at::kFloat8_e4m3fn, "mla_decode_fused: fp8 caches go through mla_decode_split");
    return decode_single(query, cache, num_splits, 1.0, "mla_decode_fused");
}

// No reference counterpart: B independent sequences packed back to back.
at::Tensor mla_decode_split_batched(const at::Tensor &query_in, const at::Tensor &cache_in,
                                    const at::Tensor &cu_seqlens_in, int64_t num_splits, double cache_scale)
{
    const char *fn = "mla_decode_split_batched";
    const bool fp8 = is_fp8_cache(query_in, cache_in);
    TORCH_CHECK(fp8 || (query_in.scalar_type() == cache_in.scalar_type() &&
                        (query_in.scalar_type() == at::kHalf || query_in.scalar_type() == at::kBFloat16)),
                fn, ": query and cache must both be float16 or both bfloat16 (or a float16 query with a "
                "float8_e4m3fn cache)");
    if (fp8)
        check_cache_scale(cache_scale, fn);
    TORCH_CHECK(cu_seqlens_in.scalar_type() == at::kInt && cu_seqlens_in.dim() == 1, fn,
                ": cu_seqlens must be a 1-D int32 tensor");
    TORCH_CHECK(query_in.dim() == 3 && query_in.size(2) == MLA_HEAD_DIM_K, fn,
                ": query must be [batch, num_heads, ", MLA_HEAD_DIM_K, "], got ", query_in.sizes());
    TORCH_CHECK(cache_in.dim() == 2 && cache_in.size(1) == MLA_HEAD_DIM_K, fn, ": cache must be [total, ",
                MLA_HEAD_DIM_K, "], got ", cache_in.sizes());
    TORCH_CHECK(query_in.size(0) >= 1 && cu_seqlens_in.size(0) == query_in.size(0) + 1, fn,
                ": cu_seqlens must have batch + 1 entries");
    TORCH_CHECK(cache_in.size(0) <= INT32_MAX, fn, ": too many tokens");
    check_heads(query_in.size(1), fn);
    TORCH_CHECK(query_in.is_cuda() && cache_in.is_cuda() && cu_seqlens_in.is_cuda(), fn,
                ": query, cache and cu_seqlens must be GPU tensors");
    TORCH_CHECK(query_in.device() == cache_in.device() && query_in.device() == cu_seqlens_in.device(), fn,
                ": all inputs must be on the same device");
    const at::OptionalDeviceGuard guard(query_in.device());
    const at::Tensor query = query_in.contiguous();
    const at::Tensor cache = cache_in.contiguous();
    const at::Tensor cu = cu_seqlens_in.contiguous();
    const int batch = static_cast<int>(query.size(0));
    const int nh = static_cast<int>(query.size(1));
    const int total = static_cast<int>(cache.size(0));
    const int splits = static_cast<int>(num_splits);
    at::Tensor out = at::empty({batch, nh, MLA_HEAD_DIM_V}, query.options());
    const size_t ws_bytes = fp8 ? mla_decode_split_fp8_workspace_size(batch, nh, total, splits)
                                : mla_decode_split_batched_workspace_size(batch, nh, total, splits);
    TORCH_CHECK(ws_bytes > 0, fn, ": unsupported sizes");
    at::Tensor ws = workspace(ws_bytes, query);
    const void *c = total > 0 ? cache.data_ptr() : nullptr;
    int st;
    if (fp8) {
        st = mla_decode_split_batched_fp8(query.data_ptr(), c, static_cast<float>(cache_scale), cu.data_ptr<int>(),
                                          out.data_ptr(), ws.data_ptr(), ws_bytes, batch, nh, total, splits,
                                          stream_of(query));
    } else {
        auto f = query.scalar_type() == at::kHalf ? mla_decode_split_batched_fp16 : mla_decode_split_batched_bf16;
        st = f(query.data_ptr(), c, cu.data_ptr<int>(), out.data_ptr(), ws.data_ptr(), ws_bytes, batch, nh, total,
               splits, stream_of(query));
    }
    check_status(st, fn);
    return out;
}

// No reference counterpart: a paged KV cache [num_pages, page_size, 576]
// addressed through block_table [batch, max_pages] (int32), with the
// sequences' lengths as prefix sums cu_seqlens [batch + 1] (int32).
// total_tokens (= cu_seqlens[batch]) is read from the device when not given,
// which synchronises the stream. A given total_tokens is not checked against
// cu_seqlens[batch]: sequences are clipped to [0, total_tokens), so a smaller
// value silently truncates the trailing sequences; a larger one only changes
// the split plan.
at::Tensor mla_decode_paged(const at::Tensor &query_in, const at::Tensor &kv_in,
                            const at::Tensor &block_table_in, const at::Tensor &cu_seqlens_in,
                            int64_t total_tokens, int64_t num_splits)
{
    const char *fn = "mla_decode_paged";
    TORCH_CHECK(query_in.scalar_type() == kv_in.scalar_type() &&
                    (query_in.scalar_type() == at::kHalf || query_in.scalar_type() == at::kBFloat16),
                fn, ": query and kv_cache must both be float16 or both bfloat16");
    TORCH_CHECK(block_table_in.scalar_type() == at::kInt && block_table_in.dim() == 2, fn,
                ": block_table must be a 2-D int32 tensor");
    TORCH_CHECK(cu_seqlens_in.scalar_type() == at::kInt && cu_seqlens_in.dim() == 1, fn,
                ": cu_seqlens must be a 1-D int32 tensor");
    TORCH_CHECK(query_in.dim() == 3 && query_in.size(2) == MLA_HEAD_DIM_K, fn,
                ": query must be [batch, num_heads, ", MLA_HEAD_DIM_K, "], got ", query_in.sizes());
    TORCH_CHECK(kv_in.dim() == 3 && kv_in.size(2) == MLA_HEAD_DIM_K && kv_in.size(0) >= 1, fn,
                ": kv_cache must be [num_pages >= 1, page_size, ", MLA_HEAD_DIM_K, "], got ", kv_in.sizes());
    const int64_t page = kv_in.size(1);
    TORCH_CHECK(page >= 32 && (page & (page - 1)) == 0, fn, ": page_size must be a power of two >= 32, got ",
                page);
    TORCH_CHECK(kv_in.size(0) <= INT32_MAX, fn, ": too many pages");
    const int64_t batch = query_in.size(0);
    TORCH_CHECK(batch >= 1 && cu_seqlens_in.size(0) == batch + 1 && block_table_in.size(0) == batch, fn,
                ": cu_seqlens must have batch + 1 entries and block_table batch rows");
    TORCH_CHECK(block_table_in.size(1) >= 1, fn, ": block_table needs at least one column");
    check_heads(query_in.size(1), fn);
    TORCH_CHECK(query_in.is_cuda() && kv_in.is_cuda() && block_table_in.is_cuda() && cu_seqlens_in.is_cuda(), fn,
                ": all inputs must be GPU tensors");
    TORCH_CHECK(query_in.device() == kv_in.device() && query_in.device() == block_table_in.device() &&
                    query_in.device() == cu_seqlens_in.device(),
                fn, ": all inputs must be on the same device");
    const at::OptionalDeviceGuard guard(query_in.device());
    const at::Tensor query = query_in.contiguous();
    const at::Tensor kv = kv_in.contiguous();
    const at::Tensor bt = block_table_in.contiguous();
    const at::Tensor cu = cu_seqlens_in.contiguous();
    if (total_tokens < 0)
        total_tokens = cu[batch].item<int>();
    TORCH_CHECK(total_tokens >= 0 && total_tokens <= INT32_MAX, fn, ": bad total_tokens ", total_tokens);
    const int nh = static_cast<int>(query.size(1));
    const int total = static_cast<int>(total_tokens);
    const int splits = static_cast<int>(num_splits);
    at::Tensor out = at::empty({batch, nh, MLA_HEAD_DIM_V}, query.options());
    const size_t ws_bytes = mla_decode_paged_workspace_size(static_cast<int>(batch), nh, total, splits);
    TORCH_CHECK(ws_bytes > 0, fn, ": unsupported sizes");
    at::Tensor ws = workspace(ws_bytes, query);
    auto f = query.scalar_type() == at::kHalf ? mla_decode_paged_fp16 : mla_decode_paged_bf16;
    const int st = f(query.data_ptr(), kv.data_ptr(), bt.data_ptr<int>(), cu.data_ptr<int>(), out.data_ptr(),
                     ws.data_ptr(), ws_bytes, static_cast<int>(batch), nh, total, static_cast<int>(page),
                     static_cast<int>(kv.size(0)), static_cast<int>(bt.size(1)), splits, stream_of(query));
    check_status(st, fn);
    return out;
}

void check_16bit(const at::Tensor &t, at::ScalarType dt, const char *fn, const char *name)
{
    TORCH_CHECK(t.scalar_type() == dt, fn, ": ", name, " must have the query's dtype (float16 or bfloat16)");
    TORCH_CHECK(t.is_cuda(), fn, ": ", name, " must be a GPU tensor");
}

// No reference code (the math is README.md:76-85): Q* = [q_nope W_UK[h], q_rope].
at::Tensor mla_absorb_query(const at::Tensor &q_nope_in, const at::Tensor &q_rope_in, const at::Tensor &w_uk_in)
{
    const char *fn = "mla_absorb_query";
    const auto dt = q_nope_in.scalar_type();
    TORCH_CHECK(dt == at::kHalf || dt == at::kBFloat16, fn, ": q_nope must be float16 or bfloat16");
    TORCH_CHECK(q_nope_in.dim() == 3 && q_nope_in.size(2) == 128 && q_nope_in.size(0) >= 1, fn,
                ": q_nope must be [batch, num_heads, 128], got ", q_nope_in.sizes());
    const int64_t b = q_nope_in.size(0), nh = q_nope_in.size(1);
    TORCH_CHECK(q_rope_in.dim() == 3 && q_rope_in.size(0) == b && q_rope_in.size(1) == nh && q_rope_in.size(2) == 64,
                fn, ": q_rope must be [batch, num_heads, 64], got ", q_rope_in.sizes());
    TORCH_CHECK(w_uk_in.dim() == 3 && w_uk_in.size(0) == nh && w_uk_in.size(1) == 128 && w_uk_in.size(2) == 512, fn,
                ": w_uk must be [num_heads, 128, 512], got ", w_uk_in.sizes());
    check_16bit(q_nope_in, dt, fn, "q_nope");
    check_16bit(q_rope_in, dt, fn, "q_rope");
    check_16bit(w_uk_in, dt, fn, "w_uk");
    const at::OptionalDeviceGuard guard(q_nope_in.device());
    const at::Tensor qn = q_nope_in.contiguous(), qr = q_rope_in.contiguous(), w = w_uk_in.contiguous();
    at::Tensor out = at::empty({b, nh, MLA_HEAD_DIM_K}, qn.options());
    auto f = dt == at::kHalf ? mla_absorb_query_fp16 : mla_absorb_query_bf16;
    check_status(f(qn.data_ptr(), qr.data_ptr(), w.data_ptr(), out.data_ptr(), static_cast<int>(b),
                   static_cast<int>(nh), stream_of(qn)),
                 fn);
    return out;
}

// No reference code (README.md:84-85): out = concat_h(O*[:, h] W_UV[h]^T) W_O^T.
at::Tensor mla_project_output(const at::Tensor &o_in, const at::Tensor &w_uv_in, const at::Tensor &w_o_in)
{
    const char *fn = "mla_project_output";
    const auto dt = o_in.scalar_type();
    TORCH_CHECK(dt == at::kHalf || dt == at::kBFloat16, fn, ": o_star must be float16 or bfloat16");
    TORCH_CHECK(o_in.dim() == 3 && o_in.size(2) == MLA_HEAD_DIM_V && o_in.size(0) >= 1, fn,
                ": o_star must be [batch, num_heads, 512], got ", o_in.sizes());
    const int64_t b = o_in.size(0), nh = o_in.size(1);
    TORCH_CHECK(w_uv_in.dim() == 3 && w_uv_in.size(0) == nh && w_uv_in.size(1) == 128 && w_uv_in.size(2) == 512, fn,
                ": w_uv must be [num_heads, 128, 512], got ", w_uv_in.sizes());
    TORCH_CHECK(w_o_in.dim() == 2 && w_o_in.size(1) == nh * 128 && w_o_in.size(0) >= 1, fn,
                ": w_o must be [d_model, num_heads * 128], got ", w_o_in.sizes());
    check_16bit(o_in, dt, fn, "o_star");
    check_16bit(w_uv_in, dt, fn, "w_uv");
    check_16bit(w_o_in, dt, fn, "w_o");
    const at::OptionalDeviceGuard guard(o_in.device());
    const at::Tensor o = o_in.contiguous(), wuv = w_uv_in.contiguous(), wo = w_o_in.contiguous();
    const int64_t d_model = wo.size(0);
    at::Tensor out = at::empty({b, d_model}, o.options());
    const size_t ws_bytes = mla_project_output_workspace_size(static_cast<int>(b), static_cast<int>(nh), static_cast<int>(d_model));
    TORCH_CHECK(ws_bytes > 0, fn, ": unsupported sizes");
    at::Tensor ws = workspace(ws_bytes, o);
    auto f = dt == at::kHalf ? mla_project_output_fp16 : mla_project_output_bf16;
    check_status(f(o.data_ptr(), wuv.data_ptr(), wo.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
                   static_cast<int>(b), static_cast<int>(nh), static_cast<int>(d_model), stream_of(o)),
                 fn);
    return out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m)
{
    m.doc() = "MI355X (gfx950) MLA decode: drop-in for the ada_mla extension's fused path";
    m.def("mla_decode_split", &mla_decode_split,
          "fp16 / bf16 (or fp32) split-KV MLA decode (query [n_h,576], cache [N,576]); a float8_e4m3fn "
          "cache (holding C / cache_scale) with a float16 query",
          pybind11::arg("query"), pybind11::arg("cache"), pybind11::arg("num_splits") = 0,
          pybind11::arg("cache_scale") = 1.0);
    m.def("mla_decode_fused", &mla_decode_fused, "fp32 MLA decode (query [n_h,576], cache [N,576])",
          pybind11::arg("query"), pybind11::arg("cache"), pybind11::arg("num_splits") = 0);
    m.def("mla_decode_split_batched", &mla_decode_split_batched,
          "batched fp16 / bf16 MLA decode (query [B,n_h,576], packed cache [sum N,576], cu_seqlens [B+1] int32); "
          "a float8_e4m3fn cache (holding C / cache_scale) with a float16 query",
          pybind11::arg("query"), pybind11::arg("cache"), pybind11::arg("cu_seqlens"),
          pybind11::arg("num_splits") = 0, pybind11::arg("cache_scale") = 1.0);
    m.def("mla_decode_paged", &mla_decode_paged,
          "paged-KV fp16 / bf16 MLA decode (query [B,n_h,576], kv_cache [pages,page_size,576], "
          "block_table [B,max_pages] int32, cu_seqlens [B+1] int32); total_tokens=-1 reads cu_seqlens[B] "
          "(synchronising); a given total_tokens is not checked: one below cu_seqlens[B] silently "
          "truncates the trailing sequences",
          pybind11::arg("query"), pybind11::arg("kv_cache"), pybind11::arg("block_table"),
          pybind11::arg("cu_seqlens"), pybind11::arg("total_tokens") = -1, pybind11::arg("num_splits") = 0);
    m.def("mla_absorb_query", &mla_absorb_query,
          "Q* [B,n_h,576] = [q_nope W_UK[h], q_rope] (q_nope [B,n_h,128], q_rope [B,n_h,64], w_uk [n_h,128,512])",
          pybind11::arg("q_nope"), pybind11::arg("q_rope"), pybind11::arg("w_uk"));
    m.def("mla_project_output", &mla_project_output,
          "out [B,d_model] = concat_h(O*[:,h] W_UV[h]^T) W_O^T (o_star [B,n_h,512], w_uv [n_h,128,512], "
          "w_o [d_model,n_h*128])",
          pybind11::arg("o_star"), pybind11::arg("w_uv"), pybind11::arg("w_o"));
    m.attr("HEAD_DIM_C") = MLA_HEAD_DIM_V;
    m.attr("HEAD_DIM_ROPE") = MLA_HEAD_DIM_K - MLA_HEAD_DIM_V;
    m.attr("HEAD_DIM_K") = MLA_HEAD_DIM_K;
}
