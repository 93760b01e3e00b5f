// The projections on either side of the absorbed MLA decode, completing the
// decode step of an MLA attention block (reference README.md:76-85, 104-110):
//
//   before:  Q*[b, h, :512] = q_nope[b, h, :] W_UK[h]        (absorbed key up-projection)
//            Q*[b, h, 512:] = q_rope[b, h, :]
//   decode:  O*[b, h, :]    = softmax(Q* C^T / sqrt(192)) C[:, :512]   (mla_decode_*)
//   after:   o[b, h, :]     = O*[b, h, :] W_UV[h]^T           (value up-projection)
//            out[b, :]      = o[b, :, :] (flattened) W_O^T    (output projection)
//
// with W_UK, W_UV [n_h][128][512] (the per-head key / value halves of the
// latent up-projection, torch Linear layout: out_features x in_features) and
// W_O [d_model][n_h * 128]. The softmax scale stays in the decode kernel, so
// Q* carries no scale. Batched over the B decode tokens.
//
// These are plain weight-streaming GEMMs (M = B rows): they run on rocBLAS
// (strided-batched over heads, fp16 / bf16 inputs, fp32 accumulation), laid
// out so that the absorbed query lands directly in Q*'s first 512 columns;
// the rope columns are copied by a small kernel. No reference code exists
// for this part (the reference stops at the decode kernel).
#include <rocblas/rocblas.h>

#include <cstdint>

#include "mla_mi355x.h"

namespace mla {
namespace {

constexpr int kNope = 128;  // per-head query / value width before absorption
constexpr int kRope = 64;
constexpr int kLatent = 512;
constexpr int kDK = kLatent + kRope;

constexpr int kMaxDevices = 64;

// One rocBLAS handle per (host thread, device), created on first use and kept
// for the life of the thread (rocBLAS allocates its own device workspace when
// a handle is created).
rocblas_handle handle_for_current_device(int *status)
{
    thread_local rocblas_handle handles[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *status = MLA_STATUS_HIP_ERROR;
        return nullptr;
    }
    if (!handles[dev] && rocblas_create_handle(&handles[dev]) != rocblas_status_success) {
        handles[dev] = nullptr;
        *status = MLA_STATUS_HIP_ERROR;
        return nullptr;
    }
    *status = MLA_STATUS_SUCCESS;
    return handles[dev];
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// q_rope [rows][64] -> q_star [rows][576] columns 512..575, 16 bytes per thread.
__global__ void copy_rope(const uint4 *__restrict__ rope, uint4 *__restrict__ q_star, int rows)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;  // (row, 16-byte chunk)
    if (i >= rows * 8)
        return;
    const int row = i >> 3, ch = i & 7;
    q_star[(size_t)row * (kDK * 2 / 16) + kLatent * 2 / 16 + ch] = rope[i];
}

int absorb(rocblas_datatype dt, const void *q_nope, const void *q_rope, const void *w_uk, void *q_star,
           int batch, int num_heads, void *stream)
{
    if (!q_nope || !q_rope || !w_uk || !q_star || batch < 1 || num_heads < 1 || num_heads > 4096 ||
        (int64_t)batch * num_heads * kDK > INT32_MAX)
        return MLA_STATUS_INVALID_VALUE;
    if (!aligned16(q_nope) || !aligned16(q_rope) || !aligned16(w_uk) || !aligned16(q_star))
        return MLA_STATUS_MISALIGNED;
    int st;
    rocblas_handle h = handle_for_current_device(&st);
    if (!h)
        return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (rocblas_set_stream(h, s) != rocblas_status_success)
        return MLA_STATUS_HIP_ERROR;
    // Row-major Q*_h [B x 512] (row stride n_h*576) = q_nope_h [B x 128]
    // (row stride n_h*128) x W_UK[h] [128 x 512]; in rocBLAS's column-major
    // terms: Q*_h^T = W_UK[h]^T q_nope_h^T, one GEMM per head.
    const float one = 1.0f, zero = 0.0f;
    const rocblas_status r = rocblas_gemm_strided_batched_ex(
        h, rocblas_operation_none, rocblas_operation_none, kLatent, batch, kNope, &one,
        w_uk, dt, kLatent, (rocblas_stride)kNope * kLatent,
        q_nope, dt, num_heads * kNope, (rocblas_stride)kNope,
        &zero, q_star, dt, num_heads * kDK, (rocblas_stride)kDK,
        q_star, dt, num_heads * kDK, (rocblas_stride)kDK,
        num_heads, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (r != rocblas_status_success)
        return MLA_STATUS_HIP_ERROR;
    const int rows = batch * num_heads;
    hipLaunchKernelGGL(copy_rope, dim3((rows * 8 + 255) / 256), dim3(256), 0, s,
                       static_cast<const uint4 *>(q_rope), static_cast<uint4 *>(q_star), rows);
    return hipGetLastError() == hipSuccess ? MLA_STATUS_SUCCESS : MLA_STATUS_HIP_ERROR;
}

int project(rocblas_datatype dt, const void *o_star, const void *w_uv, const void *w_o, void *out,
            void *workspace, size_t workspace_bytes, int batch, int num_heads, int d_model, void *stream)
{
    if (!o_star || !w_uv || !w_o || !out || !workspace || batch < 1 || num_heads < 1 || num_heads > 4096 ||
        d_model < 1 || (int64_t)batch * num_heads * kLatent > INT32_MAX || (int64_t)batch * d_model > INT32_MAX)
        return MLA_STATUS_INVALID_VALUE;
    if (!aligned16(o_star) || !aligned16(w_uv) || !aligned16(w_o) || !aligned16(out) || !aligned16(workspace))
        return MLA_STATUS_MISALIGNED;
    if (workspace_bytes < mla_project_output_workspace_size(batch, num_heads))
        return MLA_STATUS_WORKSPACE_TOO_SMALL;
    int st;
    rocblas_handle h = handle_for_current_device(&st);
    if (!h)
        return st;
    if (rocblas_set_stream(h, static_cast<hipStream_t>(stream)) != rocblas_status_success)
        return MLA_STATUS_HIP_ERROR;
    const float one = 1.0f, zero = 0.0f;
    const int hv = num_heads * kNope;
    // o_h [B x 128] (row stride n_h*128, in the workspace) = O*_h [B x 512]
    // (row stride n_h*512) x W_UV[h]^T; column-major: o_h^T = W_UV[h] O*_h^T.
    rocblas_status r = rocblas_gemm_strided_batched_ex(
        h, rocblas_operation_transpose, rocblas_operation_none, kNope, batch, kLatent, &one,
        w_uv, dt, kLatent, (rocblas_stride)kNope * kLatent,
        o_star, dt, num_heads * kLatent, (rocblas_stride)kLatent,
        &zero, workspace, dt, hv, (rocblas_stride)kNope,
        workspace, dt, hv, (rocblas_stride)kNope,
        num_heads, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (r != rocblas_status_success)
        return MLA_STATUS_HIP_ERROR;
    // out [B x d_model] = o [B x n_h*128] x W_O^T; column-major: out^T = W_O o^T.
    r = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, d_model, batch, hv, &one,
                        w_o, dt, hv, workspace, dt, hv, &zero, out, dt, d_model, out, dt, d_model,
                        rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    return r == rocblas_status_success ? MLA_STATUS_SUCCESS : MLA_STATUS_HIP_ERROR;
}

}  // namespace
}  // namespace mla

extern "C" {

size_t mla_project_output_workspace_size(int batch, int num_heads)
{
    if (batch < 1 || num_heads < 1 || num_heads > 4096)
        return 0;
    return ((size_t)batch * num_heads * mla::kNope * 2 + 255) / 256 * 256;
}

int mla_absorb_query_fp16(const void *q_nope, const void *q_rope, const void *w_uk, void *q_star, int batch,
                          int num_heads, void *stream)
{
    return mla::absorb(rocblas_datatype_f16_r, q_nope, q_rope, w_uk, q_star, batch, num_heads, stream);
}

int mla_absorb_query_bf16(const void *q_nope, const void *q_rope, const void *w_uk, void *q_star, int batch,
                          int num_heads, void *stream)
{
    return mla::absorb(rocblas_datatype_bf16_r, q_nope, q_rope, w_uk, q_star, batch, num_heads, stream);
}

int mla_project_output_fp16(const void *o_star, const void *w_uv, const void *w_o, void *out, void *workspace,
                            size_t workspace_bytes, int batch, int num_heads, int d_model, void *stream)
{
    return mla::project(rocblas_datatype_f16_r, o_star, w_uv, w_o, out, workspace, workspace_bytes, batch,
                        num_heads, d_model, stream);
}

int mla_project_output_bf16(const void *o_star, const void *w_uv, const void *w_o, void *out, void *workspace,
                            size_t workspace_bytes, int batch, int num_heads, int d_model, void *stream)
{
    return mla::project(rocblas_datatype_bf16_r, o_star, w_uv, w_o, out, workspace, workspace_bytes, batch,
                        num_heads, d_model, stream);
}

}  // extern "C"
