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
// These are weight-streaming GEMMs with M = B rows. The two per-head ones
// (W_UK, W_UV: 128 KB of weights per head) run as MFMA kernels here, one
// workgroup per (head, column slice), with the rope columns of Q* copied by
// the absorption kernel; the output projection (one [B x n_h*128] x
// [n_h*128 x d_model] GEMM) runs on rocBLAS. fp16 / bf16 inputs, fp32
// accumulation. No reference code exists for this part (the reference stops
// at the decode kernel).
#include <rocblas/rocblas.h>

#include <cstdint>

#include "mla_device.hpp"
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

// Absorption, one workgroup (4 waves) per (head h, 128-column slice cs):
//   Q*[b, h, 128 cs + n] = sum_k q_nope[b, h, k] W_UK[h][k][128 cs + n],
// computed as its transpose D[n][b] on 16x16x32 MFMAs: the W_UK slice
// (128 x 128) is staged in LDS, rows 256 bytes apart with 16-byte chunk c of
// row k at c ^ (k mod 16), and read as the A operand (n x k) with the LDS
// transpose read; q_nope rows are the B operand, read from global memory.
// Wave w owns columns 32 w .. +31 (two 16-column tiles) for all B rows.
// The slice cs = 0 also copies the 64 rope columns of each row.
template <typename E>
__global__ __launch_bounds__(256) void absorb_kernel(const E *__restrict__ q_nope, const E *__restrict__ q_rope,
                                                     const E *__restrict__ w_uk, E *__restrict__ q_star,
                                                     int batch, int num_heads)
{
    using E8 = typename Vec<E>::v8;
    using E4 = typename Vec<E>::v4;
    __shared__ __attribute__((aligned(16))) E s_w[kNope * 128];
    const int h = blockIdx.x >> 2, cs = blockIdx.x & 3;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    // B operands of the first two 16-row tiles, requested before the weights
    // so that both round trips overlap: lane (g, b) holds q_nope[b0 + b][h][32 kk + 8 g .. +7]
    auto load_q = [&](int b, int kk) -> E8 {
        return b < batch ? *(const E8 *)(q_nope + ((size_t)b * num_heads + h) * kNope + 32 * kk + 8 * g) : E8{};
    };
    E8 q0[2][kNope / 32];
#pragma unroll
    for (int bt = 0; bt < 2; ++bt)
#pragma unroll
        for (int kk = 0; kk < kNope / 32; ++kk)
            q0[bt][kk] = load_q(16 * bt + l16, kk);
    // stage W_UK[h][:, 128 cs .. +127]: 16-byte chunk c of row k (16 per row)
    const E *wsrc = w_uk + (size_t)h * kNope * kLatent + 128 * cs;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int lin = tid + 256 * i, k = lin >> 4, c = lin & 15;
        *(uint4 *)(s_w + k * 128 + 8 * (c ^ (k & 15))) = *(const uint4 *)(wsrc + (size_t)k * kLatent + 8 * c);
    }
    if (cs == 0) {  // the rope columns, 8 chunks of 16 bytes per row
        for (int i = tid; i < batch * 8; i += 256) {
            const int b = i >> 3, c = i & 7;
            *(uint4 *)(q_star + ((size_t)b * num_heads + h) * kDK + kLatent + 8 * c) =
                *(const uint4 *)(q_rope + ((size_t)b * num_heads + h) * kRope + 8 * c);
        }
    }
    __syncthreads();
    // A operands (n x k): lane (g, i) holds W[32 kk + 8 g .. +7][n0 + i], from
    // two transpose reads of 4 rows each
    E8 a[2][kNope / 32];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int n0 = 32 * wave + 16 * nt;
#pragma unroll
        for (int kk = 0; kk < kNope / 32; ++kk) {
            E4 part[2];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int row = 32 * kk + 8 * g + 4 * hf + (l16 >> 2);
                const int col = n0 + 4 * (l16 & 3);  // 4 columns, 8 bytes
                part[hf] = lds_read_tr16<E>(s_w + row * 128 + 8 * ((col >> 3) ^ (row & 15)) + (col & 7));
            }
            a[nt][kk] = E8{part[0][0], part[0][1], part[0][2], part[0][3], part[1][0], part[1][1], part[1][2], part[1][3]};
        }
    }
    for (int b0 = 0; b0 < batch; b0 += 16) {
        const int b = b0 + l16;
        floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
        E8 qv[kNope / 32];
#pragma unroll
        for (int kk = 0; kk < kNope / 32; ++kk)
            qv[kk] = b0 < 32 ? q0[b0 >> 4][kk] : load_q(b, kk);
#pragma unroll
        for (int kk = 0; kk < kNope / 32; ++kk) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                acc[nt] = mfma16x16x32(a[nt][kk], qv[kk], acc[nt]);
        }
        // lane (g, b) holds D[n0 + 4 g .. +3][b]
        if (b < batch) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int n = 128 * cs + 32 * wave + 16 * nt + 4 * g;
                const E4 v = {(E)acc[nt][0], (E)acc[nt][1], (E)acc[nt][2], (E)acc[nt][3]};
                *(E4 *)(q_star + ((size_t)b * num_heads + h) * kDK + n) = v;
            }
        }
    }
}

// Value up-projection, one wave per (head h, 32-row slice js of W_UV[h]):
//   o[b, h * 128 + j] = sum_k O*[b, h, k] W_UV[h][j][k],
// as its transpose D[j][b]: W_UV rows (k contiguous) are the A operand and
// O* rows the B operand, both read from global memory; the 16 K-steps' A
// operands and the B operands of the first 32 rows are loaded up front.
template <typename E>
__global__ __launch_bounds__(64) void value_proj_kernel(const E *__restrict__ o_star, const E *__restrict__ w_uv,
                                                        E *__restrict__ o, int batch, int num_heads)
{
    using E8 = typename Vec<E>::v8;
    using E4 = typename Vec<E>::v4;
    const int h = blockIdx.x >> 2, js = blockIdx.x & 3;
    const int lane = threadIdx.x, l16 = lane & 15, g = lane >> 4;
    auto load_o = [&](int b, int kk) -> E8 {
        return b < batch ? *(const E8 *)(o_star + ((size_t)b * num_heads + h) * kLatent + 32 * kk + 8 * g) : E8{};
    };
    // every load of the first two 16-row tiles is in flight at once
    E8 a[2][kLatent / 32], o0[2][kLatent / 32];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
        const E *wrow = w_uv + ((size_t)h * kNope + 32 * js + 16 * jt + l16) * kLatent + 8 * g;
#pragma unroll
        for (int kk = 0; kk < kLatent / 32; ++kk)
            a[jt][kk] = *(const E8 *)(wrow + 32 * kk);
    }
#pragma unroll
    for (int bt = 0; bt < 2; ++bt)
#pragma unroll
        for (int kk = 0; kk < kLatent / 32; ++kk)
            o0[bt][kk] = load_o(16 * bt + l16, kk);
    for (int b0 = 0; b0 < batch; b0 += 16) {
        const int b = b0 + l16;
        floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int kk = 0; kk < kLatent / 32; ++kk) {
            const E8 ov = b0 < 32 ? o0[b0 >> 4][kk] : load_o(b, kk);
#pragma unroll
            for (int jt = 0; jt < 2; ++jt)
                acc[jt] = mfma16x16x32(a[jt][kk], ov, acc[jt]);
        }
        // lane (g, b) holds D[j0 + 4 g .. +3][b]
        if (b < batch) {
#pragma unroll
            for (int jt = 0; jt < 2; ++jt) {
                const int j = 32 * js + 16 * jt + 4 * g;
                const E4 v = {(E)acc[jt][0], (E)acc[jt][1], (E)acc[jt][2], (E)acc[jt][3]};
                *(E4 *)(o + (size_t)b * num_heads * kNope + (size_t)h * kNope + j) = v;
            }
        }
    }
}

int absorb(rocblas_datatype dt, const void *q_nope, const void *q_rope, const void *w_uk, void *q_star,
           int batch, int num_heads, void *stream)
{
    if (!q_nope || !q_rope || !w_uk || !q_star || batch < 1 || num_heads < 1 || num_heads > 4096 ||
        (int64_t)batch * num_heads * kDK > INT32_MAX)
        return MLA_STATUS_INVALID_VALUE;
    if (!aligned16(q_nope) || !aligned16(q_rope) || !aligned16(w_uk) || !aligned16(q_star))
        return MLA_STATUS_MISALIGNED;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dt == rocblas_datatype_bf16_r)
        hipLaunchKernelGGL(absorb_kernel<__bf16>, dim3(num_heads * 4), dim3(256), 0, s,
                           static_cast<const __bf16 *>(q_nope), static_cast<const __bf16 *>(q_rope),
                           static_cast<const __bf16 *>(w_uk), static_cast<__bf16 *>(q_star), batch, num_heads);
    else
        hipLaunchKernelGGL(absorb_kernel<_Float16>, dim3(num_heads * 4), dim3(256), 0, s,
                           static_cast<const _Float16 *>(q_nope), static_cast<const _Float16 *>(q_rope),
                           static_cast<const _Float16 *>(w_uk), static_cast<_Float16 *>(q_star), batch, num_heads);
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
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (rocblas_set_stream(h, s) != rocblas_status_success)
        return MLA_STATUS_HIP_ERROR;
    const float one = 1.0f, zero = 0.0f;
    const int hv = num_heads * kNope;
    // o [B x n_h*128] (the workspace): o[b, h*128 + j] = O*[b, h, :] . W_UV[h][j][:]
    if (dt == rocblas_datatype_bf16_r)
        hipLaunchKernelGGL(value_proj_kernel<__bf16>, dim3(num_heads * 4), dim3(64), 0, s,
                           static_cast<const __bf16 *>(o_star), static_cast<const __bf16 *>(w_uv),
                           static_cast<__bf16 *>(workspace), batch, num_heads);
    else
        hipLaunchKernelGGL(value_proj_kernel<_Float16>, dim3(num_heads * 4), dim3(64), 0, s,
                           static_cast<const _Float16 *>(o_star), static_cast<const _Float16 *>(w_uv),
                           static_cast<_Float16 *>(workspace), batch, num_heads);
    if (hipGetLastError() != hipSuccess)
        return MLA_STATUS_HIP_ERROR;
    // out [B x d_model] = o [B x n_h*128] x W_O^T; column-major: out^T = W_O o^T.
    const rocblas_status r = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, d_model, batch, hv, &one,
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
