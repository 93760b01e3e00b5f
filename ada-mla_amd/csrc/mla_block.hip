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
// These are weight-streaming GEMMs with M = B rows, all MFMA kernels of this
// file: the two per-head ones (W_UK, W_UV: 128 KB of weights per head) one
// workgroup per (head, column slice), with the rope columns of Q* copied by
// the absorption kernel; the output projection (one [B x n_h*128] x
// [n_h*128 x d_model] product, W_O streamed once from HBM) 32 output
// columns per workgroup. fp16 / bf16 inputs, fp32 accumulation. No
// reference code exists for this part (the reference stops at the decode
// kernel).
#include <cstdint>

#include "mla_device.hpp"
#include "mla_internal.hpp"
#include "mla_mi355x.h"
#include "mla_ring.hpp"

namespace mla {
namespace {

constexpr int kNope = 128;  // per-head query / value width before absorption
constexpr int kRope = 64;
constexpr int kLatent = 512;
constexpr int kDK = kLatent + kRope;

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

// Output projection, one workgroup (4 waves) per 32 output columns n0 .. +31:
//   out[b, n] = sum_k x[b, k] W_O[n, k]      (x = the value projection, [B x K])
// as its transpose D[n][b] on 16x16x32 MFMAs, with W_O rows as the A operand
// and x rows as the B operand, for rows b in groups of 32. Both stream
// through a kStages-deep LDS ring in chunks of kChunk K: 32 rows of W_O and
// 32 rows of x per stage, filled by direct global->LDS loads whose units are
// 512 contiguous bytes of two rows each, so HBM sees long runs of W_O (which
// is read once; x stays in L2 for every workgroup). Every load is one of
// these, so the waits are explicit counts that leave the later stages in
// flight. 16-byte chunk c of a 512-byte row sits at c ^ (row mod 16), which
// spreads the operand reads (16 rows, one chunk each) over the LDS banks.
// Wave w computes K-steps 2w and 2w + 1 of each chunk, and the four partial
// tiles are summed through LDS. Columns past N and rows past B read clamped
// addresses and are not stored.
constexpr int kChunk = 256;   // K per ring stage (512 bytes of a row)
constexpr int kStages = 4;    // ring stages (32 KB each: 16 KB of W_O, 16 KB of x)
constexpr int kUnitsPerWave = 8;  // load units per wave and stage (4 of W_O, 4 of x)

template <typename E>
__global__ __launch_bounds__(256) void out_proj_kernel(const E *__restrict__ x, const E *__restrict__ w,
                                                       E *__restrict__ out, int batch, int K, int N)
{
    using E8 = typename Vec<E>::v8;
    using E4 = typename Vec<E>::v4;
    constexpr int kRowHalves = kChunk;        // one row of a stage
    constexpr int kPart = 32 * kRowHalves;    // halves: the W_O part (x part follows)
    __shared__ __attribute__((aligned(1024))) E s_ring[kStages][2 * kPart];
    __shared__ floatx4 s_red[4][2][2][64];  // [wave][column tile][row tile][lane]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the load bases are scalars
    const int l16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 32;
    const int nchunk = K / kChunk;
    for (int b0 = 0; b0 < batch; b0 += 32) {
        // load unit u (0..15) of a part: rows 2u, 2u + 1 (lanes 0-31, 32-63);
        // lane: stored chunk position, fetching logical chunk
        // (lane & 31) ^ (row mod 16)
        auto unit = [&](const E *rows_base, int row_lim, int c, int st, int part, int u) {
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int r = 2 * u + (ln >> 5);
            const E *src = rows_base + (size_t)min(2 * u, row_lim) * K + (size_t)c * kChunk;
            // rows 2u and 2u + 1 are K apart; a row past row_lim re-reads row_lim
            const int dr = min(2 * u + 1, row_lim) - min(2 * u, row_lim);
            global_to_lds16(src, (ln >> 5) * dr * K * 2 + 16 * ((ln & 31) ^ (r & 15)),
                            &s_ring[st][part * kPart + 2 * u * kRowHalves]);
        };
        auto issue = [&](int c, int st) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                unit(w + (size_t)n0 * K, N - 1 - n0, c, st, 0, 4 * wave + i);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                unit(x + (size_t)b0 * K, batch - 1 - b0, c, st, 1, 4 * wave + i);
        };
        // operand of K-step kk of rows 16 t + l16 of a part of stage st
        auto op = [&](int st, int part, int t, int kk) -> E8 {
            const int row = 16 * t + l16;
            return *(const E8 *)(&s_ring[st][part * kPart + row * kRowHalves + 8 * ((4 * kk + g) ^ (row & 15))]);
        };
        floatx4 acc[2][2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int bt = 0; bt < 2; ++bt)
                acc[nt][bt] = floatx4{0.f, 0.f, 0.f, 0.f};
        __syncthreads();  // the ring and s_red are free (previous row group)
#pragma unroll
        for (int c = 0; c < kStages; ++c)
            if (c < nchunk)
                issue(c, c);
        for (int c = 0; c < nchunk; ++c) {
            const int st = c % kStages;
            // this wave's units of chunk c have landed (later stages may still
            // be in flight), then every wave's
            const int after = min(kStages - 1, nchunk - 1 - c);
            if (after >= 3)
                MLA_WAIT_VMCNT(3 * kUnitsPerWave);
            else if (after == 2)
                MLA_WAIT_VMCNT(2 * kUnitsPerWave);
            else if (after == 1)
                MLA_WAIT_VMCNT(kUnitsPerWave);
            else
                MLA_WAIT_VMCNT(0);
            lds_barrier();
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int kk = 2 * wave + k;
                const E8 a0 = op(st, 0, 0, kk), a1 = op(st, 0, 1, kk);
                const E8 x0 = op(st, 1, 0, kk), x1 = op(st, 1, 1, kk);
                acc[0][0] = mfma16x16x32(a0, x0, acc[0][0]);
                acc[0][1] = mfma16x16x32(a0, x1, acc[0][1]);
                acc[1][0] = mfma16x16x32(a1, x0, acc[1][0]);
                acc[1][1] = mfma16x16x32(a1, x1, acc[1][1]);
            }
            lds_barrier();  // every wave has read stage st
            if (c + kStages < nchunk)
                issue(c + kStages, st);
        }
        // lane (g, b) of tile (nt, bt) holds D[n0 + 16 nt + 4 g .. +3][b0 + 16 bt + b]
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int bt = 0; bt < 2; ++bt)
                s_red[wave][nt][bt][lane] = acc[nt][bt];
        __syncthreads();
        {
            const int nt = wave >> 1, bt = wave & 1;
            const floatx4 v = s_red[0][nt][bt][lane] + s_red[1][nt][bt][lane] + s_red[2][nt][bt][lane] +
                              s_red[3][nt][bt][lane];
            const int b = b0 + 16 * bt + l16;
            const int n = n0 + 16 * nt + 4 * g;
            if (b < batch) {
                E *o = out + (size_t)b * N + n;
                if (n + 3 < N && (N & 3) == 0) {
                    *(E4 *)o = E4{(E)v[0], (E)v[1], (E)v[2], (E)v[3]};
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (n + i < N)
                            o[i] = (E)v[i];
                }
            }
        }
    }
}

int absorb(bool bf16, const void *q_nope, const void *q_rope, const void *w_uk, void *q_star,
           int batch, int num_heads, void *stream)
{
    if (!q_nope || !q_rope || !w_uk || !q_star || batch < 1 || num_heads < 1 || num_heads > 4096 ||
        (int64_t)batch * num_heads * kDK > INT32_MAX)
        return MLA_STATUS_INVALID_VALUE;
    if (!aligned16(q_nope) || !aligned16(q_rope) || !aligned16(w_uk) || !aligned16(q_star))
        return MLA_STATUS_MISALIGNED;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (bf16)
        hipLaunchKernelGGL(absorb_kernel<__bf16>, dim3(num_heads * 4), dim3(256), 0, s,
                           static_cast<const __bf16 *>(q_nope), static_cast<const __bf16 *>(q_rope),
                           static_cast<const __bf16 *>(w_uk), static_cast<__bf16 *>(q_star), batch, num_heads);
    else
        hipLaunchKernelGGL(absorb_kernel<_Float16>, dim3(num_heads * 4), dim3(256), 0, s,
                           static_cast<const _Float16 *>(q_nope), static_cast<const _Float16 *>(q_rope),
                           static_cast<const _Float16 *>(w_uk), static_cast<_Float16 *>(q_star), batch, num_heads);
    const hipError_t e = hipPeekAtLastError();
    return e == hipSuccess ? MLA_STATUS_SUCCESS : record_hip_error(e);
}

int project(bool bf16, const void *o_star, const void *w_uv, const void *w_o, void *out,
            void *workspace, size_t workspace_bytes, int batch, int num_heads, int d_model, void *stream)
{
    if (!o_star || !w_uv || !w_o || !out || !workspace || batch < 1 || num_heads < 1 || num_heads > 4096 ||
        d_model < 1 || (int64_t)batch * num_heads * kLatent > INT32_MAX || (int64_t)batch * d_model > INT32_MAX)
        return MLA_STATUS_INVALID_VALUE;
    if (!aligned16(o_star) || !aligned16(w_uv) || !aligned16(w_o) || !aligned16(out) || !aligned16(workspace))
        return MLA_STATUS_MISALIGNED;
    if (workspace_bytes < mla_project_output_workspace_size(batch, num_heads))
        return MLA_STATUS_WORKSPACE_TOO_SMALL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int hv = num_heads * kNope;
    // o [B x n_h*128] (the workspace): o[b, h*128 + j] = O*[b, h, :] . W_UV[h][j][:]
    if (bf16)
        hipLaunchKernelGGL(value_proj_kernel<__bf16>, dim3(num_heads * 4), dim3(64), 0, s,
                           static_cast<const __bf16 *>(o_star), static_cast<const __bf16 *>(w_uv),
                           static_cast<__bf16 *>(workspace), batch, num_heads);
    else
        hipLaunchKernelGGL(value_proj_kernel<_Float16>, dim3(num_heads * 4), dim3(64), 0, s,
                           static_cast<const _Float16 *>(o_star), static_cast<const _Float16 *>(w_uv),
                           static_cast<_Float16 *>(workspace), batch, num_heads);
    // out [B x d_model] = o [B x n_h*128] W_O^T
    const dim3 grid((d_model + 31) / 32);
    if (bf16)
        hipLaunchKernelGGL(out_proj_kernel<__bf16>, grid, dim3(256), 0, s, static_cast<const __bf16 *>(workspace),
                           static_cast<const __bf16 *>(w_o), static_cast<__bf16 *>(out), batch, hv, d_model);
    else
        hipLaunchKernelGGL(out_proj_kernel<_Float16>, grid, dim3(256), 0, s, static_cast<const _Float16 *>(workspace),
                           static_cast<const _Float16 *>(w_o), static_cast<_Float16 *>(out), batch, hv, d_model);
    const hipError_t e = hipPeekAtLastError();
    return e == hipSuccess ? MLA_STATUS_SUCCESS : record_hip_error(e);
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
    return mla::absorb(false, q_nope, q_rope, w_uk, q_star, batch, num_heads, stream);
}

int mla_absorb_query_bf16(const void *q_nope, const void *q_rope, const void *w_uk, void *q_star, int batch,
                          int num_heads, void *stream)
{
    return mla::absorb(true, q_nope, q_rope, w_uk, q_star, batch, num_heads, stream);
}

int mla_project_output_fp16(const void *o_star, const void *w_uv, const void *w_o, void *out, void *workspace,
                            size_t workspace_bytes, int batch, int num_heads, int d_model, void *stream)
{
    return mla::project(false, o_star, w_uv, w_o, out, workspace, workspace_bytes, batch,
                        num_heads, d_model, stream);
}

int mla_project_output_bf16(const void *o_star, const void *w_uv, const void *w_o, void *out, void *workspace,
                            size_t workspace_bytes, int batch, int num_heads, int d_model, void *stream)
{
    return mla::project(true, o_star, w_uv, w_o, out, workspace, workspace_bytes, batch,
                        num_heads, d_model, stream);
}

}  // extern "C"
