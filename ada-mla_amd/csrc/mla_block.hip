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
#include <algorithm>
#include <cstdint>
#include <type_traits>

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

// Output projection:
//   out[b, n] = sum_k x[b, k] W_O[n, k]      (x = the value projection, [B x K], K = n_h * 128)
// as its transpose D[n][b] on 16x16x32 MFMAs, W_O rows the A operand and x
// rows the B operand. W_O (168 MB at n_h = 128, d_model 5120) is the one
// large operand and is streamed from HBM once.
//  * Work: a unit is 64 output columns (64 rows of W_O) x 32 rows of x over
//    all K, in kChunk-column chunks; the (unit, chunk) steps, units
//    outermost, are cut into equal contiguous ranges, one per workgroup of a
//    grid of at most one workgroup per CU (stream-K). Every CU thus streams
//    the same share of W_O whatever d_model / 64 is (160 column blocks of 32
//    on 256 CUs would leave 96 idle). A unit that one workgroup covers whole
//    is stored directly; the pieces of a unit split between workgroups (at
//    most a first and a last one per workgroup) are stored as fp32 partial
//    tiles that reduce_units_kernel adds in a fixed order. Plain stores and
//    loads: against nontemporal ones the call (value projection, W_O and the
//    reduce, cold weights) read 41.2-41.4 against 41.6 us at B = 32, d_model
//    5120, and 0.4-1.9% less at four other shapes. (Adding the pieces up in
//    the kernel instead, by the last workgroup to finish a piece of the unit
//    on agent-scope completion counters, measured slower: 40.3 us against
//    32.4 + 4.8 us for the two kernels, from the release / acquire cache
//    maintenance.)
//  * Within a workgroup the chunks run through one kStages-deep LDS ring
//    with no break at unit boundaries: 64 rows of W_O and 32 rows of x per
//    stage, filled by direct global->LDS loads of 512 contiguous bytes of two
//    rows each. Every load is one of these, so the waits are explicit counts
//    that leave the later stages in flight. 16-byte chunk c of a 512-byte row
//    sits at c ^ (row mod 16), which spreads the operand reads (16 rows, one
//    chunk each) over the LDS banks.
//  * Wave w owns the 16 columns 16w .. +15 of the unit for both 16-row tiles
//    of x over every K-step, so no sums cross waves. x (1 MB for B = 32 at
//    n_h = 128) is re-read from L2 by every workgroup, half a byte per byte
//    of W_O; measured, these x loads were the largest cost beside W_O itself.
//  * K is a multiple of 128: a last chunk of 128 columns re-reads each row's
//    last 16 valid bytes in place of the missing ones and skips its K-steps
//    past K. Columns past N and rows past B read clamped addresses and are
//    not stored.
constexpr int kChunk = 256;        // K per ring stage (512 bytes of a row)
constexpr int kStages = 3;         // ring stages (48 KB each: 32 KB of W_O, 16 KB of x)
constexpr int kCols = 64;          // output columns (W_O rows) per unit
constexpr int kUnitsPerWave = 12;  // load units per wave and stage (8 of W_O, 4 of x)
constexpr int kMaxGrid = 512;      // workgroups of the output projection (partial slots: 2 each)
constexpr int kPartTile = kCols * 32;  // floats of one partial tile [32 rows][64 columns]

// the (unit, chunk) steps [g P, min(T, (g + 1) P)) of workgroup g
struct OutProjGeom {
    int n_blocks;  // column blocks of kCols
    int chunks;    // K chunks per unit
    int steps;     // T = units x chunks
    int per_wg;    // P
    int grid;
};

template <typename E>
__global__ __launch_bounds__(256) void out_proj_kernel(const E *__restrict__ x, const E *__restrict__ w,
                                                       E *__restrict__ out, float *__restrict__ part,
                                                       int batch, int K, int N, OutProjGeom geo)
{
    using E8 = typename Vec<E>::v8;
    using E4 = typename Vec<E>::v4;
    constexpr int kRowHalves = kChunk;           // one row of a stage
    constexpr int kXOff = kCols * kRowHalves;     // halves: x rows follow the W_O rows
    constexpr int kStage = kXOff + 32 * kRowHalves;
    __shared__ __attribute__((aligned(1024))) E s_ring[kStages][kStage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the load bases are scalars
    const int l16 = lane & 15, g = lane >> 4;
    const int s_first = (int)blockIdx.x * geo.per_wg;
    const int n_steps = min(geo.steps - s_first, geo.per_wg);

    struct Step {
        int unit, c, n0, b0;
    };
    auto step_at = [&](int j) -> Step {
        Step st;
        const int gs = s_first + j;
        st.unit = __builtin_amdgcn_readfirstlane(gs / geo.chunks);
        st.c = __builtin_amdgcn_readfirstlane(gs - st.unit * geo.chunks);
        st.n0 = __builtin_amdgcn_readfirstlane((st.unit % geo.n_blocks) * kCols);
        st.b0 = __builtin_amdgcn_readfirstlane((st.unit / geo.n_blocks) * 32);
        return st;
    };
    // load unit u of a stage: rows 2u, 2u + 1 (lanes 0-31, 32-63) of the
    // W_O part (u < 32) or of the x part; lane: stored chunk position,
    // fetching logical chunk (lane & 31) ^ (row mod 16), at most the chunk's
    // last valid one
    auto unit = [&](const E *rows_base, int row_lim, int c, int st, int off, int u) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int r = 2 * u + (ln >> 5);
        const int valid = min(kChunk, K - c * kChunk) / 8;  // 16-byte chunks of this K-chunk (16 or 32)
        const E *src = rows_base + (size_t)min(2 * u, row_lim) * K + (size_t)c * kChunk;
        // rows 2u and 2u + 1 are K apart; a row past row_lim re-reads row_lim
        const int dr = min(2 * u + 1, row_lim) - min(2 * u, row_lim);
        global_to_lds16(src, (ln >> 5) * dr * K * 2 + 16 * min((ln & 31) ^ (r & 15), valid - 1),
                        &s_ring[st][off + 2 * u * kRowHalves]);
    };
    auto issue = [&](int j, int st) {
        const Step sp = step_at(j);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            unit(w + (size_t)sp.n0 * K, N - 1 - sp.n0, sp.c, st, 0, 8 * wave + i);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            unit(x + (size_t)sp.b0 * K, batch - 1 - sp.b0, sp.c, st, kXOff, 4 * wave + i);
    };
    // operand of K-step kk of row `row` of the part at `off` of stage st
    auto op = [&](int st, int off, int row, int kk) -> E8 {
        return *(const E8 *)(&s_ring[st][off + row * kRowHalves + 8 * ((4 * kk + g) ^ (row & 15))]);
    };
    floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
    bool first_piece = true;  // the unit in progress is this workgroup's first
    int piece_c0 = step_at(0).c;
#pragma unroll
    for (int j = 0; j < kStages; ++j)
        if (j < n_steps)
            issue(j, j);
    for (int j = 0; j < n_steps; ++j) {
        const int st = j % kStages;
        const Step sp = step_at(j);
        // this wave's units of chunk j have landed (later stages may still be
        // in flight; tile stores issued since are younger than them), then
        // every wave's
        const int after = min(kStages - 1, n_steps - 1 - j);
        if (after >= 2)
            MLA_WAIT_VMCNT(2 * kUnitsPerWave);
        else if (after == 1)
            MLA_WAIT_VMCNT(kUnitsPerWave);
        else
            MLA_WAIT_VMCNT(0);
        lds_barrier();
        auto ksteps = [&](auto n) {  // n K-steps of 32: 8, or 4 in a 128-column last chunk
#pragma unroll
            for (int kk = 0; kk < decltype(n)::value; ++kk) {
                const E8 a = op(st, 0, 16 * wave + l16, kk);
                const E8 x0 = op(st, kXOff, l16, kk), x1 = op(st, kXOff, 16 + l16, kk);
                acc[0] = mfma16x16x32(a, x0, acc[0]);
                acc[1] = mfma16x16x32(a, x1, acc[1]);
            }
        };
        if (K - sp.c * kChunk >= kChunk)
            ksteps(std::integral_constant<int, kChunk / 32>{});
        else
            ksteps(std::integral_constant<int, kChunk / 64>{});
        lds_barrier();  // every wave has read stage st
        if (j + kStages < n_steps)
            issue(j + kStages, st);
        const bool unit_end = sp.c == geo.chunks - 1;
        if (!unit_end && j != n_steps - 1)
            continue;
        // ---- end of this workgroup's piece of a unit: lane (g, b) of tile bt
        // holds D[n0 + 16 wave + 4 g .. +3][b0 + 16 bt + b]
        const bool whole = piece_c0 == 0 && unit_end;
        const int slot = 2 * (int)blockIdx.x + (first_piece ? 0 : 1);
#pragma unroll
        for (int bt = 0; bt < 2; ++bt) {
            const floatx4 v = acc[bt];
            acc[bt] = floatx4{0.f, 0.f, 0.f, 0.f};
            const int bl = 16 * bt + l16;        // row within the unit
            const int cl = 16 * wave + 4 * g;    // column within the unit
            const int b = sp.b0 + bl, n = sp.n0 + cl;
            if (!whole) {
                // every row and column of the tile, so the sums stay in bounds
                *(floatx4 *)(part + (size_t)slot * kPartTile + bl * kCols + cl) = v;
            } else if (b < batch) {
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
        first_piece = false;
        piece_c0 = 0;
    }

}

// out of the units split between workgroups: the sum of their pieces,
// workgroup by workgroup (one thread per 4 columns of a row)
template <typename E>
__global__ __launch_bounds__(256) void reduce_units_kernel(const float *__restrict__ part, E *__restrict__ out,
                                                           int batch, int N, OutProjGeom geo)
{
    using E4 = typename Vec<E>::v4;
    const int quads = (N + 3) / 4;
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= batch * quads)
        return;
    const int b = t / quads, n = 4 * (t - b * quads);
    const int u = (b / 32) * geo.n_blocks + n / kCols;
    const int g_lo = u * geo.chunks / geo.per_wg, g_hi = (u * geo.chunks + geo.chunks - 1) / geo.per_wg;
    if (g_lo == g_hi)  // one workgroup covered the unit and stored it
        return;
    // the pieces in batches of 8 whose loads are all in flight before the
    // sums (in workgroup order)
    floatx4 v = {0.f, 0.f, 0.f, 0.f};
    const float *tile0 = part + (b % 32) * kCols + n % kCols;
    for (int g0 = g_lo; g0 <= g_hi; g0 += 8) {
        floatx4 p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int g = g0 + i;
            const int slot = 2 * g + (u == g * geo.per_wg / geo.chunks ? 0 : 1);
            p[i] = g <= g_hi ? *(const floatx4 *)(tile0 + (size_t)slot * kPartTile)
                             : floatx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v += p[i];
    }
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

OutProjGeom out_proj_geom(int batch, int K, int N, int cu_count)
{
    OutProjGeom geo;
    geo.n_blocks = (N + kCols - 1) / kCols;
    geo.chunks = (K + kChunk - 1) / kChunk;
    geo.steps = geo.n_blocks * ((batch + 31) / 32) * geo.chunks;
    const int grid = std::max(1, std::min({cu_count, kMaxGrid, geo.steps}));
    geo.per_wg = (geo.steps + grid - 1) / grid;
    geo.grid = (geo.steps + geo.per_wg - 1) / geo.per_wg;
    return geo;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

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
    if (workspace_bytes < mla_project_output_workspace_size(batch, num_heads, d_model))
        return MLA_STATUS_WORKSPACE_TOO_SMALL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int hv = num_heads * kNope;
    // workspace: o [B x n_h*128] (16-bit), then the W_O kernel's partial tiles
    const OutProjGeom geo = out_proj_geom(batch, hv, d_model, current_cu_count());
    const bool split = geo.per_wg % geo.chunks != 0 && geo.grid > 1;  // some unit is shared
    char *ws = static_cast<char *>(workspace);
    float *part = reinterpret_cast<float *>(ws + align256((size_t)batch * hv * 2));
    const int quads = batch * ((d_model + 3) / 4);
    // o[b, h*128 + j] = O*[b, h, :] . W_UV[h][j][:], then
    // out [B x d_model] = o W_O^T
    if (bf16) {
        hipLaunchKernelGGL(value_proj_kernel<__bf16>, dim3(num_heads * 4), dim3(64), 0, s,
                           static_cast<const __bf16 *>(o_star), static_cast<const __bf16 *>(w_uv),
                           reinterpret_cast<__bf16 *>(ws), batch, num_heads);
        hipLaunchKernelGGL(out_proj_kernel<__bf16>, dim3(geo.grid), dim3(256), 0, s,
                           reinterpret_cast<const __bf16 *>(ws), static_cast<const __bf16 *>(w_o),
                           static_cast<__bf16 *>(out), part, batch, hv, d_model, geo);
        if (split)
            hipLaunchKernelGGL(reduce_units_kernel<__bf16>, dim3((quads + 255) / 256), dim3(256), 0, s, part,
                               static_cast<__bf16 *>(out), batch, d_model, geo);
    } else {
        hipLaunchKernelGGL(value_proj_kernel<_Float16>, dim3(num_heads * 4), dim3(64), 0, s,
                           static_cast<const _Float16 *>(o_star), static_cast<const _Float16 *>(w_uv),
                           reinterpret_cast<_Float16 *>(ws), batch, num_heads);
        hipLaunchKernelGGL(out_proj_kernel<_Float16>, dim3(geo.grid), dim3(256), 0, s,
                           reinterpret_cast<const _Float16 *>(ws), static_cast<const _Float16 *>(w_o),
                           static_cast<_Float16 *>(out), part, batch, hv, d_model, geo);
        if (split)
            hipLaunchKernelGGL(reduce_units_kernel<_Float16>, dim3((quads + 255) / 256), dim3(256), 0, s, part,
                               static_cast<_Float16 *>(out), batch, d_model, geo);
    }
    const hipError_t e = hipPeekAtLastError();
    return e == hipSuccess ? MLA_STATUS_SUCCESS : record_hip_error(e);
}

}  // namespace
}  // namespace mla

extern "C" {

size_t mla_project_output_workspace_size(int batch, int num_heads, int d_model)
{
    if (batch < 1 || num_heads < 1 || num_heads > 4096 || d_model < 1)
        return 0;
    // the value projection [B x n_h*128] (16-bit), then the output
    // projection's fp32 partial tiles (two per workgroup, at most kMaxGrid
    // workgroups on any device)
    const mla::OutProjGeom geo = mla::out_proj_geom(batch, num_heads * mla::kNope, d_model, mla::kMaxGrid);
    return mla::align256((size_t)batch * num_heads * mla::kNope * 2) + (size_t)2 * geo.grid * mla::kPartTile * 4;
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
