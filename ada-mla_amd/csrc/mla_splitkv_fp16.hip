// fp16 split-KV MLA decode for gfx950:
//   O*_partial = sum_t exp2(s_t - m) C_N[t],  s_t = log2(e) * scale * (Q* . C[t])
// for one (chunk of tokens, tile of heads) per workgroup, written as fp32
// partials (O unnormalised, running max m, running sum l) that
// mla_combine.hip merges.
//
// Replaces mla_decode_splitk_mma_fp16 (reference
// csrc/mla_decode_splitk_fwd.cuh:559-892), with a different design:
//  * 256 threads = 4 wave64s. Each C block (kBT tokens x 576) is staged once
//    in LDS and read by both products.
//  * Q* C^T is computed as S^T = C Q*^T on 16x16x32 MFMAs: wave w owns a
//    16-token x 16-head tile over the full K = 576, with its Q* fragment
//    resident in VGPRs for the whole chunk (no K slicing, no cross-wave sum
//    of logits).
//  * Online softmax in fp32 (log2 domain), running max started at -inf; the
//    per-head block max crosses the 4 lane groups with shuffles and the token
//    tiles through a 128-byte LDS exchange.
//  * P C_N is computed as O^T = C_N^T P^T: wave w owns 128 output columns for
//    all heads of the tile, so the online-softmax rescale is one scalar per
//    lane; the C_N^T operand comes straight from the staged block with the
//    LDS transpose read (ds_read_b64_tr_b16).
//  * The next block is prefetched into VGPRs one iteration ahead and written
//    to the other LDS slot between the two barriers of each iteration, so a
//    slot is never overwritten while any wave still reads it.
#include "mla_device.hpp"
#include "mla_internal.hpp"

namespace mla {
namespace {

template <int HT>
struct F16Tile {
    static constexpr int kNHS = HT / 16;                    // 16-head sub-tiles
    static constexpr int kNTT = 4 / kNHS;                   // 16-token tiles per block
    static constexpr int kBT = 16 * kNTT;                   // tokens per block
    static constexpr int kRow = kDK + 8;                    // LDS row stride (halves)
    static constexpr int kRowChunks = kDK / 8;              // 16-byte chunks per row
    static constexpr int kStage = kBT * kRowChunks / 256;   // chunks per thread
    static constexpr int kPRow = kBT + 8;                   // P row stride (halves)
    static constexpr int kK2 = kBT / 32;                    // P C_N k-steps per block
    static_assert(kBT * kRowChunks % 256 == 0, "stage split");
    static_assert(kBT % 32 == 0, "P C_N k-step");
};

template <int HT, bool kTr>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256),
                          amdgpu_waves_per_eu(HT == 32 ? 2 : 1, HT == 32 ? 2 : 1)))
void splitkv_fp16_kernel(const _Float16 *__restrict__ q,
                         const _Float16 *__restrict__ c,
                         const int *__restrict__ cu_seqlens,
                         float *__restrict__ o_part,
                         float *__restrict__ m_part,
                         float *__restrict__ l_part,
                         int num_heads, int batch, int total_tokens, int chunk,
                         int n_head_tiles, int xcd_remap, float scale_log2)
{
    using T = F16Tile<HT>;
    __shared__ __attribute__((aligned(16))) _Float16 s_c[2 * T::kBT * T::kRow];
    __shared__ __attribute__((aligned(16))) _Float16 s_p[HT * T::kPRow];
    __shared__ float s_red[T::kNTT * HT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l16 = lane & 15;
    const int g = lane >> 4;

    // workgroup -> (chunk, head tile). With xcd_remap the head tiles of one
    // chunk get ids that are equal mod 8, i.e. land on the same XCD (blocks
    // are dispatched round-robin over the 8 XCDs), so C is pulled from HBM
    // into that XCD's L2 once and re-read from L2 by the other head tiles.
    int split, ht;
    {
        const int bid = blockIdx.x;
        if (xcd_remap) {
            const int x = bid & 7, li = bid >> 3;
            split = (li / n_head_tiles) * 8 + x;
            ht = li % n_head_tiles;
        } else {
            split = bid / n_head_tiles;
            ht = bid - split * n_head_tiles;
        }
    }
    const int lo = split * chunk;
    const int hi = min(lo + chunk, total_tokens);
    if (lo >= hi)
        return;

    const int hs1 = wave % T::kNHS;  // head sub-tile of this wave's logits
    const int tt = wave / T::kNHS;   // token tile of this wave's logits
    const int head0 = ht * HT;

    // First sequence containing token lo (largest b with cu[b] <= lo).
    int b = 0;
    const int nseq = cu_seqlens ? batch : 1;
    if (cu_seqlens) {
        int l = 0, r = batch;
        while (r - l > 1) {
            const int mid = (l + r) >> 1;
            if (cu_seqlens[mid] <= lo) l = mid; else r = mid;
        }
        b = l;
    }

    for (; b < nseq; ++b) {
        int seq_lo = 0, seq_hi = total_tokens;
        if (cu_seqlens) {
            seq_lo = min(max(cu_seqlens[b], 0), total_tokens);
            seq_hi = min(max(cu_seqlens[b + 1], seq_lo), total_tokens);
        }
        if (seq_lo >= hi)
            break;
        const int p_lo = max(seq_lo, lo);
        const int p_hi = min(seq_hi, hi);
        if (p_lo >= p_hi)
            continue;
        const int slot = split + b;
        const int nblk = (p_hi - p_lo + T::kBT - 1) / T::kBT;

        __syncthreads();  // LDS is reused from the previous piece

        // Q* fragment (B operand of S^T = C Q*^T): lane holds head
        // head0 + 16*hs1 + l16, dims 32*kk + 8*g .. +7.
        half8 qf[kDK / 32];
        {
            const _Float16 *qrow = q + ((size_t)b * num_heads + head0 + 16 * hs1 + l16) * kDK + 8 * g;
#pragma unroll
            for (int kk = 0; kk < kDK / 32; ++kk)
                qf[kk] = *(const half8 *)(qrow + 32 * kk);
        }

        half8 stage[T::kStage];
        auto load_stage = [&](int t0) {
#pragma unroll
            for (int s = 0; s < T::kStage; ++s) {
                const int ci = tid + 256 * s;
                const int tok = ci / T::kRowChunks;
                const int col = ci - tok * T::kRowChunks;
                const int gt = t0 + tok;
                if (gt < p_hi)
                    stage[s] = *(const half8 *)(c + (size_t)gt * kDK + col * 8);
                else
                    stage[s] = half8{0, 0, 0, 0, 0, 0, 0, 0};
            }
        };
        auto store_stage = [&](int which) {
            _Float16 *dst = s_c + which * T::kBT * T::kRow;
#pragma unroll
            for (int s = 0; s < T::kStage; ++s) {
                const int ci = tid + 256 * s;
                const int tok = ci / T::kRowChunks;
                const int col = ci - tok * T::kRowChunks;
                *(half8 *)(dst + tok * T::kRow + col * 8) = stage[s];
            }
        };

        load_stage(p_lo);
        store_stage(0);
        if (nblk > 1)
            load_stage(p_lo + T::kBT);

        float m_run[T::kNHS];
#pragma unroll
        for (int hs = 0; hs < T::kNHS; ++hs)
            m_run[hs] = -INFINITY;
        float l_run = 0.f;
        floatx4 o[T::kNHS][8];
#pragma unroll
        for (int hs = 0; hs < T::kNHS; ++hs)
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                o[hs][dt] = floatx4{0.f, 0.f, 0.f, 0.f};

        __syncthreads();

        for (int blk = 0; blk < nblk; ++blk) {
            const int cur = blk & 1;
            const int t0 = p_lo + blk * T::kBT;
            const _Float16 *cs = s_c + cur * T::kBT * T::kRow;

            // ---- S^T tile: tokens t0 + 16*tt + (0..15), heads 16*hs1 + (0..15)
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            {
                const _Float16 *arow = cs + (16 * tt + l16) * T::kRow + 8 * g;
#pragma unroll
                for (int kk = 0; kk < kDK / 32; ++kk)
                    acc = mfma16x16x32(*(const half8 *)(arow + 32 * kk), qf[kk], acc);
            }

            // ---- block max per head (log2 units), masked tail tokens = -inf
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = t0 + 16 * tt + 4 * g + i;
                sv[i] = tok < p_hi ? acc[i] * scale_log2 : -INFINITY;
                mx = fmaxf(mx, sv[i]);
            }
            mx = max_over_lane_groups(mx);
            if (g == 0)
                s_red[tt * HT + 16 * hs1 + l16] = mx;
            __syncthreads();

            // ---- new running max for every head sub-tile this wave touches
            float alpha[T::kNHS];
#pragma unroll
            for (int hs = 0; hs < T::kNHS; ++hs) {
                float mb = s_red[16 * hs + l16];
#pragma unroll
                for (int t2 = 1; t2 < T::kNTT; ++t2)
                    mb = fmaxf(mb, s_red[t2 * HT + 16 * hs + l16]);
                const float mn = fmaxf(m_run[hs], mb);
                alpha[hs] = fast_exp2(m_run[hs] - mn);
                m_run[hs] = mn;
            }
            {
                float mcur = m_run[0];
                float acur = alpha[0];
#pragma unroll
                for (int hs = 1; hs < T::kNHS; ++hs)
                    if (hs == hs1) { mcur = m_run[hs]; acur = alpha[hs]; }
                half4 ph;
                float psum = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = fast_exp2(sv[i] - mcur);
                    psum += p;
                    ph[i] = (_Float16)p;
                }
                l_run = l_run * acur + psum;
                *(half4 *)(s_p + (16 * hs1 + l16) * T::kPRow + 16 * tt + 4 * g) = ph;
            }

            if (blk + 1 < nblk)
                store_stage(cur ^ 1);
            if (blk + 2 < nblk)
                load_stage(t0 + 2 * T::kBT);
            __syncthreads();

            // ---- O^T[dims 128*wave .. +128][heads] += C_N^T P^T
#pragma unroll
            for (int hs = 0; hs < T::kNHS; ++hs)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
                    o[hs][dt] *= alpha[hs];
#pragma unroll
            for (int ks = 0; ks < T::kK2; ++ks) {
                half8 pb[T::kNHS];
#pragma unroll
                for (int hs = 0; hs < T::kNHS; ++hs)
                    pb[hs] = *(const half8 *)(s_p + (16 * hs + l16) * T::kPRow + 32 * ks + 8 * g);
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const int d0 = 128 * wave + 16 * dt;
                    half8 a;
                    if constexpr (kTr) {
                        const _Float16 *p = cs + (32 * ks + 8 * g + (l16 >> 2)) * T::kRow + d0 + 4 * (l16 & 3);
                        const half4 lo4 = lds_read_tr16(p);
                        const half4 hi4 = lds_read_tr16(p + 4 * T::kRow);
                        a = half8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                    } else {
                        const _Float16 *p = cs + (32 * ks + 8 * g) * T::kRow + d0 + l16;
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            a[j] = p[j * T::kRow];
                    }
#pragma unroll
                    for (int hs = 0; hs < T::kNHS; ++hs)
                        o[hs][dt] = mfma16x16x32(a, pb[hs], o[hs][dt]);
                }
            }
        }

        // ---- epilogue: partial (O, m, l) of this piece into its slot
        const float lsum = sum_over_lane_groups(l_run);
        if (g == 0)
            s_red[tt * HT + 16 * hs1 + l16] = lsum;  // s_red reads all ended before the last barrier
        __syncthreads();
        if (tid < HT) {
            float L = 0.f;
#pragma unroll
            for (int t2 = 0; t2 < T::kNTT; ++t2)
                L += s_red[t2 * HT + tid];
            float mv = m_run[0];
#pragma unroll
            for (int hs = 1; hs < T::kNHS; ++hs)
                if ((tid >> 4) == hs) mv = m_run[hs];
            m_part[(size_t)slot * num_heads + head0 + tid] = mv;
            l_part[(size_t)slot * num_heads + head0 + tid] = L;
        }
#pragma unroll
        for (int hs = 0; hs < T::kNHS; ++hs) {
            float *orow = o_part + ((size_t)slot * num_heads + head0 + 16 * hs + l16) * kDV + 128 * wave + 4 * g;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                *(floatx4 *)(orow + 16 * dt) = o[hs][dt];
        }
    }
}

template <int HT, bool kTr>
hipError_t launch_ht(const Problem &pb, const Plan &p, const Partials &w, hipStream_t s)
{
    const dim3 grid(p.n_chunks * p.n_head_tiles), block(256);
    hipLaunchKernelGGL((splitkv_fp16_kernel<HT, kTr>), grid, block, 0, s,
                       (const _Float16 *)pb.q, (const _Float16 *)pb.c, pb.cu_seqlens,
                       w.o, w.m, w.l, pb.num_heads, pb.batch, pb.total_tokens,
                       p.chunk, p.n_head_tiles, p.xcd_remap, pb.scale_log2);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_splitkv_fp16(const Problem &pb, const Plan &p, const Partials &w,
                               bool tr_load, hipStream_t s)
{
    if (p.n_chunks == 0)
        return hipSuccess;
    if (p.head_tile == 32)
        return tr_load ? launch_ht<32, true>(pb, p, w, s) : launch_ht<32, false>(pb, p, w, s);
    return tr_load ? launch_ht<16, true>(pb, p, w, s) : launch_ht<16, false>(pb, p, w, s);
}

}  // namespace mla
