// fp32 split-KV MLA decode for gfx950 (the --fp32 path): same math and the
// same partial tile layout as the fp16 kernel, with O kept unnormalised in
// fp32, on fp32 MFMAs (16x16x4f32) so that products and sums keep fp32
// precision end to end.
//
// Replaces mla_decode_fused (reference csrc/mla_decode_fused_fwd.cuh:50-352,
// launcher csrc/mla_decode_fused_fwd_sm89.cu:6-60), which ran one CTA per 16
// heads over the whole sequence (8 CTAs at 128 heads). Here the sequence is
// split so the grid fills the GPU, and the splits are merged by
// mla_combine.hip.
//
// Workgroup = 8 wave64s (two per SIMD), 16 or 32 heads (one or two 16-head
// sub-tiles carried by every wave), blocks of 16 tokens, in two roles
// pipelined one block apart: at step t the S waves form the logits and the
// softmax of block t while the O waves add block t - 1 into O, so one wave's
// softmax and LDS traffic overlap the other's MFMAs on each SIMD. The roles
// run separate loops with the same two barriers per step.
//  * S waves 0..3: S^T = C Q*^T, wave w owning K-quarter [144w, 144w + 144)
//    of each 16x16 tile (its Q* slices stay in VGPRs); the four partial tiles
//    are summed through LDS (barrier X), and every S wave of a sub-tile
//    redoes its (tiny) softmax, so all of them hold the running max and sum;
//    one publishes P and the rescale factor of each head for the O waves.
//    Each lane reads 4 consecutive K of both operands with one 16-byte LDS
//    read and feeds them to 4 MFMAs per sub-tile (the same K permutation on A
//    and B).
//  * O waves 4..7: O^T = C_N^T P^T, wave 4 + w owning 128 output columns,
//    read from LDS as 16-byte runs: MFMA tile t (0..3) of half h takes as its
//    row i the value dim 128w + 64h + 4i + t, so one ds_read_b128 of dims
//    128w + 64h + 4i .. +3 feeds four MFMAs and the 16 lanes of a token row
//    read 256 contiguous bytes. The store undoes the permutation: lane
//    (head j, g) of the four tiles holds the 16 dims of natural tile
//    8w + 4h + g. An O wave runs one of its block's four token quads (two at
//    32 heads) before barrier X and the rest after it, so that its MFMAs fill
//    the S wave's softmax on the same SIMD.
//  * C blocks go HBM -> LDS by the direct global->LDS load (36 loads of 1 KB
//    per block: 20 issued by the O waves before their MFMAs, 16 by the S
//    waves after their softmax) into a 4-slot ring, two blocks ahead of the
//    S waves; Q* comes through ring slots 2 (and 3) the same way at the
//    start of a piece. Rows are 2304 bytes with 16-byte chunk c of row r at
//    c ^ (r mod 16), so the S waves' row reads (16 rows, one chunk) and the
//    O waves' token-row reads (16 chunks of one row) both touch 16 distinct
//    chunk positions of a 256-byte bank period.
#include <type_traits>

#include "mla_device.hpp"
#include "mla_internal.hpp"
#include "mla_ring.hpp"

namespace mla {

#ifdef MLA_TIMELINE
// Timeline build only (see mla_splitkv_fp16.hip): per workgroup of the fp32
// kernel, wave 0 (an S wave) records s_memrealtime at entry (slot 0), at the
// first step (1), at the end of the step loop (2) and after its stores
// complete (3), the block count (11), and s_memtime sums over the steps: to
// barrier X (6), from X to the wait before barrier Y (7), that wait and Y
// (8), and its own work before X (4) and after it (5); wave 4 (an O wave)
// records its own work before X (9) and after it (10).
constexpr int kTimelineWorkgroupsF32 = 8192;
__device__ unsigned long long mla_timeline_stamps_f32[kTimelineWorkgroupsF32 * 16];
#define MLA_STAMP32W(w, e, v)                                                              \
    do {                                                                                   \
        if (wave == (w) && lane == 0 && blockIdx.x < kTimelineWorkgroupsF32)               \
            mla_timeline_stamps_f32[blockIdx.x * 16 + (e)] = (unsigned long long)(v);      \
    } while (0)
#define MLA_STAMP32(e, v) MLA_STAMP32W(0, e, v)
#define MLA_MT32() __builtin_amdgcn_s_memtime()
#else
#define MLA_STAMP32(e, v) \
    do {                  \
    } while (0)
#define MLA_STAMP32W(w, e, v) \
    do {                      \
    } while (0)
#endif

namespace {

constexpr int kBT = 16;                  // tokens per block
constexpr int kRing = 4;                 // C ring slots
constexpr int kRowChunks = kDK / 4;      // 16-byte chunks per row (144)
constexpr int kSlot = kBT * kDK;         // floats per ring slot (36 KB)
constexpr int kLoads = kSlot * 4 / 1024; // 1 KB direct loads per block (36)
// O wave 4 + w issues units w, w + 4, ... (kLoadsO of them) before its first
// MFMAs of a step, S wave w units 4 kLoadsO + w, + 4, ... (kLoadsS) after its
// softmax: such a load holds its wave until it is accepted, so each role
// issues its share where it has slack
constexpr int kLoadsO = 5;
constexpr int kLoadsS = 4;
static_assert(4 * (kLoadsO + kLoadsS) == kLoads, "load split");
constexpr int kWaves = 8;
constexpr int kKQ = kDK / 4;             // K per S wave (144)
// The small tiles exchanged through LDS at every step -- the partial S^T
// tiles [wave][head][token] and P [head][token] -- have rows of 16 floats,
// four 16-byte chunks, chunk k of row r stored at k ^ ((r >> 1) & 3). The
// 16-byte accesses of lanes (row j, chunk g) are then free of bank
// conflicts (measured on gfx950 with SQ_LDS_BANK_CONFLICT in probe kernels;
// rows of 20 floats conflicted on the reads, 0.33 of LDS-active cycles).
// P is stored quad-transposed: token 4 ks + g of head j is element ks of
// chunk g of row j, so lane (j, g) of an O wave reads its tokens g, g + 4,
// g + 8, g + 12 as one 16-byte chunk.
constexpr int kTRow = 16;
__device__ __forceinline__ int tile_at(int row, int chunk)
{
    return row * kTRow + 4 * (chunk ^ ((row >> 1) & 3));
}
static_assert(kRowChunks % 16 == 0, "the row swizzle stays within a row");
static_assert(kLoads == 36, "block loads");

// HT: heads per workgroup (16 or 32), as HT / 16 sub-tiles of 16 heads that
// every wave carries side by side: the S waves' C rows and the O waves' C_N
// columns are read from LDS once for all of them, so a 32-head workgroup
// fills each C block once for twice the heads.
template <int HT>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kWaves, 64 * kWaves), amdgpu_waves_per_eu(2, 2)))
void splitkv_fp32_kernel(const float *__restrict__ q,
                         const float *__restrict__ c,
                         const int *__restrict__ cu_seqlens,
                         float *__restrict__ o_part,
                         float *__restrict__ m_part,
                         float *__restrict__ l_part,
                         int num_heads, int batch, int total_tokens, int chunk,
                         int n_head_tiles, int xcd_remap, float scale_log2)
{
    constexpr int kNS = HT / 16;          // 16-head sub-tiles
    // O waves' token quads before barrier X (the rest after it, beside the
    // S waves' softmax). A SIMD's S and O waves share one MFMA pipe (one
    // fp32 16x16x4 per 32 cycles), so quads moved before X only lengthen that
    // phase; after X they hide the softmax. 32-head tiles run all four after
    // X; 16-head tiles measure the same with one quad before it.
    constexpr int kQuadsA = kNS == 1 ? 1 : 0;
    __shared__ __attribute__((aligned(1024))) float s_c[kRing * kSlot];
    __shared__ __attribute__((aligned(16))) float s_s[4 * HT * kTRow];
    __shared__ __attribute__((aligned(16))) float s_p[2 * HT * kTRow];
    __shared__ float s_alpha[2 * HT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool s_role = wave < 4;
    const int w4 = wave & 3;  // K quarter (S waves) or 128-column group (O waves)
    // S waves: the sub-tile whose softmax this wave runs (S waves w4 < kNS
    // publish its P and rescale factors and store its m and l)
    const int my_sh = w4 % kNS;
    const int l16 = lane & 15;
    const int g = lane >> 4;
    MLA_STAMP32(0, __builtin_amdgcn_s_memrealtime());
#ifdef MLA_TIMELINE
    unsigned long long ph_a = 0, ph_b = 0, ph_o = 0, tm = 0, wk_a = 0, wk_b = 0;
#endif

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
    if ((long long)split * chunk >= total_tokens)  // a padding workgroup of the grid
        return;
    const int lo = split * chunk;
    const int hi = min(lo + chunk, total_tokens);
    const int head0 = ht * HT;

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

    // LDS float offset of (row, logical 16-byte chunk) in a slot
    auto slot_at = [](int row, int ch) { return row * kDK + 4 * (ch ^ (row & 15)); };

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
        const int nblk = (p_hi - p_lo + kBT - 1) / kBT;

        // the ring and the P / alpha buffers of a previous piece are free
        __syncthreads();

        // block j's direct loads of this wave into ring slot j % kRing: unit
        // u covers the slot's physical chunks [64u, 64u + 64); lane i's chunk
        // p = 64u + i is row p / 144, stored chunk p % 144, i.e. logical
        // chunk (p % 144) ^ (row mod 16). Rows past the piece repeat its last
        // token (their logits are masked).
        // 16 rows of 576 floats from base (rows past `last` repeat row
        // `last`) into the ring slot at dst
        auto issue_rows = [&](const float *base, int last, const float *dst) {
#pragma unroll
            for (int k = 0; k < (s_role ? kLoadsS : kLoadsO); ++k) {
                const int u = (s_role ? 4 * kLoadsO : 0) + w4 + 4 * k;
                const int pch = 64 * u + lane;
                const int row = pch / kRowChunks;
                const int sch = pch - row * kRowChunks;
                const int lch = sch ^ (row & 15);
                const int src_row = min(row, last);
                global_to_lds16(base, (src_row * kRowChunks + lch) * 16, dst + 256 * u);
            }
        };
        auto issue_block = [&](int j) {
            const int t0 = p_lo + j * kBT;
            issue_rows(c + (size_t)t0 * kDK, p_hi - 1 - t0, s_c + (j % kRing) * kSlot);
        };

        // Prologue: Q* of the head tile (16 heads per sub-tile, swizzled like
        // C rows) into ring slots 2 .. 2 + kNS - 1, blocks 0 and 1 into slots
        // 0 and 1, all by direct loads; the block loop starts once Q* and
        // block 0 have landed and the S waves hold Q* in registers. Q* does
        // not pass through the compiler's own loads: it would count them,
        // and not the direct loads issued after them, and then wait for them
        // inside the block loop, where its vmcnt waits would drain the ring
        // loads of block t + 2 at every step.
#pragma unroll
        for (int sh = 0; sh < kNS; ++sh)
            issue_rows(q + ((size_t)b * num_heads + head0 + 16 * sh) * kDK, 15, s_c + (2 + sh) * kSlot);
        issue_block(0);
        if (nblk > 1) {
            issue_block(1);
            if (s_role) MLA_WAIT_VMCNT(kLoadsS); else MLA_WAIT_VMCNT(kLoadsO);
        } else {
            MLA_WAIT_VMCNT(0);
        }
        __syncthreads();

        // The two roles run separate loops with the same barriers (two per
        // step), so that the S waves' Q* and the O waves' accumulators share
        // registers.
        if (s_role) {
            // Q* slices, head head0 + 16 sh + l16, dims kKQ*w4 + 16*kq + 4*g .. +3
            floatx4 qf[kNS][kKQ / 16];
#pragma unroll
            for (int sh = 0; sh < kNS; ++sh) {
                const float *qs = s_c + (2 + sh) * kSlot;
#pragma unroll
                for (int kq = 0; kq < kKQ / 16; ++kq)
                    qf[sh][kq] = *(const floatx4 *)(qs + slot_at(l16, 36 * w4 + 4 * kq + g));
            }
            __syncthreads();  // Q* read: slots 2 .. take blocks 2 .. from step 0 on
            MLA_STAMP32(1, __builtin_amdgcn_s_memrealtime());
            MLA_STAMP32(11, nblk);

            float m_run = -INFINITY, l_run = 0.f;  // sub-tile my_sh
            for (int t = 0; t <= nblk; ++t) {
#ifdef MLA_TIMELINE
                tm = MLA_MT32();
#endif
                if (t < nblk) {
                    // ---- partial S^T of block t over this wave's K-quarter
                    const float *cs = s_c + (t % kRing) * kSlot;
                    floatx4 acc[kNS];
#pragma unroll
                    for (int sh = 0; sh < kNS; ++sh)
                        acc[sh] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kq = 0; kq < kKQ / 16; ++kq) {
                        const floatx4 a = *(const floatx4 *)(cs + slot_at(l16, 36 * w4 + 4 * kq + g));
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                            for (int sh = 0; sh < kNS; ++sh)
                                acc[sh] = mfma16x16x4f32(a[jj], qf[sh][kq][jj], acc[sh]);
                    }
#pragma unroll
                    for (int sh = 0; sh < kNS; ++sh)
                        *(floatx4 *)(s_s + tile_at(w4 * HT + 16 * sh + l16, g)) = acc[sh];
                }
#ifdef MLA_TIMELINE
                wk_a += MLA_MT32() - tm;
#endif
                __syncthreads();  // barrier X: the four partial S^T tiles are in LDS
#ifdef MLA_TIMELINE
                { const unsigned long long t2 = MLA_MT32(); ph_a += t2 - tm; tm = t2; }
#endif
                if (t < nblk) {
                    // ---- full tile and softmax of sub-tile my_sh (every S
                    // wave of the sub-tile, identical results)
                    const int t0 = p_lo + t * kBT;
                    const float *sp = s_s + tile_at(16 * my_sh + l16, g);  // (the swizzle repeats every 16 rows)
                    const floatx4 sdot = ((*(const floatx4 *)sp + *(const floatx4 *)(sp + HT * kTRow)) +
                                          *(const floatx4 *)(sp + 2 * HT * kTRow)) +
                                         *(const floatx4 *)(sp + 3 * HT * kTRow);
                    float sv[4];
                    float mx = -INFINITY;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        sv[i] = (t0 + 4 * g + i) < p_hi ? sdot[i] * scale_log2 : -INFINITY;
                        mx = fmaxf(mx, sv[i]);
                    }
                    mx = max_over_lane_groups(mx);
                    const float mn = fmaxf(m_run, mx);
                    const float alpha = fast_exp2(m_run - mn);
                    m_run = mn;
                    floatx4 pv;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        pv[i] = fast_exp2(sv[i] - mn);
                    l_run = l_run * alpha + ((pv[0] + pv[1]) + (pv[2] + pv[3]));
                    if (w4 < kNS) {
                        // token 4g + i is element g of chunk i (quad-transposed)
                        float *pw = s_p + (t & 1) * HT * kTRow;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            pw[tile_at(16 * my_sh + l16, i) + g] = pv[i];
                        if (g == 0)
                            s_alpha[(t & 1) * HT + 16 * my_sh + l16] = alpha;
                    }
                }
                // the S waves' share of block t + 2; block t + 1 landed before
                // the barrier (block t + 2's loads stay in flight)
                if (t + 2 < nblk) {
                    issue_block(t + 2);
                    MLA_WAIT_VMCNT(kLoadsS);
                } else {
                    MLA_WAIT_VMCNT(0);
                }
#ifdef MLA_TIMELINE
                { const unsigned long long t2 = MLA_MT32(); ph_b += t2 - tm; wk_b += t2 - tm; tm = t2; }
#endif
                __syncthreads();  // barrier Y: P and alpha of block t, block t + 1 are in LDS
#ifdef MLA_TIMELINE
                { const unsigned long long t2 = MLA_MT32(); ph_o += t2 - tm; }
#endif
            }
            MLA_STAMP32(2, __builtin_amdgcn_s_memrealtime());
#ifdef MLA_TIMELINE
            MLA_STAMP32(6, ph_a);
            MLA_STAMP32(7, ph_b);
            MLA_STAMP32(8, ph_o);
            MLA_STAMP32W(0, 4, wk_a);
            MLA_STAMP32W(0, 5, wk_b);
#endif
            const float lsum = sum_over_lane_groups(l_run);
            if (w4 < kNS && lane < 16) {
                const size_t mi = (size_t)slot * num_heads + head0 + 16 * my_sh + lane;
                __builtin_nontemporal_store(m_run, m_part + mi);
                __builtin_nontemporal_store(lsum, l_part + mi);
            }
        } else {
            __syncthreads();  // the S waves' Q* reads

            floatx4 o[kNS][8];
#pragma unroll
            for (int sh = 0; sh < kNS; ++sh)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
                    o[sh][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
            // P of block j for this lane's tokens g, g + 4, g + 8, g + 12
            floatx4 pq[kNS];
            // token quads [ks0, ks1) of block j's second product
            auto o_quads = [&](int j, auto ks0, auto ks1) {
                const float *cs = s_c + (j % kRing) * kSlot;
#pragma unroll
                for (int ks = decltype(ks0)::value; ks < decltype(ks1)::value; ++ks) {
                    const int row = 4 * ks + g;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const floatx4 a = *(const floatx4 *)(cs + slot_at(row, 32 * w4 + 16 * h + l16));
#pragma unroll
                        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                            for (int sh = 0; sh < kNS; ++sh)
                                o[sh][4 * h + tt] = mfma16x16x4f32(a[tt], pq[sh][ks], o[sh][4 * h + tt]);
                    }
                }
            };
            for (int t = 0; t <= nblk; ++t) {
#ifdef MLA_TIMELINE
                tm = MLA_MT32();
#endif
                // block t + 2 into the slot that block t - 2 left at the end
                // of the previous step (the O waves' share)
                if (t + 2 < nblk)
                    issue_block(t + 2);
                if (t >= 1) {
                    // ---- O^T += C_N^T P^T of block t - 1 (rescaled by its alpha first)
#pragma unroll
                    for (int sh = 0; sh < kNS; ++sh) {
                        pq[sh] = *(const floatx4 *)(s_p + ((t - 1) & 1) * HT * kTRow + tile_at(16 * sh + l16, g));
                        const float alpha = s_alpha[((t - 1) & 1) * HT + 16 * sh + l16];
#pragma unroll
                        for (int dt = 0; dt < 8; ++dt)
                            o[sh][dt] *= alpha;
                    }
                    o_quads(t - 1, std::integral_constant<int, 0>{}, std::integral_constant<int, kQuadsA>{});
                }
#ifdef MLA_TIMELINE
                wk_a += MLA_MT32() - tm;
                tm = MLA_MT32();
#endif
                __syncthreads();  // barrier X
                if (t >= 1)
                    o_quads(t - 1, std::integral_constant<int, kQuadsA>{}, std::integral_constant<int, 4>{});
                if (t + 2 < nblk)
                    MLA_WAIT_VMCNT(kLoadsO);
                else
                    MLA_WAIT_VMCNT(0);
#ifdef MLA_TIMELINE
                wk_b += MLA_MT32() - tm;
#endif
                __syncthreads();  // barrier Y
            }
#ifdef MLA_TIMELINE
            MLA_STAMP32W(4, 9, wk_a);
            MLA_STAMP32W(4, 10, wk_b);
#endif
            // in the MFMA accumulator order of natural 16 x 16 tiles (frag_offset):
            // lane (head j, g) holds, over o[sh][4h .. 4h+3], dims 16g .. 16g+15 of
            // tile 8*w4 + 4h + g of sub-tile sh, element r of o[sh][4h + t]
            // being dim 4r + t of it; each store writes 4 runs of 256
            // contiguous bytes. Nontemporal, as the partials are read once,
            // by the combine (see mla_splitkv_fp16.hip)
            float *obase = o_part + (size_t)slot * num_heads * kDV;
#pragma unroll
            for (int sh = 0; sh < kNS; ++sh)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const floatx4 v = {o[sh][4 * h][r], o[sh][4 * h + 1][r], o[sh][4 * h + 2][r],
                                           o[sh][4 * h + 3][r]};
                        __builtin_nontemporal_store(
                            v, (floatx4 *)(obase + frag_offset(head0 + 16 * sh + l16,
                                                               128 * w4 + 64 * h + 16 * g + 4 * r)));
                    }
        }
#ifdef MLA_TIMELINE
        MLA_WAIT_VMCNT(0);
#endif
        MLA_STAMP32(3, __builtin_amdgcn_s_memrealtime());
    }
}

}  // namespace

hipError_t launch_splitkv_fp32(const Problem &pb, const Plan &p, const Partials &w, hipStream_t s)
{
    if (p.n_chunks == 0)
        return hipSuccess;
    if (p.head_tile != 16 && p.head_tile != 32)
        return hipErrorInvalidValue;
    const dim3 grid(grid_chunks(p) * p.n_head_tiles), block(64 * kWaves);
    hipLaunchKernelGGL(p.head_tile == 32 ? splitkv_fp32_kernel<32> : splitkv_fp32_kernel<16>, grid, block, 0, s,
                       (const float *)pb.q, (const float *)pb.c, pb.cu_seqlens,
                       static_cast<float *>(w.o), w.m, w.l, pb.num_heads, pb.batch, pb.total_tokens,
                       p.chunk, p.n_head_tiles, p.xcd_remap, pb.scale_log2);
    // the launch's own error; hipPeekAtLastError leaves a sticky error from
    // the caller's earlier work in place for the caller to see
    return hipPeekAtLastError();
}

}  // namespace mla

#ifdef MLA_TIMELINE
extern "C" int mla_timeline_read_f32(void *dst, size_t bytes)
{
    const size_t n = bytes < sizeof(mla::mla_timeline_stamps_f32) ? bytes : sizeof(mla::mla_timeline_stamps_f32);
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(mla::mla_timeline_stamps_f32), n, 0, hipMemcpyDeviceToHost);
}
#endif
