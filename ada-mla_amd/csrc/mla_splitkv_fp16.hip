// fp16 split-KV MLA decode for gfx950:
//   O*_partial = sum_t 2^(s_t - m) C_N[t],  s_t = log2(e) * scale * (Q* . C[t])
// for one (chunk of tokens, tile of heads) per workgroup, written as fp32
// partials (O unnormalised, running max m, running sum l) that
// mla_combine.hip merges.
//
// Replaces mla_decode_splitk_mma_fp16 (reference
// csrc/mla_decode_splitk_fwd.cuh:559-892), with a different design:
//  * 512 threads = 8 wave64s, one workgroup per CU, in two roles with one
//    wave of each role on every SIMD, so that one role's LDS and softmax
//    latencies hide behind the other role's MFMAs:
//      - S waves (HT/16 of them) compute the logits and the online softmax
//        of block t+1: S^T = C Q*^T on 16x16x32 MFMAs, each wave owning 16
//        heads x 32 tokens over the full K = 576 (eight independent
//        accumulation chains) with its Q* fragment resident in registers,
//        so no wave needs another wave's logits;
//      - O waves (4) accumulate block t: O^T = C_N^T P^T, each owning 128
//        output columns for all heads of the tile, with the C_N^T operand
//        read from the ring slot by the LDS transpose read
//        (ds_read_b64_tr_b16); they also feed the ring.
//    P (fp16) and the rescale factors pass from S to O waves through a
//    double-buffered LDS area; one workgroup barrier per block.
//  * C streams through a 4-slot LDS ring of 32-token blocks filled by
//    direct global->LDS loads (global_load_lds_dwordx4), two blocks ahead of
//    the S waves; each block is read from LDS by both products.
//  * Online softmax in fp32 (log2 domain), running max started at -inf; the
//    O rescale is skipped when no head's max moved (exact: the factor is 1).
//  * Rows of a ring slot are XOR-swizzled in 16-byte chunks so that both the
//    row-wise reads of the first product and the transpose reads of the
//    second hit distinct LDS banks.
//  * Barriers are plain s_barrier after an LDS counter wait: the
//    global->LDS loads are tracked with explicit vmcnt waits by the waves
//    that issue them, so a barrier never drains the loads in flight.
#include "mla_device.hpp"
#include "mla_internal.hpp"

namespace mla {
namespace {

template <int HT>
struct F16Tile {
    static constexpr int kWaves = 8;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kBT = 32;                      // tokens per block
    static constexpr int kRing = 4;                     // LDS ring slots
    static constexpr int kSWaves = HT / 16;             // S waves (16 heads each)
    static constexpr int kOWave0 = 4;                   // O waves are 4..7
    static constexpr int kNHS = HT / 16;                // 16-head sub-tiles per tile
    static constexpr int kChains = 4;                   // accumulation chains per S^T tile
    static constexpr int kSlot = kBT * kDK;             // halves per slot (36 KB)
    static constexpr int kUnits = kSlot * 2 / 1024;     // 1 KB load units per slot
    static constexpr int kLoadsPerWave = kUnits / 4;    // per O wave per block
    static constexpr int kPRow = kBT + 8;               // P row stride (halves)
    // Q* of the head tile is staged through the top ring slots at the start
    // of each piece (HT rows of 1152 bytes, swizzled like C rows).
    static constexpr int kQUnits = HT * kDK * 2 / 1024;
    static constexpr int kQLoadsPerWave = (kQUnits + 3) / 4;
    static constexpr int kQSlots = (HT * kDK + kSlot - 1) / kSlot;
    static constexpr int kPreBlocks = kRing - kQSlots;  // blocks issued with Q*
    static_assert(kUnits % 4 == 0, "units per wave");
    static_assert(kSWaves <= kOWave0, "S waves");
    static_assert(kQSlots >= 1 && kQSlots <= 2, "Q slots");
};

// XOR swizzle of the 16-byte chunk index within a 1152-byte row. Bits of the
// row (mod 16) are permuted so that 16 consecutive rows at one chunk hit 16
// distinct chunk positions (S^T operand reads), and the 32-byte chunk pairs
// read by the transpose loads of rows {r..r+3, r+8..r+11} land on 8 distinct
// pairs. Chunks 64..71 (the rope columns, never read transposed) use the low
// 3 bits only so they stay inside their 8-chunk group.
__device__ __forceinline__ int row_swizzle(int row)
{
    return ((row >> 2) & 1) | ((row & 3) << 1) | (row & 8);
}

__device__ __forceinline__ int phys_chunk(int c, int swz)
{
    return c < 64 ? (c ^ swz) : (c ^ (swz & 7));
}

// s_waitcnt vmcnt(n) leaving the other counters unconstrained.
#define MLA_WAIT_VMCNT(n) \
    __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (7 << 4) | (0xF << 8))

// Workgroup barrier that waits only for this wave's LDS operations; the
// memory clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16 bytes per lane from base + off (bytes) into LDS at lds + 16 * lane
// (global_load_lds_dwordx4; lds must be wave-uniform). Issued as inline asm
// so that the compiler does not model it: it would otherwise wait for every
// such load before each LDS read. The kernel orders these loads itself with
// MLA_WAIT_VMCNT; the compiler's own vmcnt waits stay correct because
// vector-memory loads retire in order, so loads it does not count only make
// its waits more conservative.
__device__ __forceinline__ void global_to_lds16(const _Float16 *base, int off, const void *lds)
{
    const unsigned l = __builtin_amdgcn_readfirstlane(
        (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)lds);
    unsigned saved_m0;
    // m0 carries the LDS address; its previous value is restored so the asm
    // leaves the (compiler-reserved) register unchanged.
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %3\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved_m0) : "v"(off), "s"(base), "s"(l) : "memory");
}

template <int HT, bool kTr>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
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
    __shared__ __attribute__((aligned(1024))) _Float16 s_ring[T::kRing * T::kSlot];
    __shared__ __attribute__((aligned(16))) _Float16 s_p[2][HT * T::kPRow];
    __shared__ float s_alpha[2][HT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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

    const bool s_wave = wave < T::kSWaves;   // logits + softmax of 16 heads
    const bool o_wave = wave >= T::kOWave0;  // 128 output columns + ring loads
    const int hg = s_wave ? wave : 0;        // S wave: its 16-head group
    const int ow = wave - T::kOWave0;        // O wave: its column quarter
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

    // Per-lane chunk offsets of the S^T operand reads (rows 16*tt + l16,
    // logical chunk 4*kk + g). For kk < 16 the swizzle permutes kk within
    // aligned groups of 4 and g within 0..3, so four offsets plus immediates
    // cover them; the rope chunks 64..71 have two more.
    const int swz_a = row_swizzle(l16);
    int a_off[6];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        a_off[j] = 8 * (4 * (j ^ (swz_a >> 2)) + ((g ^ swz_a) & 3));
#pragma unroll
    for (int j = 0; j < 2; ++j)
        a_off[4 + j] = 8 * (64 + ((4 * j + g) ^ (swz_a & 7)));
    auto a_chunk = [&](int kk) { return kk < 16 ? a_off[kk & 3] + 128 * (kk >> 2) : a_off[kk - 12]; };

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
        const int slot_out = split + b;
        const int nblk = (p_hi - p_lo + T::kBT - 1) / T::kBT;

        lds_barrier();  // the ring and the P / alpha buffers are reused from the previous piece

        // Global -> LDS load of block `blk` into ring slot blk % kRing by the
        // O waves. Load unit u (1 KB) = chunk positions [64u, 64u + 64) of
        // the slot; lane l fetches the logical chunk stored at position
        // 64u + l. Rows past the end of the piece re-read its last token
        // (finite data, masked later); a block past the last one re-reads
        // only that token.
        auto issue_block = [&](int blk) {
            const int t0 = min(p_lo + blk * T::kBT, p_hi - 1);
            const int lim = p_hi - 1 - t0;
            const _Float16 *base = c + (size_t)t0 * kDK;
            _Float16 *slot = s_ring + (blk % T::kRing) * T::kSlot;
#pragma unroll
            for (int k = 0; k < T::kLoadsPerWave; ++k) {
                const int u = ow + 4 * k;
                const int pos = 64 * u + lane;
                const int row = pos / 72;
                const int pc = pos - 72 * row;
                const int lc = phys_chunk(pc, row_swizzle(row));
                global_to_lds16(base, (min(row, lim) * kDK + lc * 8) * 2, slot + u * 512);
            }
        };

        // Prologue: Q* rows of this head tile go to the top kQSlots ring
        // slots (their blocks are not needed yet), blocks 0.. to the others;
        // blocks 0..2 are always issued (past the last block as re-reads of
        // the last token), so every wait count is a constant.
        if (o_wave) {
            const _Float16 *qbase = q + ((size_t)b * num_heads + head0) * kDK;
            _Float16 *qslot = s_ring + T::kPreBlocks * T::kSlot;
#pragma unroll
            for (int k = 0; k < T::kQLoadsPerWave; ++k) {
                const int u = min(ow + 4 * k, T::kQUnits - 1);
                const int pos = 64 * u + lane;
                const int row = pos / 72;
                const int pc = pos - 72 * row;
                global_to_lds16(qbase, (row * kDK + 8 * phys_chunk(pc, row_swizzle(row))) * 2,
                                qslot + u * 512);
            }
#pragma unroll
            for (int blk = 0; blk < T::kPreBlocks; ++blk)
                issue_block(blk);
            MLA_WAIT_VMCNT(T::kPreBlocks * T::kLoadsPerWave);  // Q* has landed
        }
        lds_barrier();

        // Each role runs its own copy of the step loop (t = -1 .. nblk-1,
        // S waves on block t+1, O waves on block t) with the same sequence of
        // barriers, so that the registers of one role (Q* fragments, logit
        // accumulators) and of the other (O accumulators) can share space.
        if (s_wave) {
            // Q* fragment (B operand of S^T = C Q*^T): lane holds head
            // 16*hg + l16 of the tile, dims 32*kk + 8*g .. +7.
            half8 qf[kDK / 32];
            {
                const _Float16 *qs = s_ring + T::kPreBlocks * T::kSlot + (16 * hg + l16) * kDK;
#pragma unroll
                for (int kk = 0; kk < kDK / 32; ++kk)
                    qf[kk] = *(const half8 *)(qs + a_chunk(kk));
            }
            lds_barrier();  // Q* slots are free again
            lds_barrier();  // block 0 has landed

            float m_run = -INFINITY, l_run = 0.f;  // head 16*hg + l16
            for (int t = -1; t < nblk; ++t) {
                if (t + 1 < nblk) {
                    const int blk = t + 1;
                    const int t0 = p_lo + blk * T::kBT;
                    const _Float16 *cs = s_ring + (blk % T::kRing) * T::kSlot;
                    // ---- S^T tiles: tokens t0 + 16*tt + (0..15), heads 16*hg + (0..15).
                    // The 36 operand reads go out in batches of 3 K-steps one
                    // batch ahead of the MFMAs that consume them.
                    floatx4 acc[2][T::kChains];
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                        for (int j = 0; j < T::kChains; ++j)
                            acc[tt][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                    constexpr int kB = 3;  // K-steps per batch
                    half8 ab[2][kB][2];
                    auto load_batch = [&](int buf, int k0) {
#pragma unroll
                        for (int k = 0; k < kB; ++k)
#pragma unroll
                            for (int tt = 0; tt < 2; ++tt)
                                ab[buf][k][tt] = *(const half8 *)(cs + (16 * tt + l16) * kDK + a_chunk(k0 + k));
                    };
                    load_batch(0, 0);
#pragma unroll
                    for (int kb = 0; kb < kDK / 32 / kB; ++kb) {
                        if (kb + 1 < kDK / 32 / kB)
                            load_batch((kb + 1) & 1, (kb + 1) * kB);
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int k = 0; k < kB; ++k)
#pragma unroll
                            for (int tt = 0; tt < 2; ++tt) {
                                const int kk = kb * kB + k;
                                acc[tt][kk % T::kChains] =
                                    mfma16x16x32(ab[kb & 1][k][tt], qf[kk], acc[tt][kk % T::kChains]);
                            }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    // ---- online softmax over the block for this wave's heads
                    float sv[2][4];
                    float mx = -INFINITY;
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const floatx4 st = (acc[tt][0] + acc[tt][1]) + (acc[tt][2] + acc[tt][3]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int tok = t0 + 16 * tt + 4 * g + i;
                            sv[tt][i] = tok < p_hi ? st[i] * scale_log2 : -INFINITY;
                            mx = fmaxf(mx, sv[tt][i]);
                        }
                    }
                    mx = max_over_lane_groups(mx);
                    const float mn = fmaxf(m_run, mx);
                    const float alpha = fast_exp2(m_run - mn);
                    m_run = mn;
                    float psum = 0.f;
                    _Float16 *prow = s_p[blk & 1] + (16 * hg + l16) * T::kPRow + 4 * g;
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        half4 ph;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float p = fast_exp2(sv[tt][i] - mn);
                            psum += p;
                            ph[i] = (_Float16)p;
                        }
                        *(half4 *)(prow + 16 * tt) = ph;
                    }
                    l_run = l_run * alpha + psum;
                    if (g == 0)
                        s_alpha[blk & 1][16 * hg + l16] = alpha;
                }
                lds_barrier();
            }
            // ---- epilogue: m and l of this wave's heads
            const float ls = sum_over_lane_groups(l_run);
            if (g == 0) {
                m_part[(size_t)slot_out * num_heads + head0 + 16 * hg + l16] = m_run;
                l_part[(size_t)slot_out * num_heads + head0 + 16 * hg + l16] = ls;
            }
        } else if (o_wave) {
            lds_barrier();  // Q* slots are free again
#pragma unroll
            for (int blk = T::kPreBlocks; blk < T::kRing - 1; ++blk)
                issue_block(blk);
            // block 0 has landed; blocks 1 and 2 may stay in flight
            MLA_WAIT_VMCNT(2 * T::kLoadsPerWave);
            lds_barrier();

            floatx4 o[T::kNHS][8];
#pragma unroll
            for (int hs = 0; hs < T::kNHS; ++hs)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
                    o[hs][dt] = floatx4{0.f, 0.f, 0.f, 0.f};

            for (int t = -1; t < nblk; ++t) {
                if (t >= 0 && t + T::kRing - 1 < nblk)
                    issue_block(t + T::kRing - 1);  // into the slot block t-1 left
                if (t >= 0) {
                    const int blk = t;
                    const _Float16 *cs = s_ring + (blk % T::kRing) * T::kSlot;
                    // ---- rescale, skipped when no head's max moved
                    float alpha[T::kNHS];
                    bool moved = false;
#pragma unroll
                    for (int hs = 0; hs < T::kNHS; ++hs) {
                        alpha[hs] = s_alpha[blk & 1][16 * hs + l16];
                        moved |= alpha[hs] != 1.0f;
                    }
                    if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
                        for (int hs = 0; hs < T::kNHS; ++hs)
#pragma unroll
                            for (int dt = 0; dt < 8; ++dt)
                                o[hs][dt] *= alpha[hs];
                    }
                    // ---- O^T[dims 128*ow .. +128][heads] += C_N^T P^T. All 20
                    // operand reads are issued before the 32 MFMAs.
                    half8 pb[T::kNHS];
#pragma unroll
                    for (int hs = 0; hs < T::kNHS; ++hs)
                        pb[hs] = *(const half8 *)(s_p[blk & 1] + (16 * hs + l16) * T::kPRow + 8 * g);
                    half8 av[8];
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) {
                        if constexpr (kTr) {
                            // lane (g, j): rows 8g + j/4 (+4), dims 128*ow + 16*dt + 4*(j%4) .. +3
                            const int r0 = 8 * g + (l16 >> 2);
                            const int cl = 16 * ow + 2 * dt + ((l16 & 3) >> 1);
                            const int sub = 4 * (l16 & 1);
                            const _Float16 *p0 = cs + r0 * kDK + 8 * phys_chunk(cl, row_swizzle(r0)) + sub;
                            const _Float16 *p1 = cs + (r0 + 4) * kDK + 8 * phys_chunk(cl, row_swizzle(r0 + 4)) + sub;
                            const half4 lo4 = lds_read_tr16(p0);
                            const half4 hi4 = lds_read_tr16(p1);
                            av[dt] = half8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                        } else {
                            const int col = 128 * ow + 16 * dt + l16;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                const int r = 8 * g + j;
                                av[dt][j] = cs[r * kDK + 8 * phys_chunk(col >> 3, row_swizzle(r)) + (col & 7)];
                            }
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                        for (int hs = 0; hs < T::kNHS; ++hs)
                            o[hs][dt] = mfma16x16x32(av[dt], pb[hs], o[hs][dt]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // ---- block t+2 (the S waves' next-but-one) must have landed
                // before the barrier; block t+3 may stay in flight
                if (t >= 0 && t + T::kRing - 1 < nblk) MLA_WAIT_VMCNT(T::kLoadsPerWave);
                else MLA_WAIT_VMCNT(0);
                lds_barrier();
            }
            // ---- epilogue: the unnormalised O of this piece
            float *obase = o_part + ((size_t)slot_out * num_heads + head0 + l16) * kDV + 128 * ow + 4 * g;
#pragma unroll
            for (int hs = 0; hs < T::kNHS; ++hs)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
                    *(floatx4 *)(obase + 16 * hs * kDV + 16 * dt) = o[hs][dt];
        } else {
            // waves with no role at this head-tile size keep the barrier count
            lds_barrier();
            lds_barrier();
            for (int t = -1; t < nblk; ++t)
                lds_barrier();
        }
    }
}

template <int HT, bool kTr>
hipError_t launch_ht(const Problem &pb, const Plan &p, const Partials &w, hipStream_t s)
{
    const dim3 grid(p.n_chunks * p.n_head_tiles), block(F16Tile<HT>::kThreads);
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
    switch (p.head_tile) {
    case 64: return tr_load ? launch_ht<64, true>(pb, p, w, s) : launch_ht<64, false>(pb, p, w, s);
    case 32: return tr_load ? launch_ht<32, true>(pb, p, w, s) : launch_ht<32, false>(pb, p, w, s);
    default: return tr_load ? launch_ht<16, true>(pb, p, w, s) : launch_ht<16, false>(pb, p, w, s);
    }
}

}  // namespace mla
