// fp16 split-KV MLA decode for gfx950:
//   O*_partial = sum_t 2^(s_t - m) C_N[t] / l,  l = sum_t 2^(s_t - m),
//   s_t = log2(e) * scale * (Q* . C[t])
// for one (chunk of tokens, tile of heads) per workgroup, written as
// partials (O normalised by l in fp16; running max m and sum l in fp32)
// that mla_combine.hip merges. Normalised, O is a convex combination of C_N
// rows, so fp16 holds it at fp16's relative precision whatever the chunk
// length; the reference's split partials were fp16 as well (unnormalised).
//
// Replaces mla_decode_splitk_mma_fp16 (reference
// csrc/mla_decode_splitk_fwd.cuh:559-892), with a different design:
//  * 512 threads = 8 wave64s (640 = 10 at 32-head tiles), one workgroup per
//    CU, in two roles with one wave of each role on every SIMD, so that one
//    role's LDS and softmax latencies hide behind the other role's MFMAs:
//      - S waves compute the logits and the online softmax of block t+1:
//        S^T = C Q*^T on 16x16x32 MFMAs over the full K = 576. Wave
//        (head group, token half) owns up to 32 heads x 16 tokens of each
//        32-token block, with the Q* of its heads resident in registers, so
//        each C row is read from LDS once per head group. Each wave keeps its
//        own running max: the two token halves of a head agree on a common
//        reference only in the O waves (below), so no wave waits for
//        another's logits.
//      - O waves (4) accumulate block t: O^T = C_N^T P^T, each owning 128
//        output columns for all heads of the tile, with the C_N^T operand
//        read by the LDS transpose read (ds_read_b64_tr_b16) one step ahead,
//        between the MFMAs of the current block. Per head they take M = max
//        of the two halves' running maxima, scale each half's P by
//        2^(m_half - M) and the accumulator by 2^(M_old - M).
//      - the ring is fed (global->LDS loads) by the O waves, between their
//        MFMAs, when the head tile is 64; for tiles of 16 heads two S waves
//        suffice and waves 2 and 3 only feed the ring, which keeps the
//        load-issue stalls off the O waves; tiles of 32 heads run four
//        16-head S waves and two more waves, 8 and 9, that feed.
//    P (fp16) and the halves' maxima pass from S to O waves through a
//    double-buffered LDS area; one workgroup barrier per block.
//  * C streams through a 4-slot LDS ring of 32-token blocks filled by
//    direct global->LDS loads (global_load_lds_dwordx4). Q* of the head tile
//    comes first, through the top slots, so the S waves can load it into
//    registers while blocks 0.. arrive; afterwards block t+4 is requested
//    into the slot of block t as soon as step t begins (its C_N^T operand
//    is already in registers by then). Each block is read from LDS by both
//    products.
//  * Online softmax in fp32 (log2 domain), running max started at -inf; the
//    O rescale is skipped when no head's max moved (exact: the factor is 1).
//  * Rows of a ring slot are XOR-swizzled in 16-byte chunks so that both the
//    row-wise reads of the first product and the transpose reads of the
//    second hit distinct LDS banks.
//  * Barriers are plain s_barrier after an LDS counter wait: the
//    global->LDS loads are tracked with explicit vmcnt waits by the waves
//    that issue them, so a barrier never drains the loads in flight.
//  * The partial O is stored tile by tile in the MFMA accumulator order
//    (frag_offset): every store instruction writes 512 B of contiguous memory.
//    The partials (O, m, l) are written with nontemporal stores: they are read
//    once, by the combine kernel, and kept out of the L2 they need not be
//    written back from at the end of the kernel. Measured at N = 4096 (4.2 MB
//    of partials): 12.78 -> 11.85 us per call. Plans whose combine runs on
//    few workgroups store them plainly instead (part_plain; the planner's
//    choose_part_plain has the measurements).
#include <type_traits>

#include "mla_device.hpp"
#include "mla_internal.hpp"
#include "mla_ring.hpp"

namespace mla {

#ifdef MLA_TIMELINE
// Timeline build only (python ada-mla_amd/build.py --timeline, read by
// ada-mla_amd/timeline.py through mla_timeline_read): per workgroup, 16
// stamps of its last piece -- s_memrealtime (100 MHz, one clock for the whole
// GPU) at the phase boundaries of wave 0 (an S wave) and wave 4 (an O wave),
// s_memtime (shader clock) around both waves' block loops, the piece's block
// count and the hardware ids. The normal build compiles none of it.
constexpr int kTimelineWorkgroups = 8192;
__device__ unsigned long long mla_timeline_stamps[kTimelineWorkgroups * 16];
#define MLA_STAMP(w, e, v)                                                              \
    do {                                                                               \
        if (wave == (w) && lane == 0 && blockIdx.x < kTimelineWorkgroups)              \
            mla_timeline_stamps[blockIdx.x * 16 + (e)] = (unsigned long long)(v);      \
    } while (0)
#define MLA_RT() __builtin_amdgcn_s_memrealtime()
#define MLA_MT() __builtin_amdgcn_s_memtime()
#else
#define MLA_STAMP(w, e, v) \
    do {                   \
    } while (0)
#endif

namespace {

template <int HT>
struct F16Tile {
    // kTen: 32-head tiles run 10 waves -- four 16-head S waves (head group,
    // token half), four O waves and two dedicated feeders (waves 8 and 9),
    // three waves on SIMDs 0 and 1 (at most 168 registers each). With two
    // 32-head S waves (8 waves) the first product and the softmax of a block
    // ran on SIMDs 0 and 1 only; split over four SIMDs the step went from
    // 1630 to 1283 cycles at N = 65536 (the clock fell from 2.0 to 1.86 GHz:
    // 0.815 -> 0.696 us) and the split kernel from 30.0 to 28.8 us (same box).
    static constexpr bool kTen = HT == 32;
    static constexpr int kWaves = kTen ? 10 : 8;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kBT = 32;                      // tokens per block
    static constexpr int kRing = 4;                     // LDS ring slots
    static constexpr int kSH = kTen ? 16 : HT < 32 ? HT : 32;  // heads per S wave
    static constexpr int kNS = kSH / 16;                // 16-head sub-tiles per S wave
    static constexpr int kNHG = HT / kSH;               // head groups
    static constexpr int kSWaves = 2 * kNHG;            // S waves: (head group, token half)
    static constexpr int kChains = 4 / kNS;             // accumulation chains per sub-tile
    static constexpr int kOWave0 = 4;                   // O waves are 4..7
    static constexpr int kNHS = HT / 16;                // 16-head sub-tiles per tile
    static constexpr int kSlot = kBT * kDK;             // halves per slot (36 KB)
    static constexpr int kRope = kBT * kDV;             // halves: rope area of a slot (after the C_N rows)
    static constexpr int kUnits = kSlot * 2 / 1024;     // 1 KB load units per slot
    static constexpr int kPRow = kBT + 8;               // P row stride (halves)
    // Q* of the head tile is staged through the top ring slots at the start
    // of each piece (HT rows of 1152 bytes, swizzled like C rows).
    static constexpr int kQBlocks = (HT + kBT - 1) / kBT;
    static constexpr int kPre = kRing - kQBlocks;       // blocks issued with Q*
    // Feeding of the ring (global -> LDS): the O waves at HT = 64, else the
    // two waves after the S waves; each feeder owns kFeedRows rows of a block.
    static constexpr bool kOFeeds = !kTen && kSWaves == kOWave0;
    static constexpr int kFeedWave0 = kOFeeds ? kOWave0 : kTen ? 8 : kSWaves;  // first feeder wave
    static constexpr int kFeeders = kOFeeds ? 4 : 2;
    static constexpr int kFeedRows = kBT / kFeeders;
    static constexpr int kFeedUnits = kFeedRows + kFeedRows / 8;  // C_N rows + rope units
    static_assert(kFeeders * kFeedUnits == kUnits, "feeder split");
    static_assert(kOFeeds || kSWaves == 2 || kTen, "feeder waves are 2 and 3 (8 and 9 with kTen)");
    static_assert(3 * kFeedUnits <= 63, "vmcnt range");
};

// kF32Part: the partial O is stored in fp32 (still normalised) instead of E.
// kF8: the cache C is OCP fp8 (E4M3FN) [tokens][576] bytes and c points to
// it (E is then fp16 for Q* and P). The ring holds the fp8 bytes as loaded
// (a block takes the first 18 KB of its slot; the load units are 512 bytes,
// 32 lanes of a global->LDS load, except for the feeders' 1 KB units of
// two rows), so a CU fills half the bytes of a 16-bit
// cache; the S and O waves convert their operands to fp16 after each LDS
// read, exactly (every E4M3 value is an fp16 value). The per-tensor cache
// scale is folded into scale_log2 and out_scale.
// kMode: kModeBatch (cu_seqlens: a chunk may hold pieces of several
// sequences), kModeSingle (one sequence: the chunk is one piece, whose
// prologue loads go out at kernel entry) or kModeDirect (kModeSingle with a
// single chunk: its normalised O is the output, so the O waves write it to
// out ([head][512]) and no partials, m or l are stored; the call needs no
// combine launch).
constexpr int kModeBatch = 0;
constexpr int kModeSingle = 1;
constexpr int kModeDirect = 2;

template <int HT, bool kTr, typename E, bool kPaged, bool kF32Part, bool kF8, int kMode>
__global__ __attribute__((amdgpu_flat_work_group_size(F16Tile<HT>::kThreads, F16Tile<HT>::kThreads),
                          amdgpu_waves_per_eu(F16Tile<HT>::kWaves > 8 ? 3 : 2, F16Tile<HT>::kWaves > 8 ? 3 : 2)))
// Arguments: what the workgroup mapping and a single sequence's entry loads
// need come first, within the 16 dwords preloaded into SGPRs at wave launch
// (the library is built with -amdgpu-kernarg-preload-count=16).
void splitkv_fp16_kernel(const E *__restrict__ q,
                         const E *__restrict__ c,
                         const int *__restrict__ cu_seqlens,
                         int num_heads, int batch, int total_tokens, int chunk,
                         int n_head_tiles, int xcd_remap,
                         void *__restrict__ o_part,
                         float *__restrict__ m_part,
                         float *__restrict__ l_part,
                         float scale_log2, Paging pg,
                         float out_scale, E *__restrict__ out, int part_plain, int seq_cost)
{
    using T = F16Tile<HT>;
    constexpr bool kDirect = kMode == kModeDirect;
    // fp8 cache, tiles of 32 or 64 heads: the first product on fp8 MFMAs
    // (Q* split, below); tiles of 16 heads convert C to fp16 for it instead,
    // where the split's fixed cost per piece exceeds what it saves
    constexpr bool kF8M = kF8 && HT >= 32;
    static_assert(kMode == kModeBatch || !kPaged, "a paged cache comes with cu_seqlens");
    static_assert(!(kF8 && (kPaged || !__is_same(E, _Float16))), "fp8 cache: packed layout, fp16 query");
    using E8 = typename Vec<E>::v8;
    using E4 = typename Vec<E>::v4;
    __shared__ __attribute__((aligned(1024))) E s_ring[T::kRing * T::kSlot];
    __shared__ __attribute__((aligned(16))) E s_p[2][HT * T::kPRow];
    // [P buffer][head % 16][head / 16][token half]: running max of the half,
    // so that an O wave reads the maxima of all its heads (both halves) with
    // one or two 16-byte reads per lane; m_at(h, th) indexes a buffer
    __shared__ __attribute__((aligned(16))) float s_m[2][2 * HT];
    auto m_at = [](int h, int th) { return ((h & 15) * T::kNHS + (h >> 4)) * 2 + th; };
    __shared__ float s_l[2][HT];     // [token half][head]: running sum at the end of a piece
    __shared__ float s_mref[HT];     // [head]: the O accumulators' reference max at the end of a piece

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15;
    const int g = lane >> 4;
    MLA_STAMP(0, 0, MLA_RT());

    // workgroup -> (chunk, head tile). With xcd_remap the head tiles of one
    // chunk get ids that are equal mod 8, i.e. land on the same XCD (blocks
    // are dispatched round-robin over the 8 XCDs), so C is pulled from HBM
    // into that XCD's L2 once and re-read from L2 by the other head tiles.
    // The grid then holds a multiple of 8 chunks; the padding workgroups
    // (split >= n_chunks) return below.
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
    // The chunk's tokens [lo, hi). A batch is chunked over its virtual
    // length (seq_virtual_bound): chunk w covers virtual positions
    // [w chunk, (w + 1) chunk), every sequence start counting seq_cost
    // tokens, so that chunks holding more pieces hold fewer tokens.
    // b_first: the first sequence with tokens at or after lo.
    int lo, hi, b_first = 0;
    int first_lo = 0, first_hi = 0;  // bounds of sequence b_first
    const int nseq = cu_seqlens ? batch : 1;
    if (cu_seqlens) {
        b_first = seq_virtual_bound(cu_seqlens, batch, total_tokens, seq_cost, (long long)split * chunk, lane, lo,
                                    first_lo, first_hi);
        int u0, u1;
        seq_virtual_bound(cu_seqlens, batch, total_tokens, seq_cost, (long long)(split + 1) * chunk, lane, hi, u0, u1);
        if (lo >= hi)  // a padding workgroup, or a chunk that falls between sequences
            return;
    } else {
        if ((long long)split * chunk >= total_tokens)  // a padding workgroup of the grid
            return;
        lo = split * chunk;
        hi = min(lo + chunk, total_tokens);
    }
    const int head0 = ht * HT;
    // Calls body(b, seq_lo, p_org, p_lo, p_hi) for every non-empty piece
    // [p_lo, p_hi) of sequence b (whose first token is seq_lo) inside this
    // chunk. Blocks of the piece start at p_org: p_lo itself, or, for a paged
    // cache, p_lo rounded down to a multiple of 32 tokens of the sequence, so
    // that no block straddles a page (tokens before p_lo are masked). Every
    // wave walks the same pieces and, per piece, passes the same number of
    // barriers (nblk + 5; nblk + 4 for the chunk's first piece, whose
    // prologue loads go out at kernel entry and need no piece-start barrier;
    // one more with an fp8 cache and 32 or 64 heads, before the split of Q*).
    auto for_each_piece = [&](auto &&body) {
        for (int b = b_first; b < nseq; ++b) {
            int seq_lo = 0, seq_hi = total_tokens;
            if (cu_seqlens) {
                seq_lo = __builtin_amdgcn_readfirstlane(min(max(cu_seqlens[b], 0), total_tokens));
                seq_hi = __builtin_amdgcn_readfirstlane(min(max(cu_seqlens[b + 1], seq_lo), total_tokens));
            }
            if (seq_lo >= hi)
                break;
            const int p_lo = max(seq_lo, lo);
            const int p_hi = min(seq_hi, hi);
            const int p_org = kPaged ? p_lo - ((p_lo - seq_lo) & (T::kBT - 1)) : p_lo;
            if (p_lo < p_hi)
                body(b, seq_lo, p_org, p_lo, p_hi);
        }
    };

    // ---- global -> LDS loads of the ring (one 1 KB load unit per call):
    // the C_N part of row `row` of a 32-row block whose row 0 is at `base`
    // (lane = stored chunk position; it fetches logical chunk
    // lane ^ row_swizzle(row)), or the rope part of rows 8*ru .. 8*ru+7
    // (lane -> row 8*ru + lane/8, stored position lane % 8). Rows past `lim`
    // re-read row `lim` (finite data, masked later or never read).
    // The lane index is passed through an empty asm so that the offsets are
    // recomputed at each load (a few VALU ops) instead of being kept live,
    // or spilled, across the piece: a spill reload here would make the
    // compiler wait for every outstanding global->LDS load.
    auto dma_row = [&](const E *base, int lim, int slot, int row) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        global_to_lds16(base, min(row, lim) * (kDK * 2) + 16 * (ln ^ row_swizzle(row)),
                        s_ring + slot * T::kSlot + row * kDV);
    };
    auto dma_rope = [&](const E *base, int lim, int slot, int ru) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int rrow = 8 * ru + (ln >> 3);
        global_to_lds16(base, min(rrow, lim) * (kDK * 2) + 2 * (kDV + 8 * ((ln & 7) ^ rope_swizzle(rrow))),
                        s_ring + slot * T::kSlot + T::kRope + 512 * ru);
    };
    // Steady-state ring feeding: the lane part of a unit's global offset is
    // the same for every block, so each feeder forms it once (feed_off) and
    // a load then takes the block's first-row address (the row of a C_N
    // unit added to it, clamped to `lim`, on the scalar unit), that offset
    // and the slot's LDS address. A block cut short by the end of a piece
    // (lim < 31) loads its rope rows through dma_rope, which clamps per lane.
    const unsigned ring_lds = (unsigned)(uintptr_t)(const MLA_LDS E *)s_ring;
    auto feed_off = [&](int row_or_ru, bool rope) -> int {
        if (!rope)
            return 16 * (lane ^ row_swizzle(row_or_ru));
        const int r = lane >> 3;  // row within the unit's 8
        return r * (kDK * 2) + 2 * (kDV + 8 * ((lane & 7) ^ rope_swizzle(8 * row_or_ru + r)));
    };
    auto feed_row = [&](const E *base, int lim, int slot, int row, int off) {
        global_to_lds16_at(base + (size_t)min(row, lim) * kDK, off, ring_lds + 2 * (slot * T::kSlot + row * kDV));
    };
    auto feed_rope = [&](const E *base, int lim, int slot, int ru, int off) {
        if (lim >= 8 * ru + 7)
            global_to_lds16_at(base + (size_t)8 * ru * kDK, off, ring_lds + 2 * (slot * T::kSlot + T::kRope + 512 * ru));
        else
            dma_rope(base, lim, slot, ru);
    };
    // Global address of token t0 of sequence b (first token seq_lo), in two
    // steps so that a paged cache's block-table read can be issued early:
    // page_of reads the page id (0 for the packed layout), src_at forms the
    // address. The rows of a block that starts at t0 follow it contiguously
    // (same page).
    auto page_of = [&](int b, int seq_lo, int t0) -> int {
        if constexpr (kPaged) {
            // clamped: inconsistent tables stay memory-safe (wrong, not faulting)
            const int col = min((t0 - seq_lo) >> pg.page_shift, pg.bt_stride - 1);
            // a scalar load: the index is wave-uniform, and a vector load
            // here would be waited for with vmcnt, i.e. behind every
            // global->LDS load in flight
            const auto *bt = (const __attribute__((address_space(4))) int *)pg.block_table;
            return bt[(size_t)b * pg.bt_stride + col];
        } else {
            return 0;
        }
    };
    auto src_at = [&](int page, int seq_lo, int t0) -> const E * {
        if constexpr (kPaged) {
            page = min(max(page, 0), pg.num_pages - 1);
            const int l = t0 - seq_lo;
            return c + (((size_t)page << pg.page_shift) + (l & ((1 << pg.page_shift) - 1))) * kDK;
        } else {
            return c + (size_t)t0 * kDK;
        }
    };
    // fp8 ring slot (first 18 KB of a slot): the 512-byte C_N part of row r
    // at byte 512 r, its 16-byte chunk c stored at c ^ (r mod 16); the
    // 64-byte rope part at 16384 + 64 r, chunk c (0..3) at c ^ ((r / 4) mod 4).
    // The first product's 8-byte row reads and the second's transpose reads
    // (ds_read_b64_tr_b8) then touch 16 distinct 16-byte bank groups per 32
    // lanes. A load unit is 32 lanes x 16 bytes: one C_N row, or the rope
    // parts of 8 rows -- 36 units per block, as for a 16-bit cache.
    const unsigned char *c8 = reinterpret_cast<const unsigned char *>(c);
    unsigned char *ring8 = reinterpret_cast<unsigned char *>(s_ring);
    auto dma_row8 = [&](const unsigned char *base, int lim, int slot, int row) {
        if (lane < 32) {
            int ln = lane;
            asm volatile("" : "+v"(ln));
            global_to_lds16(base, min(row, lim) * kDK + 16 * (ln ^ row_swizzle(row)),
                            ring8 + slot * (T::kSlot * 2) + row * kDV);
        }
    };
    auto dma_rope8 = [&](const unsigned char *base, int lim, int slot, int ru) {
        if (lane < 32) {
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int rrow = 8 * ru + (ln >> 2);
            global_to_lds16(base, min(rrow, lim) * kDK + kDV + 16 * ((ln & 3) ^ ((rrow >> 2) & 3)),
                            ring8 + slot * (T::kSlot * 2) + kF8Rope + 512 * ru);
        }
    };
    // fp8, one 64-lane load unit: C_N rows row0 and row0 + 1 (lanes 0-31 and
    // 32-63; the two 512-byte rows are adjacent in the slot), or the rope
    // parts of rows 16 rr .. 16 rr + 15 (1 KB). The dedicated feeders use
    // these, so that a block takes 18 load instructions instead of 36.
    auto dma_row8x2 = [&](const unsigned char *base, int lim, int slot, int row0) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int row = row0 + (ln >> 5);
        global_to_lds16(base, min(row, lim) * kDK + 16 * ((ln & 31) ^ row_swizzle(row)),
                        ring8 + slot * (T::kSlot * 2) + row0 * kDV);
    };
    auto dma_rope8x16 = [&](const unsigned char *base, int lim, int slot, int rr) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int rrow = 16 * rr + (ln >> 2);
        global_to_lds16(base, min(rrow, lim) * kDK + kDV + 16 * ((ln & 3) ^ ((rrow >> 2) & 3)),
                        ring8 + slot * (T::kSlot * 2) + kF8Rope + 1024 * rr);
    };
    // 8 fp8 values -> 8 fp16 values (byte k -> element k)
    auto f8_to_f16 = [](uint2 v) -> half8 {
        const half2v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v.x, 1.0f, false);
        const half2v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v.x, 1.0f, true);
        const half2v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v.y, 1.0f, false);
        const half2v e = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(v.y, 1.0f, true);
        return half8{a[0], a[1], b[0], b[1], d[0], d[1], e[0], e[1]};
    };
    // a block's load units for either cache type: src is its first row
    auto block_src = [&](int page, int seq_lo, int t0) -> const void * {
        if constexpr (kF8)
            return c8 + (size_t)t0 * kDK;
        else
            return src_at(page, seq_lo, t0);
    };
    auto blk_row = [&](const void *src, int lim, int slot, int row) {
        if constexpr (kF8)
            dma_row8(static_cast<const unsigned char *>(src), lim, slot, row);
        else
            dma_row(static_cast<const E *>(src), lim, slot, row);
    };
    auto blk_rope = [&](const void *src, int lim, int slot, int ru) {
        if constexpr (kF8)
            dma_rope8(static_cast<const unsigned char *>(src), lim, slot, ru);
        else
            dma_rope(static_cast<const E *>(src), lim, slot, ru);
    };
    // Prologue loads of a piece, issued by all 8 waves (wave w: C_N rows
    // 4w..4w+3 and, for w < 4, the rope rows 8w..8w+7 of each block, i.e.
    // 5 load units per block for w < 4, else 4): Q* of the head tile into the top
    // kQBlocks slots first, then blocks 0..kPre-1. Each wave waits for its
    // own loads of Q* and block 0 only (prologue_own_wait); the barrier after
    // this (A) then publishes them to every wave, and blocks 1..kPre-1 land
    // while block 0 is computed (prologue_wait, and the feeders' first wait).
    // (waves 8 and 9 of a 10-wave tile, dedicated feeders, issue none)
    auto prologue_issue = [&](int b, int seq_lo, int p_org, int p_hi) {
        if (T::kWaves > 8 && wave >= 8)
            return;
        const E *qb = q + ((size_t)b * num_heads + head0) * kDK;
        // Q* rows past the tile's HT (16-head tiles: waves 4..7, and the rope
        // units of waves 2, 3) are not loaded: nothing reads them, and as
        // clamped re-reads of the last row they cost 18 KB of the 144 KB
        // the prologue issued per CU. (The waits count younger loads only, so
        // a wave that issues fewer Q* units waits the same way.)
#pragma unroll
        for (int j = 0; j < T::kQBlocks; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (4 * wave + r < HT - 32 * j)
                    dma_row(qb + (size_t)32 * j * kDK, HT - 1 - 32 * j, T::kPre + j, 4 * wave + r);
            if (wave < 4 && 8 * wave < HT - 32 * j)
                dma_rope(qb + (size_t)32 * j * kDK, HT - 1 - 32 * j, T::kPre + j, wave);
        }
        int pages[T::kPre];  // all page reads first: one wait for them all
#pragma unroll
        for (int blk = 0; blk < T::kPre; ++blk)
            pages[blk] = page_of(b, seq_lo, min(p_org + blk * T::kBT, p_hi - 1));
#pragma unroll
        for (int blk = 0; blk < T::kPre; ++blk) {
            const int t0 = min(p_org + blk * T::kBT, p_hi - 1);
            const void *src = block_src(pages[blk], seq_lo, t0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                blk_row(src, p_hi - 1 - t0, blk, 4 * wave + r);
            if (wave < 4)
                blk_rope(src, p_hi - 1 - t0, blk, wave);
        }
    };
    auto prologue_own_wait = [&]() {
        if (wave < 4)
            MLA_WAIT_VMCNT(5 * (T::kPre - 1));
        else if (T::kWaves == 8 || wave < 8)
            MLA_WAIT_VMCNT(4 * (T::kPre - 1));
    };
    // A single sequence's prologue loads (its chunk is one piece, [lo, hi))
    // go out at once, before the roles' set-up code: from a cold start the
    // waves take ~0.5-0.8 us to reach the first barrier (measured), which
    // the loads now overlap (same box, N = 4096: 11.85 -> 11.64 us per call;
    // n_h = 16: 16.8 -> 16.3 us). Batches issue every piece's loads after the
    // piece-start barrier, once the ring is free (piece_prologue), except
    // for the chunk's first piece, whose bounds the sequence search at entry
    // already found.
    int first_b = -1;
    if constexpr (kMode != kModeBatch) {
        first_b = 0;
        prologue_issue(0, 0, lo, hi);
    } else if (cu_seqlens) {
        // a batch's first piece: its bounds came with the chunk's (the
        // sequence search), so its loads go out now as well
        const int p_hi0 = min(first_hi, hi);
        if (b_first < batch && lo < p_hi0) {
            first_b = b_first;
            prologue_issue(b_first, first_lo, kPaged ? lo - ((lo - first_lo) & (T::kBT - 1)) : lo, p_hi0);
        }
    }
    // fp8 cache: the first product runs on fp8 MFMAs with Q* split into
    // two fp8 operands, so that C is used as stored (no conversion of the
    // first product's operand). Head h's Q* row is scaled by 2^e_h, a power
    // of two that puts its largest |q| in [128, 256), and
    //   hi = fp8(2^e q),  lo = fp8(16 (2^e q - hi)),
    // so q = 2^-e (hi + lo / 16) to about 2^-8 relative (hi holds 4
    // significant bits, lo the next 4; 16 (2^e q - hi) is at most 2^e q in
    // magnitude, so lo neither overflows nor, for the head's large entries,
    // goes subnormal). The S waves accumulate the products with hi and with
    // lo separately, combine them as hi + lo / 16 and scale by 2^-e_h in the
    // softmax (s_qsc[h] = scale_log2 2^-e_h).
    // 8 fp16 values -> 8 bytes of hi and of lo (byte k <- value k), two
    // values per instruction: the scaled conversions compute fp8(v / s)
    // and fp8 * s (round to nearest even, checked on gfx950), so with
    // si = 2^-e and sl = 2^-(e+4):
    //   hi = fp8(q / si),  r = q - hi * si (fp16, exact: hi * si is q
    //   rounded to 4 significant bits, within a factor 2 of q),
    //   lo = fp8(r / sl) = fp8(16 (2^e q - hi)).
    // kHalf: for heads whose largest |q| is 2^15 or more. Rounded to 4
    // significant bits, an entry of 63488 or more becomes 65536, which fp16
    // cannot hold (hi * si would be inf), so such heads form the residual at
    // half scale: r / 2 = q / 2 - hi * (si / 2), both terms exact in fp16
    // (q / 2 loses nothing for |q| >= 2^-14, and smaller entries are below
    // 2^-29 of the head's maximum), and lo = fp8((r / 2) / (sl / 2)).
    auto q_split8 = [](half8 x, float si, float sl, uint2 &hi, uint2 &lo, auto kHalf) {
        typedef short s16x2 __attribute__((ext_vector_type(2)));
        constexpr bool kH = decltype(kHalf)::value;
        const float sb = kH ? 0.5f * si : si, slb = kH ? 0.5f * sl : sl;
        unsigned hv[2], lv[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            half2v q0 = half2v{x[4 * p], x[4 * p + 1]}, q1 = half2v{x[4 * p + 2], x[4 * p + 3]};
            // (the first conversion of each register writes its low half; the
            // old value passed for the high half is overwritten by the second)
            s16x2 h = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(__builtin_bit_cast(s16x2, q1), q0, si, false);
            h = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(h, q1, si, true);
            const int hw = __builtin_bit_cast(int, h);
            const half2v b0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hw, sb, false);
            const half2v b1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hw, sb, true);
            if constexpr (kH) {
                q0 *= (_Float16)0.5f;
                q1 *= (_Float16)0.5f;
            }
            s16x2 l = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(__builtin_bit_cast(s16x2, q1), q0 - b0, slb, false);
            l = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(l, q1 - b1, slb, true);
            hv[p] = __builtin_bit_cast(unsigned, h);
            lv[p] = __builtin_bit_cast(unsigned, l);
        }
        hi = uint2{hv[0], hv[1]};
        lo = uint2{lv[0], lv[1]};
    };
    // The split runs once per piece, by all 8 waves, in place in the Q*
    // slots, after a barrier that follows Q*'s arrival (piece_prologue)
    // and before barrier A, while the first blocks are still landing: wave w
    // converts heads kQR*w .. +kQR-1, each by kQAct lanes of kQCpl 16-byte
    // chunks (8 values) of its 72 (64 C_N, 8 rope). A head's row keeps its
    // place: its C_N kilobyte then holds hi (bytes 0..511) and lo
    // (512..1023), 16-byte chunk c at c ^ (row mod 16); its 128-byte rope
    // part holds hi (0..63) and lo (64..127), 8-byte unit u at
    // u ^ ((row / 2) mod 8). A wave reads all its rows' chunks before it
    // writes any, and no other wave touches them.
    constexpr int kQR = HT / 8;                                      // heads per wave
    constexpr int kQLR = 64 / kQR;                                   // lanes per head
    constexpr int kQCpl = kQLR == 8 ? 9 : (kQLR == 16 ? 6 : 3);      // chunks per lane
    constexpr int kQAct = 72 / kQCpl;                                // active lanes per head
    static_assert(kQAct <= kQLR && kQAct * kQCpl == 72, "Q* split mapping");
    __shared__ float s_qsc[kF8M ? HT : 1];
    auto q_split_lds = [&]() __attribute__((always_inline)) {  // three call sites, one per role
        int ln = lane;  // opaque: the addresses below are formed here, not kept live
        asm volatile("" : "+v"(ln));
        const int h = kQR * wave + ln / kQLR;
        const int j = ln % kQLR;
        const int rr = h % 32;
        E *const qrow = s_ring + (T::kPre + h / 32) * T::kSlot + rr * kDV;
        E *const qrope = s_ring + (T::kPre + h / 32) * T::kSlot + T::kRope + rr * (kDK - kDV);
        half8 v[kQCpl];
        // max |q| over the lane's values: packed over the fp16 bit patterns
        // with the sign cleared (their unsigned order is the order of |q|)
        typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
        u16x2 mb = {0, 0};
#pragma unroll
        for (int i = 0; i < kQCpl; ++i) {
            const int ch = j + kQAct * i;
            v[i] = half8{};
            if (j < kQAct)
                v[i] = ch < 64 ? *(const half8 *)(qrow + 8 * (ch ^ row_swizzle(rr)))
                               : *(const half8 *)(qrope + 8 * ((ch - 64) ^ rope_swizzle(rr)));
            const uint4 u = __builtin_bit_cast(uint4, v[i]);
            mb = __builtin_elementwise_max(mb, __builtin_bit_cast(u16x2, u.x & 0x7fff7fffu));
            mb = __builtin_elementwise_max(mb, __builtin_bit_cast(u16x2, u.y & 0x7fff7fffu));
            mb = __builtin_elementwise_max(mb, __builtin_bit_cast(u16x2, u.z & 0x7fff7fffu));
            mb = __builtin_elementwise_max(mb, __builtin_bit_cast(u16x2, u.w & 0x7fff7fffu));
        }
        asm volatile("" ::: "memory");  // every read of the rows above the writes below
        // over the head's kQLR lanes (aligned groups of 8, 16 or 32):
        // quad swaps, then the mirrored half row and row (DPP), then the
        // other 16-lane row (v_permlane16_swap)
        int mi = mb[0] > mb[1] ? mb[0] : mb[1];
        mi = max(mi, __builtin_amdgcn_update_dpp(0, mi, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
        mi = max(mi, __builtin_amdgcn_update_dpp(0, mi, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
        mi = max(mi, __builtin_amdgcn_update_dpp(0, mi, 0x141, 0xF, 0xF, false));  // row_half_mirror
        if constexpr (kQLR >= 16)
            mi = max(mi, __builtin_amdgcn_update_dpp(0, mi, 0x140, 0xF, 0xF, false));  // row_mirror
        if constexpr (kQLR >= 32) {
            const auto sw = __builtin_amdgcn_permlane16_swap(mi, mi, false, false);
            mi = max((int)sw[0], (int)sw[1]);
        }
        const float amax = (float)__builtin_bit_cast(_Float16, (unsigned short)mi);
        // amax = m 2^x, m in [0.5, 1): 2^(8 - x) amax in [128, 256)
        const int e = 8 - __builtin_amdgcn_frexp_expf(amax);
        const float si = __builtin_ldexpf(1.f, -e);
        const bool big = amax >= 32768.f;  // the half-scale residual (q_split8)
        if (j == 0)
            s_qsc[h] = scale_log2 * si;
        unsigned char *const q8 = reinterpret_cast<unsigned char *>(qrow);
        unsigned char *const r8 = reinterpret_cast<unsigned char *>(qrope);
#pragma unroll
        for (int i = 0; i < kQCpl; ++i) {
            const int ch = j + kQAct * i;
            if (j < kQAct) {
                uint2 hi, lo;
                if (big)
                    q_split8(v[i], si, 0.0625f * si, hi, lo, std::true_type{});
                else
                    q_split8(v[i], si, 0.0625f * si, hi, lo, std::false_type{});
                if (ch < 64) {
                    const int o = 16 * ((ch >> 1) ^ (rr & 15)) + 8 * (ch & 1);
                    *(uint2 *)(q8 + o) = hi;
                    *(uint2 *)(q8 + 512 + o) = lo;
                } else {
                    const int o = 8 * ((ch - 64) ^ ((rr >> 1) & 7));
                    *(uint2 *)(r8 + o) = hi;
                    *(uint2 *)(r8 + 64 + o) = lo;
                }
            }
        }
    };

    auto piece_prologue = [&](int b, int seq_lo, int p_org, int p_hi) __attribute__((always_inline)) {
        if (b != first_b) {
            lds_barrier();  // piece start: buffers are reused from the previous piece
            prologue_issue(b, seq_lo, p_org, p_hi);
        }
        if constexpr (kF8M) {
            // Q* went out first: wait for it alone, so that the split runs
            // while the piece's first blocks arrive
            if (wave < 4)
                MLA_WAIT_VMCNT(5 * T::kPre);
            else if (T::kWaves == 8 || wave < 8)
                MLA_WAIT_VMCNT(4 * T::kPre);
            lds_barrier();  // Q* has landed
            if (T::kWaves == 8 || wave < 8)
                q_split_lds();
        }
        prologue_own_wait();
    };
    // End of step t (t + 2 < kPre), for a wave whose only loads in flight
    // are its prologue loads: its share of block t + 2 (the S waves' next
    // block) has landed; the one after it may stay in flight.
    static_assert(T::kPre >= 2 && T::kPre <= 3, "prologue blocks");
    auto prologue_wait = [&](int t) {
        if (t + 3 < T::kPre) {
            if (wave < 4)
                MLA_WAIT_VMCNT(5);
            else
                MLA_WAIT_VMCNT(4);
        } else {
            MLA_WAIT_VMCNT(0);
        }
    };

    // Each role runs its own piece loop and step loop (t = -1 .. nblk-1: S
    // waves on block t+1, O waves on block t) with the same sequence of
    // barriers, so that the registers of one role (Q* fragments, logit
    // accumulators) and of the other (O accumulators) can share space and
    // each role's set-up stays out of the other's instruction stream.
    if (wave < T::kSWaves) {
        const int hg = wave >> 1;  // head group
        const int th = wave & 1;   // token half of each block
        // Per-lane offsets (halves) of the row-wise operand reads: row r with
        // r % 16 == l16, logical chunk 4*kk + g. For kk < 16 the swizzle
        // permutes 4*(kk % 4) + g within aligned groups of 16 chunks, so four
        // offsets plus immediates cover them; the rope chunks 64..71 have two
        // more, relative to the rope row.
        int a_off[6];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            a_off[j] = 8 * ((4 * j + g) ^ row_swizzle(l16));
#pragma unroll
        for (int j = 0; j < 2; ++j)
            a_off[4 + j] = T::kRope + 8 * ((4 * j + g) ^ rope_swizzle(l16));
        // operand of K-step kk of row r of a slot
        auto a_at = [&](const E *slot, int r, int kk) -> E8 {
            return kk < 16 ? *(const E8 *)(slot + r * kDV + a_off[kk & 3] + 128 * (kk >> 2))
                           : *(const E8 *)(slot + r * (kDK - kDV) + a_off[kk - 12]);
        };
        // fp8 ring: the 8 bytes of K-step kk of row r (K = 32 kk + 8 g ..)
        auto a8_raw = [&](const unsigned char *slot8, int r, int kk) -> uint2 {
            const int ch = 2 * (kk & 15) + (g >> 1);  // 16-byte chunk within the C_N or rope part
            return kk < 16 ? *(const uint2 *)(slot8 + r * kDV + 16 * (ch ^ row_swizzle(r)) + 8 * (g & 1))
                           : *(const uint2 *)(slot8 + kF8Rope + r * (kDK - kDV) + 16 * (ch ^ ((r >> 2) & 3)) +
                                              8 * (g & 1));
        };
        // fp8 ring: the 32 bytes of C_N K-step kq (128 wide) of row r,
        // K = 128 kq + 32 g .. +31: stored chunks (8 kq + 2 g, +1) ^ (r mod 16)
        // (the swizzle permutes aligned groups of 16 chunks: two per-lane
        // offsets, by kq & 1, and immediates)
        auto a8_wide = [&](const unsigned char *slot8, int r, int kq) -> intx8 {
            const int c0 = 8 * (kq & 1) + 2 * g;
            const unsigned char *row = slot8 + r * kDV + 256 * (kq >> 1);
            const uint4 x = *(const uint4 *)(row + 16 * (c0 ^ row_swizzle(r)));
            const uint4 y = *(const uint4 *)(row + 16 * ((c0 + 1) ^ row_swizzle(r)));
            return intx8{(int)x.x, (int)x.y, (int)x.z, (int)x.w, (int)y.x, (int)y.y, (int)y.z, (int)y.w};
        };

#ifdef MLA_TIMELINE
        int tl_blocks = 0, tl_pieces = 0;  // the workgroup's blocks and pieces over its chunk
#endif
        for_each_piece([&](int b, int seq_lo, int p_org, int p_lo, int p_hi) {
            const int slot_out = split + b;
            const int nblk = (p_hi - p_org + T::kBT - 1) / T::kBT;
#ifdef MLA_TIMELINE
            tl_blocks += nblk;
            ++tl_pieces;
            MLA_STAMP(0, 14, tl_blocks);
            MLA_STAMP(0, 15, tl_pieces);
#endif
            piece_prologue(b, seq_lo, p_org, p_hi);
            MLA_STAMP(0, 1, MLA_RT());
            lds_barrier();  // A: Q* (split, with kF8M) and block 0 have landed
            MLA_STAMP(0, 2, MLA_RT());
            // Q* fragments (B operand of S^T = C Q*^T): lane holds head
            // kSH*hg + 16*ns + l16 of the tile, dims 32*kk + 8*g .. +7. Q*
            // rows sit in the ring in the same swizzled layout as C rows.
            E8 qf[kF8M ? 1 : T::kNS][kF8M ? 1 : kDK / 32];
            // fp8 cache: lane holds head kSH*hg + 16*ns + l16, C_N dims
            // 128 kq + 32 g .. +31 (qh / ql) and rope dims 32 rk + 8 g .. +7
            // (qrh / qrl); qsc = scale_log2 * 2^-e of that head
            intx8 qh[kF8M ? T::kNS : 1][4], ql[kF8M ? T::kNS : 1][4];
            uint2 qrh[kF8M ? T::kNS : 1][2], qrl[kF8M ? T::kNS : 1][2];
            float qsc[T::kNS];
            {
                // head h of the tile is row h % 32 of Q* slot kPre + h / 32
#pragma unroll
                for (int ns = 0; ns < T::kNS; ++ns) {
                    const int h = T::kSH * hg + 16 * ns + l16;
                    const E *qs = s_ring + (T::kPre + h / 32) * T::kSlot;
                    if constexpr (kF8M) {
                        // the split Q* (q_split_lds): hi / lo chunks
                        // 8 kq + 2 g, +1 of the row's C_N kilobyte and rope
                        // units 4 rk + g
                        const int rr = h % 32;
                        const unsigned char *q8 = reinterpret_cast<const unsigned char *>(qs + rr * kDV);
                        const unsigned char *r8 =
                            reinterpret_cast<const unsigned char *>(qs + T::kRope + rr * (kDK - kDV));
#pragma unroll
                        for (int kq = 0; kq < 4; ++kq) {
                            const int c0 = 8 * kq + 2 * g;
                            const uint4 h0 = *(const uint4 *)(q8 + 16 * (c0 ^ (rr & 15)));
                            const uint4 h1 = *(const uint4 *)(q8 + 16 * ((c0 + 1) ^ (rr & 15)));
                            const uint4 l0 = *(const uint4 *)(q8 + 512 + 16 * (c0 ^ (rr & 15)));
                            const uint4 l1 = *(const uint4 *)(q8 + 512 + 16 * ((c0 + 1) ^ (rr & 15)));
                            qh[ns][kq] = intx8{(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w,
                                               (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
                            ql[ns][kq] = intx8{(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w,
                                               (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
                        }
#pragma unroll
                        for (int rk = 0; rk < 2; ++rk) {
                            const int o = 8 * ((4 * rk + g) ^ ((rr >> 1) & 7));
                            qrh[ns][rk] = *(const uint2 *)(r8 + o);
                            qrl[ns][rk] = *(const uint2 *)(r8 + 64 + o);
                        }
                        qsc[ns] = s_qsc[h];
                    } else {
                        qsc[ns] = scale_log2;
#pragma unroll
                        for (int kk = 0; kk < kDK / 32; ++kk)
                            qf[ns][kk] = a_at(qs, h % 32, kk);
                    }
                }
            }
            lds_barrier();  // B: the Q* slots are free again
            MLA_STAMP(0, 3, MLA_RT());
            MLA_STAMP(0, 6, MLA_MT());

            float m_run[T::kNS], l_lane[T::kNS];  // running max (uniform over g); per-lane partial sum
#pragma unroll
            for (int ns = 0; ns < T::kNS; ++ns) {
                m_run[ns] = -INFINITY;
                l_lane[ns] = 0.f;
            }
            for (int t = -1; t < nblk; ++t) {
                if (t + 1 < nblk) {
                    const int blk = t + 1;
                    const int t0 = p_org + blk * T::kBT + 16 * th;
                    const E *cslot = s_ring + (blk % T::kRing) * T::kSlot;
                    // ---- S^T tiles: tokens t0 + (0..15), heads of this wave.
                    // The 18 operand reads go out in batches of 3 K-steps,
                    // two batches ahead of the MFMAs that consume them.
                    floatx4 acc[T::kNS][T::kChains];
#pragma unroll
                    for (int ns = 0; ns < T::kNS; ++ns)
#pragma unroll
                        for (int j = 0; j < T::kChains; ++j)
                            acc[ns][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                    if constexpr (kF8M) {
                        // 4 C_N K-steps of 128 (operand reads one step
                        // ahead of their MFMAs) and 2 rope K-steps of 32;
                        // chain 2j (+ 1): products with hi (lo)
                        const unsigned char *cslot8 = ring8 + (blk % T::kRing) * (T::kSlot * 2);
                        const int rr = 16 * th + l16;
                        auto hc = [](int k) { return T::kChains == 2 ? 0 : 2 * (k & 1); };
                        intx8 aw[2];
                        uint2 ar[2];
                        aw[0] = a8_wide(cslot8, rr, 0);
#pragma unroll
                        for (int kq = 0; kq < 4; ++kq) {
                            if (kq + 1 < 4)
                                aw[(kq + 1) & 1] = a8_wide(cslot8, rr, kq + 1);
                            if (kq == 3) {
                                ar[0] = a8_raw(cslot8, rr, 16);
                                ar[1] = a8_raw(cslot8, rr, 17);
                            }
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int ns = 0; ns < T::kNS; ++ns) {
                                acc[ns][hc(kq)] = mfma16x16x128_fp8(aw[kq & 1], qh[ns][kq], acc[ns][hc(kq)]);
                                acc[ns][hc(kq) + 1] = mfma16x16x128_fp8(aw[kq & 1], ql[ns][kq], acc[ns][hc(kq) + 1]);
                            }
                            __builtin_amdgcn_sched_barrier(0);
                        }
#pragma unroll
                        for (int rk = 0; rk < 2; ++rk) {
#pragma unroll
                            for (int ns = 0; ns < T::kNS; ++ns) {
                                acc[ns][hc(rk)] = mfma16x16x32_fp8(ar[rk], qrh[ns][rk], acc[ns][hc(rk)]);
                                acc[ns][hc(rk) + 1] = mfma16x16x32_fp8(ar[rk], qrl[ns][rk], acc[ns][hc(rk) + 1]);
                            }
                        }
                    } else {
                    // 18 K-steps of 32; the operand reads go out in batches
                    // of 3 K-steps, two batches ahead of the MFMAs that
                    // consume them
                    constexpr int kB = 3;                 // K-steps per batch
                    constexpr int kNB = kDK / 32 / kB;    // batches (6)
                    using AB = typename std::conditional<kF8, uint2, E8>::type;
                    AB ab[3][kB];
                    const unsigned char *cslot8 = ring8 + (blk % T::kRing) * (T::kSlot * 2);
                    auto load_batch = [&](int buf, int k0) {
#pragma unroll
                        for (int k = 0; k < kB; ++k) {
                            if constexpr (kF8)
                                ab[buf][k] = a8_raw(cslot8, 16 * th + l16, k0 + k);
                            else
                                ab[buf][k] = a_at(cslot, 16 * th + l16, k0 + k);
                        }
                    };
                    load_batch(0, 0);
                    load_batch(1, kB);
                    // fp8 (16-head tiles): each K-step's operand is
                    // converted to fp16 one K-step ahead, into the other of
                    // two register sets, so that the conversions run while
                    // the previous MFMAs do (one set made every conversion
                    // wait for the MFMAs before it to read their operand,
                    // and every MFMA for its operand)
                    E8 cv[2];
                    if constexpr (kF8)
                        cv[0] = f8_to_f16(ab[0][0]);
#pragma unroll
                    for (int bi = 0; bi < kNB; ++bi) {
                        if (bi + 2 < kNB)
                            load_batch((bi + 2) % 3, (bi + 2) * kB);
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int k = 0; k < kB; ++k) {
                            E8 a;
                            if constexpr (kF8) {
                                const int j = bi * kB + k;  // K-step
                                a = cv[j & 1];
                                if (j + 1 < kDK / 32)
                                    cv[(j + 1) & 1] = f8_to_f16(ab[((j + 1) / kB) % 3][(j + 1) % kB]);
                            } else {
                                a = ab[bi % 3][k];
                            }
#pragma unroll
                            for (int ns = 0; ns < T::kNS; ++ns) {
                                const int kk = bi * kB + k;
                                acc[ns][kk % T::kChains] = mfma16x16x32(a, qf[ns][kk], acc[ns][kk % T::kChains]);
                            }
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    }
                    // ---- online softmax of this wave's 16 tokens, per head
#pragma unroll
                    for (int ns = 0; ns < T::kNS; ++ns) {
                        floatx4 st;
                        if constexpr (kF8M) {
                            floatx4 sh = acc[ns][0], sl = acc[ns][1];
#pragma unroll
                            for (int j = 2; j < T::kChains; j += 2) {
                                sh += acc[ns][j];
                                sl += acc[ns][j + 1];
                            }
                            st = sh + sl * 0.0625f;
                        } else {
                            st = acc[ns][0];
#pragma unroll
                            for (int j = 1; j < T::kChains; ++j)
                                st += acc[ns][j];
                        }
                        float sv[4];
                        float mx = -INFINITY;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int tok = t0 + 4 * g + i;
                            const bool valid = kPaged ? (tok >= p_lo && tok < p_hi) : tok < p_hi;
                            sv[i] = valid ? st[i] * qsc[ns] : -INFINITY;
                            mx = fmaxf(mx, sv[i]);
                        }
                        mx = max_over_lane_groups(mx);
                        const float mn = fmaxf(m_run[ns], mx);
                        // a half with no valid token yet keeps max -inf; its
                        // exponents are taken against 0 so that they are 0
                        const float ref = mn == -INFINITY ? 0.f : mn;
                        const float alpha = fast_exp2(m_run[ns] - ref);
                        m_run[ns] = mn;
                        E4 ph;
                        float ps = 0.f;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float p = fast_exp2(sv[i] - ref);
                            ps += p;
                            ph[i] = (E)p;
                        }
                        l_lane[ns] = l_lane[ns] * alpha + ps;
                        const int hrow = T::kSH * hg + 16 * ns + l16;
                        // P columns in the O waves' K order: within each
                        // 8-token group, column j holds token 2j (j < 4) or
                        // 2(j - 4) + 1. This lane's tokens 4(g & 1) + i of
                        // group g >> 1 land in columns (i, i + 2) -> base,
                        // base + 1 and base + 4, base + 5.
                        if constexpr (kF8) {
                            // the fp8 ring's transpose reads take the K (token)
                            // order natural: tokens 4g .. 4g+3 of this half
                            *(E4 *)(s_p[blk & 1] + hrow * T::kPRow + 16 * th + 4 * g) = ph;
                        } else {
                            E *pw = s_p[blk & 1] + hrow * T::kPRow + 16 * th + 8 * (g >> 1) + 2 * (g & 1);
                            using E2 = E __attribute__((ext_vector_type(2)));
                            *(E2 *)pw = E2{ph[0], ph[2]};
                            *(E2 *)(pw + 4) = E2{ph[1], ph[3]};
                        }
                        if (g == 0)
                            s_m[blk & 1][m_at(hrow, th)] = mn;
                    }
                }
                if (t + 2 < T::kPre)
                    prologue_wait(t);
                lds_barrier();
            }
            MLA_STAMP(0, 4, MLA_RT());
            MLA_STAMP(0, 7, MLA_MT());
            // ---- epilogue: this half's running max and sum per head; the
            // first half merges both and writes the piece's m and l (the
            // LDS addresses formed here from an opaque copy of the lane, not
            // kept live, or spilled, through the piece)
            int el16 = l16;
            asm volatile("" : "+v"(el16));
#pragma unroll
            for (int ns = 0; ns < T::kNS; ++ns) {
                const float ls = sum_over_lane_groups(l_lane[ns]);
                if (g == 0) {
                    s_m[0][m_at(T::kSH * hg + 16 * ns + el16, th)] = m_run[ns];
                    s_l[th][T::kSH * hg + 16 * ns + el16] = ls;
                }
            }
            lds_barrier();
            if (!kDirect && th == 0 && g == 0) {
#pragma unroll
                for (int ns = 0; ns < T::kNS; ++ns) {
                    const int h = T::kSH * hg + 16 * ns + l16;
                    // the partial's max is the O waves' reference (finite, at
                    // most kLazyRescale below the halves' maxima), so that m, l
                    // and O share one scale
                    const float mr = s_mref[h];
                    const float ls = s_l[0][h] * fast_exp2(s_m[0][m_at(h, 0)] - mr) + s_l[1][h] * fast_exp2(s_m[0][m_at(h, 1)] - mr);
                    float *const mp = m_part + (size_t)slot_out * num_heads + head0 + h;
                    float *const lp = l_part + (size_t)slot_out * num_heads + head0 + h;
                    if (part_plain) {
                        *mp = mr;
                        *lp = ls;
                    } else {
                        store_nt(mp, mr);
                        store_nt(lp, ls);
                    }
                }
            }
#ifdef MLA_TIMELINE
            MLA_WAIT_VMCNT(0);
#endif
            MLA_STAMP(0, 5, MLA_RT());
        });
    } else {
        // ---- global -> LDS feeding of the ring. kFeeders waves share each
        // block: feeder d owns rows [kFeedRows*d, +kFeedRows): one load unit
        // (1 KB) per row for the C_N part (lane = stored chunk position; it
        // fetches logical chunk lane ^ row_swizzle(row)) and one per 8 rows
        // for the rope part (lane -> row 8*ru + lane/8, stored position
        // lane % 8). The O waves feed at HT = 64; otherwise waves 2 and 3,
        // which have no other role, do.
        const int feeder = wave - T::kFeedWave0;
        // fp8: 64-lane units of two C_N rows (and, with the 16 rows of a
        // dedicated feeder, of 16 rope rows), about half the load
        // instructions per block
        constexpr bool kFeedPairs = kF8;
        constexpr int kFU = kFeedPairs ? T::kFeedRows / 2 + 1 : T::kFeedUnits;  // units per feeder and block
        static_assert(!kFeedPairs || T::kFeedRows == 16 || T::kFeedRows == 8, "paired fp8 units");
        // unit k (0..kFeedUnits-1) of this feeder's share of a block: C_N
        // row kFeedRows*feeder + k, or a rope unit of those rows; uoff[k] is
        // its lane offset (16-bit caches)
        int uoff[kFeedPairs ? 1 : kFU];
        if constexpr (!kF8) {
#pragma unroll
            for (int k = 0; k < kFU; ++k)
                uoff[k] = k < T::kFeedRows ? feed_off(T::kFeedRows * feeder + k, false)
                                           : feed_off((T::kFeedRows / 8) * feeder + (k - T::kFeedRows), true);
        }
        auto load_unit = [&](const void *base, int lim, int slot, int k) {
            if constexpr (kFeedPairs) {
                // fp8, dedicated feeders: row pairs, then one 16-row rope unit
                const unsigned char *b8 = static_cast<const unsigned char *>(base);
                if (k < T::kFeedRows / 2)
                    dma_row8x2(b8, lim, slot, T::kFeedRows * feeder + 2 * k);
                else
                    if constexpr (T::kFeedRows == 16)
                        dma_rope8x16(b8, lim, slot, feeder);
                    else
                        dma_rope8(b8, lim, slot, feeder);
            } else if constexpr (kF8) {
                if (k < T::kFeedRows)
                    blk_row(base, lim, slot, T::kFeedRows * feeder + k);
                else
                    blk_rope(base, lim, slot, (T::kFeedRows / 8) * feeder + (k - T::kFeedRows));
            } else {
                const E *eb = static_cast<const E *>(base);
                if (k < T::kFeedRows)
                    feed_row(eb, lim, slot, T::kFeedRows * feeder + k, uoff[k]);
                else
                    feed_rope(eb, lim, slot, (T::kFeedRows / 8) * feeder + (k - T::kFeedRows), uoff[k]);
            }
        };
        // End of step t: block t+2 (the S waves' next) must have landed;
        // blocks t+3 and t+4 may stay in flight. At t = -1 those are the
        // prologue's blocks after block 1 (5 or 4 units each) and blocks
        // kPre..3, issued after barrier B.
        auto feed_wait = [&](bool issued, int t) {
            if (t < 0) {
                if (wave < 4)
                    MLA_WAIT_VMCNT(5 * (T::kPre - 2) + (T::kRing - T::kPre) * kFU);
                else if (T::kWaves == 8 || wave < 8)
                    MLA_WAIT_VMCNT(4 * (T::kPre - 2) + (T::kRing - T::kPre) * kFU);
                else  // no prologue loads of its own
                    MLA_WAIT_VMCNT((T::kRing - T::kPre) * kFU);
            } else if (issued) {
                MLA_WAIT_VMCNT(2 * kFU);
            } else {
                MLA_WAIT_VMCNT(0);
            }
        };

        if (wave >= T::kOWave0 && wave < T::kOWave0 + 4) {
            const int ow = wave - T::kOWave0;  // column quarter
            // When the O waves also feed the ring (HT = 64) they carry the
            // step: they issue first when both waves of a SIMD are ready, so
            // their P reads reach the LDS ahead of the S waves' operand reads.
            // With dedicated feeders the S waves carry the step and equal
            // priorities are best.
            if constexpr (T::kOFeeds)
                __builtin_amdgcn_s_setprio(2);
            // C_N^T operand of dims 128*ow + 16*dt .. +15 from a ring slot
            // fp8 ring: the raw bytes, converted where the MFMA takes them
            using AV = typename std::conditional<kF8, uint2, E8>::type;
            auto load_av = [&](const E *cs, int dt) -> AV {
                if constexpr (kF8) {
                    // lane (g, d): dim 128*ow + 16*dt + d of tokens 8g .. 8g+7
                    // (K order natural); 16-byte chunk ch of the C_N rows
                    const unsigned char *cs8 = reinterpret_cast<const unsigned char *>(cs);
                    const int ch = 8 * ow + dt;
                    if constexpr (kTr) {
                        const int tok = 8 * g + (l16 >> 1);
                        return lds_read_tr8(cs8 + tok * kDV + 16 * (ch ^ row_swizzle(tok)) + 8 * (l16 & 1));
                    } else {
                        unsigned w[2] = {0u, 0u};
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int tok = 8 * g + j;
                            w[j >> 2] |= (unsigned)cs8[tok * kDV + 16 * (ch ^ row_swizzle(tok)) + l16] << (8 * (j & 3));
                        }
                        return uint2{w[0], w[1]};
                    }
                } else if constexpr (kTr) {
                    // lane (g, j): K index 8g + j/4 (+4) is token row 8g + 2(j/4)
                    // (+1), dims 128*ow + 16*dt + 4*(j%4) .. +3
                    const int r0 = 8 * g + 2 * (l16 >> 2);
                    const int cl = 16 * ow + 2 * dt + ((l16 & 3) >> 1);
                    const int sub = 4 * (l16 & 1);
                    const E4 lo4 = lds_read_tr16<E>(cs + r0 * kDV + 8 * (cl ^ row_swizzle(r0)) + sub);
                    const E4 hi4 = lds_read_tr16<E>(cs + (r0 + 1) * kDV + 8 * (cl ^ row_swizzle(r0 + 1)) + sub);
                    return E8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                } else {
                    E8 v;
                    const int col = 128 * ow + 16 * dt + l16;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int r = 8 * g + (j < 4 ? 2 * j : 2 * j - 7);  // K order 8g + {0,2,4,6,1,3,5,7}
                        v[j] = cs[r * kDV + 8 * ((col >> 3) ^ row_swizzle(r)) + (col & 7)];
                    }
                    return v;
                }
            };

            for_each_piece([&](int b, int seq_lo, int p_org, int p_lo, int p_hi) {
                (void)p_lo;
                const int slot_out = split + b;
                const int nblk = (p_hi - p_org + T::kBT - 1) / T::kBT;
                // unit k of this wave's share of block blk; a block past the
                // last re-reads the last token only
                auto t0_of = [&](int blk) { return min(p_org + blk * T::kBT, p_hi - 1); };
                // unit k of this wave's share of block blk, whose first row is
                // at src; a block past the last re-reads the last token only
                auto issue_unit = [&](const void *src, int blk, int k) {
                    load_unit(src, p_hi - 1 - t0_of(blk), blk % T::kRing, k);
                };
                piece_prologue(b, seq_lo, p_org, p_hi);
                // a paged cache's block-table reads: blocks kPre..3 before
                // barrier B, then each step reads the page of the block the
                // next step issues, so that the scalar load lands during a
                // barrier (lds_barrier waits for it with the LDS counter)
                int rest[T::kRing - T::kPre];
                int next = 0;
                if constexpr (T::kOFeeds) {
#pragma unroll
                    for (int blk = T::kPre; blk < T::kRing; ++blk)
                        rest[blk - T::kPre] = page_of(b, seq_lo, t0_of(blk));
                    next = page_of(b, seq_lo, t0_of(T::kRing));
                }
                lds_barrier();  // A
                lds_barrier();  // B
                MLA_STAMP(4, 8, MLA_RT());
                MLA_STAMP(4, 12, MLA_MT());
                MLA_STAMP(4, 11, nblk);
                if constexpr (T::kOFeeds) {
#pragma unroll
                    for (int blk = T::kPre; blk < T::kRing; ++blk) {
                        const void *src = block_src(rest[blk - T::kPre], seq_lo, t0_of(blk));
#pragma unroll
                        for (int k = 0; k < kFU; ++k)
                            issue_unit(src, blk, k);
                    }
                }

                floatx4 o[T::kNHS][8];
                float m_ref[T::kNHS];  // per head l16 of sub-tile hs: the accumulator's reference max
#pragma unroll
                for (int hs = 0; hs < T::kNHS; ++hs) {
                    m_ref[hs] = -INFINITY;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt)
                        o[hs][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
                }
                // C_N^T fragments of the block the next step accumulates; each
                // step reloads them for its successor right after the MFMAs
                // that consume them
                AV av[8];
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
                    av[dt] = load_av(s_ring, dt);

                for (int t = -1; t < nblk; ++t) {
                    // block t+4 goes into the slot of block t, which every
                    // wave has finished reading (its C_N^T fragments are in av)
                    const bool issue = T::kOFeeds && t >= 0 && t + T::kRing < nblk;
                    // the page of block t+4 was read by the previous step
                    const void *isrc = issue ? block_src(next, seq_lo, t0_of(t + T::kRing)) : c;
                    if (t >= 0) {
                        const int blk = t;
                        // ---- common reference max of the two token halves; P
                        // of the half this lane feeds (tokens 8g..8g+7: half
                        // g/2) is scaled onto it, the accumulator moves by
                        // 2^(M_old - M)
                        E8 pb[T::kNHS];
                        float m0[T::kNHS], m1[T::kNHS];
                        {
                            const float *mrow = s_m[blk & 1] + m_at(l16, 0);
                            if constexpr (T::kNHS == 1) {
                                const float2 v = *(const float2 *)mrow;
                                m0[0] = v.x;
                                m1[0] = v.y;
                            } else {
#pragma unroll
                                for (int q = 0; q < T::kNHS / 2; ++q) {
                                    const floatx4 v = *(const floatx4 *)(mrow + 4 * q);
                                    m0[2 * q] = v[0];
                                    m1[2 * q] = v[1];
                                    m0[2 * q + 1] = v[2];
                                    m1[2 * q + 1] = v[3];
                                }
                            }
                        }
#pragma unroll
                        for (int hs = 0; hs < T::kNHS; ++hs)
                            pb[hs] = *(const E8 *)(s_p[blk & 1] + (16 * hs + l16) * T::kPRow + 8 * g);
                        // The reference only moves when a max passes it by more
                        // than kLazyRescale (P scaled onto it then stays <= 2^8,
                        // well inside fp16), so the rescale is rare.
                        float alpha[T::kNHS];
                        bool moved = false;
#pragma unroll
                        for (int hs = 0; hs < T::kNHS; ++hs) {
                            const float mn = fmaxf(m0[hs], m1[hs]);  // finite: token p_lo is in half 0
                            const bool up = mn > m_ref[hs] + kLazyRescale;  // always at the first block
                            alpha[hs] = up ? fast_exp2(m_ref[hs] - mn) : 1.0f;
                            moved |= up;
                            if (up)
                                m_ref[hs] = mn;
                            const float f = fast_exp2((g < 2 ? m0[hs] : m1[hs]) - m_ref[hs]);
                            if constexpr (__is_same(E, _Float16)) {
                                pb[hs] *= (E)f;
                            } else {
                                // bf16: scale in fp32, so that the factor is not
                                // itself rounded to 8 bits (one error for the
                                // whole half-block)
#pragma unroll
                                for (int i = 0; i < 8; ++i)
                                    pb[hs][i] = (E)((float)pb[hs][i] * f);
                            }
                        }
                        if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
                            for (int hs = 0; hs < T::kNHS; ++hs)
#pragma unroll
                                for (int dt = 0; dt < 8; ++dt)
                                    o[hs][dt] *= alpha[hs];
                        }
                        // the page of the block the next step issues: read after
                        // this step's P and max reads (a scalar load shares the
                        // LDS counter), waited for at the step's barrier
                        if (issue)
                            next = page_of(b, seq_lo, t0_of(t + T::kRing + 1));
                        // ---- O^T[dims 128*ow .. +128][heads] += C_N^T P^T, with
                        // the next block's operand reads (and, when the O
                        // waves feed, this step's global->LDS loads) placed
                        // between the MFMAs
                        const E *cn = s_ring + ((blk + 1) % T::kRing) * T::kSlot;
                        // fp8: operands converted one dim tile ahead, into two
                        // register sets (as in the S waves)
                        E8 cva[2];
                        if constexpr (kF8)
                            cva[0] = f8_to_f16(av[0]);
#pragma unroll
                        for (int dt = 0; dt < 8; ++dt) {
                            E8 a;
                            if constexpr (kF8) {
                                a = cva[dt & 1];
                                if (dt + 1 < 8)
                                    cva[(dt + 1) & 1] = f8_to_f16(av[dt + 1]);
                            } else {
                                a = av[dt];
                            }
#pragma unroll
                            for (int hs = 0; hs < T::kNHS; ++hs)
                                o[hs][dt] = mfma16x16x32(a, pb[hs], o[hs][dt]);
                            av[dt] = load_av(cn, dt);
                            if (issue && dt < kFU)
                                issue_unit(isrc, blk + T::kRing, dt);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                        if (issue) {
#pragma unroll
                            for (int k = 8; k < kFU; ++k)
                                issue_unit(isrc, blk + T::kRing, k);
                        }
                    }
                    if constexpr (T::kOFeeds)
                        feed_wait(issue, t);
                    else if (t + 2 < T::kPre)
                        prologue_wait(t);
                    lds_barrier();
                }
                MLA_STAMP(4, 9, MLA_RT());
                MLA_STAMP(4, 13, MLA_MT());
                if (g == 0) {
#pragma unroll
                    for (int hs = 0; hs < T::kNHS; ++hs)
                        if (ow == 0)
                            s_mref[16 * hs + l16] = m_ref[hs];
                }
                lds_barrier();  // epilogue barrier of the S waves
                // ---- epilogue: O of this piece normalised by its running sum
                // (the halves' sums moved onto the reference max, exactly as
                // the S waves compute the l they store), tile by tile
                // lane through an empty asm: the epilogue's addresses are formed
                // here, not hoisted into registers held across the block loop
                int eln = lane;
                asm volatile("" : "+v"(eln));
                const size_t obase = (size_t)slot_out * num_heads * kDV + eln * 4;
#pragma unroll
                for (int hs = 0; hs < T::kNHS; ++hs) {
                    const int h = 16 * hs + l16;
                    const float ls = s_l[0][h] * fast_exp2(s_m[0][m_at(h, 0)] - m_ref[hs]) +
                                     s_l[1][h] * fast_exp2(s_m[0][m_at(h, 1)] - m_ref[hs]);
                    const float inv = out_scale / ls;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) {
                        const floatx4 v = o[hs][dt] * inv;
                        const size_t off = obase + frag_offset(head0 + 16 * hs, 128 * ow + 16 * dt);
                        if constexpr (kDirect) {
                            // lane (g, h): dims 4g .. 4g+3 of head h of this 16-dim group
                            E *const orow = out + (size_t)(head0 + 16 * hs + (eln & 15)) * kDV + 128 * ow + 4 * (eln >> 4);
                            *(E4 *)(orow + 16 * dt) = E4{(E)v[0], (E)v[1], (E)v[2], (E)v[3]};
                        } else if constexpr (kF32Part) {
                            floatx4 *const op = (floatx4 *)((float *)o_part + off);
                            if (part_plain)
                                *op = v;
                            else
                                store_nt(op, v);
                        } else {
                            const E4 hv = {(E)v[0], (E)v[1], (E)v[2], (E)v[3]};
                            E4 *const op = (E4 *)((E *)o_part + off);
                            if (part_plain)
                                *op = hv;
                            else
                                store_nt8(op, hv);
                        }
                    }
                }
#ifdef MLA_TIMELINE
                MLA_WAIT_VMCNT(0);
#endif
                MLA_STAMP(4, 10, MLA_RT());
            });
        } else {
            // dedicated feeder waves (head tiles of 16 or 32 heads)
            for_each_piece([&](int b, int seq_lo, int p_org, int p_lo, int p_hi) {
                (void)p_lo;
                const int nblk = (p_hi - p_org + T::kBT - 1) / T::kBT;
                // first token of block blk; a block past the last re-reads
                // the last token only
                auto t0_of = [&](int blk) { return min(p_org + blk * T::kBT, p_hi - 1); };
                auto issue_block = [&](const void *src, int blk) {
                    const int lim = p_hi - 1 - t0_of(blk);
#pragma unroll
                    for (int k = 0; k < kFU; ++k)
                        load_unit(src, lim, blk % T::kRing, k);
                };
                piece_prologue(b, seq_lo, p_org, p_hi);
                // pages of blocks kPre..4, read before barrier B, and of each
                // later block one step before it is issued, so that a paged
                // cache's block-table reads arrive during a barrier
                int rest[T::kRing - T::kPre];
#pragma unroll
                for (int blk = T::kPre; blk < T::kRing; ++blk)
                    rest[blk - T::kPre] = page_of(b, seq_lo, t0_of(blk));
                int next = page_of(b, seq_lo, t0_of(T::kRing));
                lds_barrier();  // A
                lds_barrier();  // B
#pragma unroll
                for (int blk = T::kPre; blk < T::kRing; ++blk)
                    issue_block(block_src(rest[blk - T::kPre], seq_lo, t0_of(blk)), blk);
                for (int t = -1; t < nblk; ++t) {
                    // block t+4 into the slot of block t
                    const bool issue = t >= 0 && t + T::kRing < nblk;
                    if (issue) {
                        issue_block(block_src(next, seq_lo, t0_of(t + T::kRing)), t + T::kRing);
                        next = page_of(b, seq_lo, t0_of(t + T::kRing + 1));
                    }
                    feed_wait(issue, t);
                    lds_barrier();
                }
                lds_barrier();  // epilogue barrier of the S waves
            });
        }
    }

}

template <int HT, bool kTr, typename E, bool kPaged, bool kF32Part, bool kF8, int kMode>
hipError_t launch_ht(const Problem &pb, const Plan &p, const Partials &w, hipStream_t s)
{
    const dim3 grid(grid_chunks(p) * p.n_head_tiles), block(F16Tile<HT>::kThreads);
    hipLaunchKernelGGL((splitkv_fp16_kernel<HT, kTr, E, kPaged, kF32Part, kF8, kMode>), grid, block, 0, s,
                       (const E *)pb.q, (const E *)pb.c, pb.cu_seqlens, pb.num_heads, pb.batch, pb.total_tokens,
                       p.chunk, p.n_head_tiles, p.xcd_remap, w.o, w.m, w.l, pb.scale_log2, pb.paging, pb.out_scale,
                       (E *)pb.out, p.part_plain, p.seq_cost);
    // the launch's own error; hipPeekAtLastError leaves a sticky error from
    // the caller's earlier work in place for the caller to see
    return hipPeekAtLastError();
}

// one instantiation per head tile of a (cache type, partials, mode) combination
template <bool kTr, typename E, bool kPaged, bool kF32Part, bool kF8, int kMode = kModeBatch>
hipError_t launch_tiles(const Problem &pb, const Plan &p, const Partials &w, hipStream_t s)
{
    switch (p.head_tile) {
    case 64: return launch_ht<64, kTr, E, kPaged, kF32Part, kF8, kMode>(pb, p, w, s);
    case 32: return launch_ht<32, kTr, E, kPaged, kF32Part, kF8, kMode>(pb, p, w, s);
    case 16: return launch_ht<16, kTr, E, kPaged, kF32Part, kF8, kMode>(pb, p, w, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

#ifdef MLA_TIMELINE
extern "C" int mla_timeline_read(void *dst, size_t bytes)
{
    const size_t n = bytes < sizeof(mla_timeline_stamps) ? bytes : sizeof(mla_timeline_stamps);
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(mla_timeline_stamps), n, 0, hipMemcpyDeviceToHost);
}
#endif

hipError_t launch_splitkv_fp16(const Problem &pb, const Plan &p, const Partials &w,
                               bool tr_load, hipStream_t s)
{
    if (p.n_chunks == 0)
        return hipSuccess;
    const bool f32_part = p.part_bytes == 4;
    if (p.merge == kMergeDirect) {
        // one chunk of a single sequence, packed cache: the output directly
        // (the partial precision does not matter: none are stored)
        if (!tr_load || pb.paging.block_table || pb.cu_seqlens || p.n_chunks != 1 || !pb.out)
            return hipErrorInvalidValue;
        if (pb.fp8)
            return launch_tiles<true, _Float16, false, false, true, kModeDirect>(pb, p, w, s);
        return pb.bf16 ? launch_tiles<true, __bf16, false, false, false, kModeDirect>(pb, p, w, s)
                       : launch_tiles<true, _Float16, false, false, false, kModeDirect>(pb, p, w, s);
    }
    // one sequence (no cu_seqlens): kModeSingle, with the prologue loads at
    // kernel entry; batches: kModeBatch
    const bool single = pb.cu_seqlens == nullptr;
    // The scalar transpose reads and fp32 partials are options of the packed
    // fp16 entry points (their flags); the bf16, paged and fp8 caches are
    // built with the LDS transpose read and 16-bit partials only. The scalar
    // transpose reads (a testing aid) are built in kModeBatch only, which
    // also serves a single sequence.
    if (!pb.bf16 && !pb.fp8 && !pb.paging.block_table) {
        if (tr_load && single)
            return f32_part ? launch_tiles<true, _Float16, false, true, false, kModeSingle>(pb, p, w, s)
                            : launch_tiles<true, _Float16, false, false, false, kModeSingle>(pb, p, w, s);
        if (tr_load)
            return f32_part ? launch_tiles<true, _Float16, false, true, false>(pb, p, w, s)
                            : launch_tiles<true, _Float16, false, false, false>(pb, p, w, s);
        return f32_part ? launch_tiles<false, _Float16, false, true, false>(pb, p, w, s)
                        : launch_tiles<false, _Float16, false, false, false>(pb, p, w, s);
    }
    if (!tr_load || f32_part)
        return hipErrorInvalidValue;
    if (pb.fp8)  // fp16 query, fp8 cache, fp16 partials
        return single ? launch_tiles<true, _Float16, false, false, true, kModeSingle>(pb, p, w, s)
                      : launch_tiles<true, _Float16, false, false, true>(pb, p, w, s);
    if (pb.paging.block_table)
        return pb.bf16 ? launch_tiles<true, __bf16, true, false, false>(pb, p, w, s)
                       : launch_tiles<true, _Float16, true, false, false>(pb, p, w, s);
    return single ? launch_tiles<true, __bf16, false, false, false, kModeSingle>(pb, p, w, s)
                  : launch_tiles<true, __bf16, false, false, false>(pb, p, w, s);
}

}  // namespace mla
