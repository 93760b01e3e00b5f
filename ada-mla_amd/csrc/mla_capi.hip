// C ABI of the MLA decode library (declared in include/mla_mi355x.h):
// argument validation, split planning, workspace carving and the two
// launches (split kernel, then combine) on the caller's stream.
#include "mla_mi355x.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <mutex>

#include "mla_internal.hpp"

// Split partials of mla_decode_split_fp16_noalloc: a file-scope device array
// of MLA_NOALLOC_SCRATCH_BYTES, one copy per GPU, held until the process ends.
// Its name is a host-side stand-in: host code uses the device address that
// hipGetSymbolAddress returns for the current device (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[MLA_NOALLOC_SCRATCH_BYTES];

namespace mla {
namespace {

thread_local int t_last_hip_error = 0;

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

}  // namespace

// CUs of the current device (cached); 256 (MI355X) if it cannot be queried.
int current_cu_count()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return 256;
    int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n > 0)
        return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    g_cu_count[dev].store(n, std::memory_order_relaxed);
    return n;
}

namespace {

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// fp32 path: smallest token count worth a split of its own (two 16-token
// blocks; with one, the fp32 partial write-back about equals the C bytes the
// split reads). Measured at 128 heads, N = 1024: 16.7 us per call with
// 32-token splits (256 workgroups), 18.4 us with 64-token splits (128).
// Re-measured on the current kernel (one box, us per call, 16 / 20 / 24 /
// 28 / 32 splits): N = 1024 13.94 / 13.92 / 13.55 / 13.55 / 13.53; N = 2048
// (16, 24, 32) 20.5 / 18.6 / 16.9; N = 4096 (24, 28, 32) 26.6 / 25.4 / 23.3.
constexpr int kMinSplitTokensF32 = 32;

// fp32 path: 32-head workgroups once their chunks hold this many tokens (12
// blocks). Measured per call on one box (16 / 32 heads per workgroup, the
// planner's split counts): n_h = 128, N = 4096 24.5 / 29.9 us, N = 8192
// 36.0 / 38.1, N = 12288 45.6 / 45.4 (192-token chunks at 32 heads),
// N = 16384 57.3 / 55.4; n_h = 64, N = 8192 23.9 / 27.6, N = 32768 57.4 /
// 55.4; n_h = 32, N = 16384 22.3 / 26.0.
constexpr int kHt32MinChunkTokensF32 = 192;

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

float scale_log2()
{
    // softmax scale 1/sqrt(192) (mla.py:46) folded with log2(e): the kernels
    // exponentiate with exp2.
    return (float)(1.4426950408889634 / std::sqrt(192.0));
}

int fail_hip(hipError_t e) { return record_hip_error(e); }

}  // namespace

int record_hip_error(hipError_t e)
{
    t_last_hip_error = (int)e;
    return MLA_STATUS_HIP_ERROR;
}

namespace {

// Chunking of total_tokens into about `w` chunks of whole blocks.
void set_chunks(Plan &p, int total_tokens, int batch, int w)
{
    w = std::max(1, std::min(w, ceil_div(total_tokens, p.block_tokens)));
    p.chunk = ceil_div(ceil_div(total_tokens, w), p.block_tokens) * p.block_tokens;
    p.n_chunks = ceil_div(total_tokens, p.chunk);
    p.n_slots = p.n_chunks + batch - 1;
    // the launch grid is padded to a multiple of 8 chunks (the padding
    // workgroups exit at once), so the head tiles of every chunk can share
    // an XCD whatever n_chunks is
    p.xcd_remap = 1;
}

#ifndef MLA_PIECE_TOKENS_64
#define MLA_PIECE_TOKENS_64 192
#endif
// Calls with cu_seqlens: what starting a piece (one sequence's part of a
// chunk: its Q* and first blocks loaded, the pipeline filled, its partial
// stored) costs, in tokens of steady-state work at each head tile. Chunks
// are cut over a virtual length in which every sequence start counts this
// many tokens, so a chunk that holds more pieces holds fewer tokens.
// Measured at 64-head tiles (config 5, B = 32): chunks of one, two and
// three pieces took 64, 71 and 76 us with equal token counts.
int piece_cost_tokens(int head_tile)
{
    return head_tile == 64 ? MLA_PIECE_TOKENS_64 : head_tile == 32 ? 224 : 288;
}

// Fixed cost (us) of a one-launch call (one chunk, the split kernel writes
// the output): the two-launch fixed cost below less the combine launch.
constexpr double kDirectFixedUs = 7.0;

// Modelled time of one 16-bit decode call (us) for a plan, fitted to MI355X
// measurements of this library (forced plans over head tile, split count and
// partial precision): a fixed cost per call (two launches, the prologue, the
// partial store); the split kernel's block loop, one 32-token step per block
// plus one at a step time that grows with the head tile (64: 1.5 us, 32:
// 0.88 us, 16: 0.65 us with every CU busy), but no shorter than the HBM
// time of every chunk in flight streaming its block at once
// (kStreamBytesPerUs); the partial round trip (written, then read by the
// combine) at ~8 TB/s; and the combine's memory round trips. Head tiles that
// share a chunk but not an XCD (xcd_remap 0, which the planner no longer
// produces) would re-read C from HBM; the model charges that as slower
// steps.
// The stream term is per block: a plan with fewer chunks than CUs streams C
// with fewer CUs and is not HBM-bound until each block's share reaches the
// step. Against a floor over the whole call (C at 6 TB/s), which made every
// split count past the floor look alike and favoured the fewest partials,
// it moved 13 of 156 plans (n_h 16 and 32, N >= 32768), all faster on one
// box: n_h = 16, N = 65536 114 -> 137 splits 22.9 -> 20.3 us, N = 262144
// 108 -> 139 splits 71.3 -> 58.5 us; n_h = 32, N = 65536 114 -> 128 splits
// 23.1 -> 20.8 us, N = 262144 (16, 108) -> (32, 179) 71.2 -> 59.0 us.
constexpr double kStreamBytesPerUs = 7.5e6;  // n_h = 16 streams C at 7.7 TB/s in the steady state
double modelled_us(const Plan &p, int num_heads, int total_tokens, int batch, int cu_count, bool paged,
                   bool direct_ok, int c_bytes)
{
    // one chunk of a single sequence: one launch, no partials, no combine
    if (direct_ok && p.n_chunks == 1)
        return kDirectFixedUs + (std::ceil((double)p.chunk / p.block_tokens) + 1.0) *
                                    (p.head_tile == 64 ? 1.5 : p.head_tile == 32 ? 0.88 : 0.65);
    const double step_us = p.head_tile == 64 ? 1.5 : p.head_tile == 32 ? 0.88 : 0.65;
    const int wgs = p.n_chunks * p.n_head_tiles;
    const double rounds = std::ceil((double)wgs / cu_count);
    const double steps = std::ceil((double)p.chunk / p.block_tokens) + (paged ? 2.0 : 1.0);
    const double share = (p.n_head_tiles > 1 && !p.xcd_remap) ? 1.3 : 1.0;
    const double partial_bytes = (double)p.n_slots * num_heads * (kDV * p.part_bytes + 8);
    // the combine merges up to 128 slots of a tile per memory round trip
    // (256 in quarter items: fewer items than CUs, or fp32 partials)
    const double slots_per_seq = std::ceil((double)p.n_slots / batch);
    const bool quarter = num_heads / 16 * (kDV / 16) * batch < cu_count || p.part_bytes == 4;
    const double combine_trips = std::ceil(slots_per_seq / (quarter ? 256.0 : 128.0));
    // a block takes its step, but no less than the HBM time of every chunk
    // in flight streaming its block at once (the head tiles of a chunk read
    // it from one L2); c_bytes: bytes per cache element (1 for fp8)
    const double chunks_live = std::min((double)wgs, (double)cu_count) / p.n_head_tiles;
    const double block_us = std::max(step_us * share, chunks_live * p.block_tokens * kDK * c_bytes / kStreamBytesPerUs);
    const double loop_us = rounds * steps * block_us;
    return 11.0 + loop_us + 0.25e-6 * partial_bytes + 1.0 * combine_trips;
}

}  // namespace

namespace {

Plan compute_plan(bool fp32, int num_heads, int total_tokens, int batch, bool seqlens,
                  int num_splits, int cu_count, CacheKind cache, bool f32_partials)
{
    const bool paged = cache == CacheKind::kPaged;  // pieces start page-aligned: one more block
    Plan p{};
    if (total_tokens <= 0) {
        p.head_tile = fp32 ? 16 : (num_heads % 64 == 0) ? 64 : (num_heads % 32 == 0) ? 32 : 16;
        p.block_tokens = fp32 ? 16 : 32;
        p.n_head_tiles = num_heads / p.head_tile;
        p.chunk = p.block_tokens;
        p.n_chunks = 0;
        p.n_slots = batch;  // unused; keeps the workspace non-empty
        p.xcd_remap = 0;
        p.seq_cost = 0;
        p.part_bytes = (fp32 || f32_partials) ? 4 : 2;
        return p;
    }
    if (fp32) {
        p.block_tokens = 16;
        // one workgroup per CU (the kernel's LDS holds one) unless the split
        // count is given
        auto splits_for = [&](int ht) {
            if (num_splits > 0)
                return num_splits;
            const int per_round = std::max(1, cu_count / (num_heads / ht));
            return std::min(per_round, ceil_div(total_tokens, kMinSplitTokensF32));
        };
        // 32 heads per workgroup fill each C block once for twice the heads,
        // but take twice the chunks' partials and half the chunks: they pay
        // where their chunks hold at least kHt32MinChunkTokensF32 tokens.
        p.head_tile = 16;
        if (num_heads % 32 == 0 && ceil_div(total_tokens, splits_for(32)) >= kHt32MinChunkTokensF32)
            p.head_tile = 32;
        p.n_head_tiles = num_heads / p.head_tile;
        const int w = splits_for(p.head_tile);
        set_chunks(p, total_tokens, batch, w);
        p.part_bytes = 4;
        return p;
    }
    // fp16: the head tile (64, 32 or 16 heads per workgroup) and the split
    // count with the smallest modelled call time, at most one workgroup per
    // CU; a requested split count fixes the chunking and only the tile is
    // chosen. Chosen splits leave chunks of at least two blocks once there
    // are 32 blocks (a one-block chunk overlaps no load with compute: on
    // MI355X the 19 plans this moved, n_h = 16 .. 128, N = 1024 .. 4096, ran
    // x0.962 by geomean, 13 faster by more than 2%, one 2.7% slower; at
    // N = 512 it was a wash).
    // min_blocks(ht): the shortest chunk (in blocks) the search takes;
    // c_bytes: bytes per cache element for the stream term.
    auto search = [&](int c_bytes, auto min_blocks, double &best_us) {
        Plan best{};
        best_us = 0.0;
        for (int ht : {64, 32, 16}) {
            if (num_heads % ht != 0)
                continue;
#ifdef MLA_TIMELINE
            // timeline build only (ada-mla_amd/timeline.py): MLA_TIMELINE_HEAD_TILE pins the tile
            if (const char *e = std::getenv("MLA_TIMELINE_HEAD_TILE"); e && std::atoi(e) != ht)
                continue;
#endif
            Plan c{};
            c.head_tile = ht;
            c.block_tokens = 32;
            c.n_head_tiles = num_heads / ht;
            c.part_bytes = f32_partials ? 4 : 2;
            // with cu_seqlens the chunks split the virtual length (piece_cost_tokens)
            // (plain token chunks if the virtual length would not fit an int)
            c.seq_cost = seqlens ? piece_cost_tokens(ht) : 0;
            if ((long long)total_tokens + (long long)c.seq_cost * batch > INT32_MAX / 2)
                c.seq_cost = 0;
            const int total_v = total_tokens + c.seq_cost * batch;
            const int blocks = ceil_div(total_v, c.block_tokens);
            int w_lo = 1, w_hi = std::max(1, std::min(cu_count / c.n_head_tiles, blocks / min_blocks(ht, blocks)));
            if (num_splits > 0)
                w_lo = w_hi = num_splits;
            for (int w = w_lo; w <= w_hi; ++w) {
                set_chunks(c, total_v, batch, w);
                const double us = modelled_us(c, num_heads, total_tokens, batch, cu_count, paged,
                                              !seqlens && cache != CacheKind::kPaged, c_bytes);
                if (best_us == 0.0 || us < best_us) {
                    best = c;
                    best_us = us;
                }
            }
        }
        return best;
    };
    double us16 = 0.0;
    Plan p16 = search(2, [](int, int blocks) { return blocks >= 32 ? 2 : 1; }, us16);
    // A plan whose blocks wait on HBM (the stream term above the step) takes
    // every CU with its head tile: the model charges the stream at a fixed
    // rate, so it stops at the fewest chunks that reach it, but more CUs keep
    // more loads in flight and pull C faster. Measured on MI355X: n_h = 16,
    // N = 131072 137 -> 256 chunks 33.5 -> 31.6 us; batches of 16 heads 5-10%
    // faster (config 5's lengths 60.3 -> 54.5 us); 32 and 48 heads within 2%.
    if (num_splits == 0 && p16.n_chunks > 1) {
        const double step_us = p16.head_tile == 64 ? 1.5 : p16.head_tile == 32 ? 0.88 : 0.65;
        const double live = std::min((double)p16.n_chunks * p16.n_head_tiles, (double)cu_count) / p16.n_head_tiles;
        if (live * p16.block_tokens * kDK * 2 / kStreamBytesPerUs > step_us)
            set_chunks(p16, total_tokens + p16.seq_cost * batch, batch, std::max(1, cu_count / p16.n_head_tiles));
    }
    if (cache != CacheKind::kF8 || num_splits > 0)
        return p16;
    // fp8 cache: its blocks stream half the bytes, so with few heads more
    // chunks than the 16-bit plan's pay -- but only long ones (measured on
    // MI355X: at 16-head tiles from four blocks per chunk, n_h = 16, N =
    // 65536: 137 -> 256 chunks 17.0 -> 14.0 us; at 32-head tiles from
    // sixteen, n_h = 32, N = 131072: 16 x 128 -> 32 x 256 27.1 -> 23.1 us;
    // shorter chunks ran up to 18% slower). The 16-bit plan stays a
    // candidate.
    double us8 = 0.0;
    const Plan p8 = search(1, [](int ht, int) { return ht == 16 ? 4 : 16; }, us8);
    const double us16_as8 = modelled_us(p16, num_heads, total_tokens, batch, cu_count, paged,
                                        !seqlens && cache != CacheKind::kPaged, 1);
    return us8 < us16_as8 ? p8 : p16;
}

}  // namespace

// compute_plan searches a few hundred candidate plans (a few us of host
// time); decode loops repeat the same arguments, so each host thread keeps
// its last few plans.
Plan make_plan(bool fp32, int num_heads, int total_tokens, int batch, bool seqlens,
               int num_splits, int cu_count, CacheKind kind, bool f32_partials)
{
    struct Entry {
        int key[9];
        Plan plan;
    };
    constexpr int kEntries = 16;
    thread_local Entry cache[kEntries];
    thread_local int filled = 0, next = 0;
    const int key[9] = {fp32, num_heads, total_tokens, batch, seqlens, num_splits, cu_count, (int)kind, f32_partials};
    for (int e = 0; e < filled; ++e) {
        bool hit = true;
        for (int k = 0; k < 9; ++k)
            hit = hit && cache[e].key[k] == key[k];
        if (hit)
            return cache[e].plan;
    }
    const Plan p = compute_plan(fp32, num_heads, total_tokens, batch, seqlens, num_splits, cu_count, kind, f32_partials);
    Entry &slot = cache[next];
    for (int k = 0; k < 9; ++k)
        slot.key[k] = key[k];
    slot.plan = p;
    next = (next + 1) % kEntries;
    filled = filled < kEntries ? filled + 1 : kEntries;
    return p;
}


size_t partials_bytes(const Plan &p, int num_heads)
{
    const size_t rows = (size_t)p.n_slots * (size_t)num_heads;
    return align_up(rows * kDV * (size_t)p.part_bytes) + 2 * align_up(rows * sizeof(float));
}

Partials carve_partials(void *ws, const Plan &p, int num_heads)
{
    const size_t rows = (size_t)p.n_slots * (size_t)num_heads;
    char *base = static_cast<char *>(ws);
    Partials w;
    w.o = base;
    base += align_up(rows * kDV * (size_t)p.part_bytes);
    w.m = reinterpret_cast<float *>(base);
    base += align_up(rows * sizeof(float));
    w.l = reinterpret_cast<float *>(base);
    return w;
}

namespace {

// Workspace of the 16-bit paths: enough for either partial precision (the
// plans of the two may differ).
size_t split_workspace_bytes(int num_heads, int total_tokens, int batch, bool seqlens, int num_splits)
{
    const int cu = current_cu_count();
    const Plan a = make_plan(false, num_heads, total_tokens, batch, seqlens, num_splits, cu, CacheKind::kPacked, false);
    const Plan b = make_plan(false, num_heads, total_tokens, batch, seqlens, num_splits, cu, CacheKind::kPacked, true);
    return std::max(partials_bytes(a, num_heads), partials_bytes(b, num_heads));
}

bool heads_ok(int num_heads) { return num_heads > 0 && num_heads % 16 == 0 && num_heads <= 4096; }

// The plan that the plan queries report: a single sequence's, on the current
// device, for the fp8-cache entries with MLA_FLAG_FP8_CACHE (whose partials
// are fp16), else for mla_decode_split_fp16_ex with these flags.
Plan query_plan(int num_heads, int seq_length, int num_splits, unsigned flags)
{
    const bool f8 = (flags & MLA_FLAG_FP8_CACHE) != 0;
    return make_plan(false, num_heads, seq_length, 1, false, num_splits, current_cu_count(),
                     f8 ? CacheKind::kF8 : CacheKind::kPacked, !f8 && (flags & MLA_FLAG_FP32_PARTIALS) != 0);
}

constexpr int kPhaseSplit = 1;
constexpr int kPhaseCombine = 2;

// Who merges the partials of a whole call (both phases) on plan p: with one
// chunk, a single-sequence 16-bit call's split kernel writes the output
// itself and the call is one launch; otherwise combine_kernel merges.
int choose_merge(const Plan &p, bool single16, unsigned flags)
{
    if (!single16 || p.n_chunks != 1 || (flags & (MLA_FLAG_TWO_LAUNCHES | MLA_FLAG_SCALAR_TRANSPOSE)) != 0)
        return kMergeCombine;
    return kMergeDirect;
}

// How the 16-bit split kernel stores its partials. Nontemporal stores keep
// them out of the L2, which the kernel's end then need not write back (N =
// 4096: 12.78 -> 11.85 us per call when introduced). A combine of only a
// few workgroups is instead bound by each CU's read latency, and reads plain
// stored partials faster. Same box, plain against nontemporal: n_h = 16
// (32 combine workgroups) 15.55 -> 14.80 us; N = 4096 (256) 10.77 -> 11.01 us,
// N = 65536 with fp32 partials (256) 37.4 -> 38.3 us, batched (512) 94.2 -> 93.5.
// The quarter-tile combine (fewer (tile, sequence) items than CUs) also
// reads plain stored partials faster: n_h = 16, 128 splits (128 combine
// workgroups of 8 waves) 14.07 -> 13.82 us. So does the tile-group combine
// of large batches (more items than resident waves), by a little: medians of
// three calls, one box, batched 94.25 -> 93.96 us, paged 97.47 -> 96.87,
// fp8 batched 82.25 -> 81.63, MLA block step 138.83 -> 138.11.
int choose_part_plain(const Plan &p, int batch, int num_heads, int cu_count)
{
    const int items = num_heads / 16 * (kDV / 16) * batch;
    const bool tile_groups = combine_waves_per_item(p, batch, items, cu_count) == 0;
    return (items < cu_count || tile_groups || 4 * combine_workgroups(p, batch, num_heads, cu_count) < cu_count) ? 1
                                                                                                               : 0;
}

// Shared body of every entry point; `phases` selects the split kernel, the
// combine, or both (in that order, on one stream).
enum class Dtype { kF16, kBF16, kF32, kF8Cache };

int run_decode(Dtype dt, const void *query, const void *cache, const int *cu_seqlens,
               void *out, void *workspace, size_t workspace_bytes, int batch,
               int num_heads, int total_tokens, int num_splits, unsigned flags,
               void *stream, int phases = kPhaseSplit | kPhaseCombine,
               const Paging *paging = nullptr, float c_scale = 1.0f)
{
    const bool split = (phases & kPhaseSplit) != 0;
    const bool combine = (phases & kPhaseCombine) != 0;
    if (!workspace || (split && (!query || !cache)) || (combine && !out))
        return MLA_STATUS_INVALID_VALUE;
    if (!aligned16(workspace) || (split && (!aligned16(query) || !aligned16(cache))) ||
        (combine && !aligned16(out)))
        return MLA_STATUS_MISALIGNED;
    const bool fp32 = dt == Dtype::kF32;
    const bool f32_part = !fp32 && !paging && dt != Dtype::kF8Cache && (flags & MLA_FLAG_FP32_PARTIALS) != 0;
    const CacheKind kind = paging != nullptr ? CacheKind::kPaged
                           : dt == Dtype::kF8Cache ? CacheKind::kF8 : CacheKind::kPacked;
    const int cu = current_cu_count();
    Plan p = make_plan(fp32, num_heads, total_tokens, batch, cu_seqlens != nullptr, num_splits, cu, kind, f32_part);
    if (workspace_bytes < partials_bytes(p, num_heads))
        return MLA_STATUS_WORKSPACE_TOO_SMALL;
    const bool tr_load = (flags & MLA_FLAG_SCALAR_TRANSPOSE) == 0;
    if (split && combine)
        p.merge = choose_merge(p, batch == 1 && !cu_seqlens && !fp32 && !paging, flags);
    p.part_plain = choose_part_plain(p, batch, num_heads, cu);

    Problem pb;
    pb.q = query;
    pb.c = cache;
    pb.cu_seqlens = cu_seqlens;
    pb.out = out;
    pb.batch = batch;
    pb.num_heads = num_heads;
    pb.total_tokens = total_tokens;
    pb.fp8 = dt == Dtype::kF8Cache;
    pb.out_scale = pb.fp8 ? c_scale : 1.0f;
    pb.scale_log2 = scale_log2() * pb.out_scale;  // fp8: logits of the dequantised cache
    pb.bf16 = dt == Dtype::kBF16;
    pb.fp32 = fp32;
    pb.paging = paging ? *paging : Paging{nullptr, 0, 0, 0};
    const Partials w = carve_partials(workspace, p, num_heads);
    hipStream_t s = static_cast<hipStream_t>(stream);

    if (split) {
        const hipError_t e = fp32 ? launch_splitkv_fp32(pb, p, w, s) : launch_splitkv_fp16(pb, p, w, tr_load, s);
        if (e != hipSuccess)
            return fail_hip(e);
    }
    if (combine && p.merge == kMergeCombine) {
        const hipError_t e = launch_combine(pb, p, w, s);
        if (e != hipSuccess)
            return fail_hip(e);
    }
    return MLA_STATUS_SUCCESS;
}

// Device address of `scratch` on the current device, looked up with
// hipGetSymbolAddress on the first call on each device and kept; nullptr
// (the HIP error recorded) if the lookup fails.
std::atomic<void *> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

void *noalloc_scratch()
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        fail_hip(e);
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        fail_hip(hipErrorInvalidDevice);
        return nullptr;
    }
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (p)
        return p;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fail_hip(e != hipSuccess ? e : hipErrorInvalidSymbol);
            return nullptr;
        }
        g_scratch[dev].store(p, std::memory_order_release);
    }
    return p;
}

}  // namespace
}  // namespace mla

extern "C" {

int mla_abi_version(void) { return MLA_ABI_VERSION; }

const char *mla_status_string(int status)
{
    switch (status) {
    case MLA_STATUS_SUCCESS: return "success";
    case MLA_STATUS_INVALID_VALUE: return "invalid value (null pointer or unsupported size)";
    case MLA_STATUS_MISALIGNED: return "pointer not 16-byte aligned";
    case MLA_STATUS_WORKSPACE_TOO_SMALL: return "workspace too small";
    case MLA_STATUS_HIP_ERROR: return "HIP error";
    case MLA_STATUS_SCRATCH_EXCEEDED:
        return "the split partials need more than the allocation-free entry point's scratch "
               "(MLA_NOALLOC_SCRATCH_BYTES); use mla_decode_split_fp16 with a workspace";
    default: return "unknown status";
    }
}

int mla_last_hip_error(void) { return mla::t_last_hip_error; }

int mla_decode_split_num_splits(int num_heads, int seq_length, int num_splits, unsigned flags)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return 0;
    return mla::query_plan(num_heads, seq_length, num_splits, flags).n_chunks;
}

int mla_decode_split_head_tile(int num_heads, int seq_length, int num_splits, unsigned flags)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return 0;
    return mla::query_plan(num_heads, seq_length, num_splits, flags).head_tile;
}

int mla_decode_split_launches(int num_heads, int seq_length, int num_splits, unsigned flags)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return 0;
    return mla::choose_merge(mla::query_plan(num_heads, seq_length, num_splits, flags), true, flags) ==
                   mla::kMergeCombine
               ? 2
               : 1;
}

size_t mla_decode_split_workspace_size(int num_heads, int seq_length, int num_splits)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return 0;
    return mla::split_workspace_bytes(num_heads, seq_length, 1, false, num_splits);
}

int mla_decode_split_fp16_ex(const void *query, const void *cache, void *out,
                             void *workspace, size_t workspace_bytes,
                             int num_heads, int seq_length, int num_splits,
                             unsigned flags, void *stream)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return MLA_STATUS_INVALID_VALUE;
    return mla::run_decode(mla::Dtype::kF16, query, cache, nullptr, out, workspace, workspace_bytes, 1,
                           num_heads, seq_length, num_splits, flags, stream);
}

int mla_decode_split_fp16(const void *query, const void *cache, void *out,
                          void *workspace, size_t workspace_bytes,
                          int num_heads, int seq_length, int num_splits, void *stream)
{
    return mla_decode_split_fp16_ex(query, cache, out, workspace, workspace_bytes, num_heads,
                                    seq_length, num_splits, 0u, stream);
}

int mla_decode_split_fp16_noalloc(const void *query, const void *cache, void *out, int num_heads,
                                  int seq_length, int num_splits, void *stream)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return MLA_STATUS_INVALID_VALUE;
    // the same plan as mla_decode_split_fp16; its partials must fit the scratch
    const mla::Plan p = mla::make_plan(false, num_heads, seq_length, 1, false, num_splits, mla::current_cu_count(),
                                       mla::CacheKind::kPacked, false);
    if (mla::partials_bytes(p, num_heads) > (size_t)MLA_NOALLOC_SCRATCH_BYTES)
        return MLA_STATUS_SCRATCH_EXCEEDED;
    void *ws = mla::noalloc_scratch();
    if (!ws)
        return MLA_STATUS_HIP_ERROR;
    return mla::run_decode(mla::Dtype::kF16, query, cache, nullptr, out, ws, (size_t)MLA_NOALLOC_SCRATCH_BYTES, 1,
                           num_heads, seq_length, num_splits, 0u, stream);
}

int mla_decode_split_fp16_partials(const void *query, const void *cache, void *workspace,
                                   size_t workspace_bytes, int num_heads, int seq_length,
                                   int num_splits, unsigned flags, void *stream)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return MLA_STATUS_INVALID_VALUE;
    return mla::run_decode(mla::Dtype::kF16, query, cache, nullptr, nullptr, workspace, workspace_bytes, 1,
                           num_heads, seq_length, num_splits, flags, stream, mla::kPhaseSplit);
}

int mla_decode_split_fp16_combine(const void *workspace, size_t workspace_bytes, void *out,
                                  int num_heads, int seq_length, int num_splits, unsigned flags,
                                  void *stream)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return MLA_STATUS_INVALID_VALUE;
    return mla::run_decode(mla::Dtype::kF16, nullptr, nullptr, nullptr, out, const_cast<void *>(workspace),
                           workspace_bytes, 1, num_heads, seq_length, num_splits, flags, stream,
                           mla::kPhaseCombine);
}

size_t mla_decode_fused_workspace_size(int num_heads, int seq_length, int num_splits)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return 0;
    const mla::Plan p = mla::make_plan(true, num_heads, seq_length, 1, false, num_splits, mla::current_cu_count());
    return mla::partials_bytes(p, num_heads);
}

int mla_decode_fused_fp32(const float *query, const float *cache, float *out,
                          void *workspace, size_t workspace_bytes,
                          int num_heads, int head_dim_c, int seq_length,
                          int num_splits, void *stream)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1 || head_dim_c != MLA_HEAD_DIM_K)
        return MLA_STATUS_INVALID_VALUE;
    return mla::run_decode(mla::Dtype::kF32, query, cache, nullptr, out, workspace, workspace_bytes, 1,
                           num_heads, seq_length, num_splits, 0u, stream);
}

size_t mla_decode_split_batched_workspace_size(int batch, int num_heads, int total_tokens,
                                               int num_splits)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0)
        return 0;
    return mla::split_workspace_bytes(num_heads, total_tokens, batch, true, num_splits);
}

int mla_decode_split_batched_fp16(const void *query, const void *cache, const int *cu_seqlens,
                                  void *out, void *workspace, size_t workspace_bytes,
                                  int batch, int num_heads, int total_tokens, int num_splits,
                                  void *stream)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0 || !cu_seqlens)
        return MLA_STATUS_INVALID_VALUE;
    if (total_tokens == 0 && !cache)
        cache = query;  // nothing is read from the cache
    return mla::run_decode(mla::Dtype::kF16, query, cache, cu_seqlens, out, workspace, workspace_bytes,
                           batch, num_heads, total_tokens, num_splits, 0u, stream);
}

int mla_decode_split_batched_fp16_partials(const void *query, const void *cache, const int *cu_seqlens,
                                           void *workspace, size_t workspace_bytes, int batch, int num_heads,
                                           int total_tokens, int num_splits, void *stream)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0 || !cu_seqlens)
        return MLA_STATUS_INVALID_VALUE;
    if (total_tokens == 0 && !cache)
        cache = query;  // nothing is read from the cache
    return mla::run_decode(mla::Dtype::kF16, query, cache, cu_seqlens, nullptr, workspace, workspace_bytes,
                           batch, num_heads, total_tokens, num_splits, 0u, stream, mla::kPhaseSplit);
}

int mla_decode_split_batched_fp16_combine(const void *workspace, size_t workspace_bytes, const int *cu_seqlens,
                                          void *out, int batch, int num_heads, int total_tokens, int num_splits,
                                          void *stream)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0 || !cu_seqlens)
        return MLA_STATUS_INVALID_VALUE;
    return mla::run_decode(mla::Dtype::kF16, nullptr, nullptr, cu_seqlens, out, const_cast<void *>(workspace),
                           workspace_bytes, batch, num_heads, total_tokens, num_splits, 0u, stream,
                           mla::kPhaseCombine);
}

size_t mla_decode_paged_workspace_size(int batch, int num_heads, int total_tokens, int num_splits)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0)
        return 0;
    const mla::Plan p = mla::make_plan(false, num_heads, total_tokens, batch, true, num_splits,
                                       mla::current_cu_count(), mla::CacheKind::kPaged);
    return mla::partials_bytes(p, num_heads);
}

namespace {

int paged_decode(mla::Dtype dt, const void *query, const void *kv_cache, const int *block_table,
                 const int *cu_seqlens, void *out, void *workspace, size_t workspace_bytes, int batch,
                 int num_heads, int total_tokens, int page_size, int num_pages, int block_table_stride,
                 int num_splits, void *stream)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0 || !cu_seqlens || !block_table ||
        page_size < 32 || page_size > (1 << 20) || (page_size & (page_size - 1)) != 0 || num_pages < 1 ||
        block_table_stride < 1)
        return MLA_STATUS_INVALID_VALUE;
    if (total_tokens == 0 && !kv_cache)
        kv_cache = query;  // nothing is read from the cache
    mla::Paging pg{block_table, __builtin_ctz((unsigned)page_size), block_table_stride, num_pages};
    return mla::run_decode(dt, query, kv_cache, cu_seqlens, out, workspace, workspace_bytes, batch,
                           num_heads, total_tokens, num_splits, 0u, stream,
                           mla::kPhaseSplit | mla::kPhaseCombine, &pg);
}

}  // namespace

int mla_decode_paged_fp16(const void *query, const void *kv_cache, const int *block_table,
                          const int *cu_seqlens, void *out, void *workspace, size_t workspace_bytes,
                          int batch, int num_heads, int total_tokens, int page_size, int num_pages,
                          int block_table_stride, int num_splits, void *stream)
{
    return paged_decode(mla::Dtype::kF16, query, kv_cache, block_table, cu_seqlens, out, workspace,
                        workspace_bytes, batch, num_heads, total_tokens, page_size, num_pages,
                        block_table_stride, num_splits, stream);
}

int mla_decode_paged_bf16(const void *query, const void *kv_cache, const int *block_table,
                          const int *cu_seqlens, void *out, void *workspace, size_t workspace_bytes,
                          int batch, int num_heads, int total_tokens, int page_size, int num_pages,
                          int block_table_stride, int num_splits, void *stream)
{
    return paged_decode(mla::Dtype::kBF16, query, kv_cache, block_table, cu_seqlens, out, workspace,
                        workspace_bytes, batch, num_heads, total_tokens, page_size, num_pages,
                        block_table_stride, num_splits, stream);
}

size_t mla_decode_split_fp8_workspace_size(int batch, int num_heads, int total_tokens, int num_splits)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0)
        return 0;
    // one size for both fp8 entries: with batch 1 it also covers the
    // single-sequence entry's plan (no cu_seqlens, so no piece costs)
    const int cu = mla::current_cu_count();
    const mla::Plan p = mla::make_plan(false, num_heads, total_tokens, batch, true, num_splits, cu,
                                       mla::CacheKind::kF8);
    size_t bytes = mla::partials_bytes(p, num_heads);
    if (batch == 1) {
        const mla::Plan q = mla::make_plan(false, num_heads, total_tokens, 1, false, num_splits, cu,
                                           mla::CacheKind::kF8);
        bytes = std::max(bytes, mla::partials_bytes(q, num_heads));
    }
    return bytes;
}

int mla_decode_split_batched_fp8(const void *query, const void *cache_fp8, float cache_scale,
                                 const int *cu_seqlens, void *out, void *workspace, size_t workspace_bytes,
                                 int batch, int num_heads, int total_tokens, int num_splits, void *stream)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0 || !cu_seqlens ||
        !(cache_scale > 0.0f && cache_scale < INFINITY))
        return MLA_STATUS_INVALID_VALUE;
    if (total_tokens == 0 && !cache_fp8)
        cache_fp8 = query;  // nothing is read from the cache
    return mla::run_decode(mla::Dtype::kF8Cache, query, cache_fp8, cu_seqlens, out, workspace, workspace_bytes,
                           batch, num_heads, total_tokens, num_splits, 0u, stream,
                           mla::kPhaseSplit | mla::kPhaseCombine, nullptr, cache_scale);
}

int mla_decode_split_fp8(const void *query, const void *cache_fp8, float cache_scale, void *out,
                         void *workspace, size_t workspace_bytes, int num_heads, int seq_length,
                         int num_splits, void *stream)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1 || !(cache_scale > 0.0f && cache_scale < INFINITY))
        return MLA_STATUS_INVALID_VALUE;
    return mla::run_decode(mla::Dtype::kF8Cache, query, cache_fp8, nullptr, out, workspace, workspace_bytes, 1,
                           num_heads, seq_length, num_splits, 0u, stream, mla::kPhaseSplit | mla::kPhaseCombine,
                           nullptr, cache_scale);
}

int mla_decode_split_bf16(const void *query, const void *cache, void *out,
                          void *workspace, size_t workspace_bytes,
                          int num_heads, int seq_length, int num_splits, void *stream)
{
    if (!mla::heads_ok(num_heads) || seq_length < 1)
        return MLA_STATUS_INVALID_VALUE;
    return mla::run_decode(mla::Dtype::kBF16, query, cache, nullptr, out, workspace, workspace_bytes, 1,
                           num_heads, seq_length, num_splits, 0u, stream);
}

int mla_decode_split_batched_bf16(const void *query, const void *cache, const int *cu_seqlens,
                                  void *out, void *workspace, size_t workspace_bytes,
                                  int batch, int num_heads, int total_tokens, int num_splits,
                                  void *stream)
{
    if (!mla::heads_ok(num_heads) || batch < 1 || total_tokens < 0 || !cu_seqlens)
        return MLA_STATUS_INVALID_VALUE;
    if (total_tokens == 0 && !cache)
        cache = query;  // nothing is read from the cache
    return mla::run_decode(mla::Dtype::kBF16, query, cache, cu_seqlens, out, workspace, workspace_bytes,
                           batch, num_heads, total_tokens, num_splits, 0u, stream);
}

}  // extern "C"
