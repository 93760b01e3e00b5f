// LSE-weighted merge of split-KV partials into the decode output:
//   m = max_s m_s,  l = sum_s l_s 2^(m_s - m),  O* = sum_s w_s O_s / l
// over the slots s of one (sequence, head); m_s are in log2 units, and
// w_s = l_s 2^(m_s - m) for partials normalised by their sum (fp16 path) or
// 2^(m_s - m) for unnormalised ones (fp32 path).
//
// Replaces mla_decode_combine (reference csrc/mla_decode_splitk_fwd.cuh:894-939),
// which ran one 128-thread block per head looping serially over the splits
// with the weight e^(m_s - m) recomputed per column. Here:
//  * the max starts at -inf; an empty sequence writes zeros;
//  * a sequence's slot range follows from the split plan (any number of
//    splits, any batch);
//  * the unit of work is an item = (16 x 16 output tile, sequence). The
//    partial O is stored tile by tile in MFMA accumulator order
//    (frag_offset), so a wave reads one slot's tile as one contiguous run
//    (512 B in fp16, 1 KB in fp32); lane (g, h) owns head h, dims 4g..4g+3.
//  * W waves share an item (W = 1..16, chosen from the slots per sequence so
//    that a wave merges about 4 slots): wave k merges slots k, k + W, ...
//    online (running max, rescaled sums), with the loads of its next 8 slots
//    in flight while it merges the current 8, and the W wave results are
//    merged through LDS. A workgroup holds max(8, W) waves, i.e. 8 / W items
//    for W < 8.
//  * with more items than the GPU keeps resident (large batches), one wave
//    instead merges 4 consecutive tiles of a sequence (same heads), so one
//    m / l load serves 4 tiles and the grid runs in one round
//    (combine_tiles_kernel).
//  * with fewer items than CUs (one sequence at fewer than 128 heads), and
//    with fp32 partials, the unit is a quarter tile (16 heads x 4 dims), so
//    four times as many workgroups share the reads (combine_quarter_kernel).
//  * the kernels' arguments (14 dwords) are preloaded into SGPRs at wave
//    launch (the library is built with -amdgpu-kernarg-preload-count=16), so
//    the first loads do not wait for a kernel-argument fetch.
#include <type_traits>

#include "mla_device.hpp"
#include "mla_internal.hpp"

namespace mla {

#ifdef MLA_TIMELINE
// Timeline build only (python ada-mla_amd/build.py --timeline, read by
// ada-mla_amd/timeline.py --combine through mla_timeline_read_combine): per
// wave of the last combine launch, s_memrealtime (100 MHz, one clock for the
// whole GPU) at entry, when its slots are merged (every load landed), before
// its store and after the store completes. The normal build compiles none of it.
constexpr int kCombineTimelineWaves = 16384;
__device__ unsigned long long mla_combine_stamps[kCombineTimelineWaves * 4];
#define MLA_CSTAMP(gw, e)                                                                      \
    do {                                                                                      \
        if (lane == 0 && (gw) < kCombineTimelineWaves)                                        \
            mla_combine_stamps[(gw) * 4 + (e)] = __builtin_amdgcn_s_memrealtime();            \
    } while (0)
#else
#define MLA_CSTAMP(gw, e) \
    do {                  \
    } while (0)
#endif

namespace {

constexpr int kU = 8;  // slots per load batch and wave

template <typename PartT>
struct SlotBatch {
    using V = typename std::conditional<
        sizeof(PartT) == 4, floatx4,
        typename std::conditional<std::is_same<PartT, __bf16>::value, bf16x4, half4>::type>::type;
    V v[kU];
    float m[kU];
    float l[kU];
};

__device__ __forceinline__ floatx4 to_f32(const floatx4 &v) { return v; }
__device__ __forceinline__ floatx4 to_f32(const half4 &v)
{
    return floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ floatx4 to_f32(const bf16x4 &v)
{
    return floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

// PartT: the partials' type; OutT: the output's. On the 16-bit paths
// (OutT fp16 / bf16) the partials are normalised by their sums and stored in
// OutT or fp32; on the fp32 path they are unnormalised fp32.
template <typename PartT, typename OutT, int W>
__global__ __launch_bounds__(64 * (W > 8 ? W : 8))
void combine_kernel(const PartT *__restrict__ o_part,
                    const float *__restrict__ m_part,
                    const float *__restrict__ l_part,
                    const int *__restrict__ cu_seqlens,
                    void *__restrict__ out,
                    int num_heads, int total_tokens, int chunk, int n_items, int n_chunks, int seq_cost)
{
    constexpr int kWaves = W > 8 ? W : 8;
    constexpr int kItems = kWaves / W;
    constexpr bool kNorm = !std::is_same<OutT, float>::value;
    using Batch = SlotBatch<PartT>;
    using V = typename Batch::V;
    __shared__ float s_m[W > 1 ? kWaves : 1][64];
    __shared__ float s_l[W > 1 ? kWaves : 1][64];
    __shared__ floatx4 s_o[W > 1 ? kWaves : 1][64];

    const int lane = threadIdx.x & 63;
    // wave-uniform values live in SGPRs: the index arithmetic (divisions
    // included) runs once per wave on the scalar unit, ahead of the loads
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = blockIdx.x * kItems + w / W;
    const int k = w % W;  // this wave's place among the item's W waves
    const bool valid = item < n_items;
    MLA_CSTAMP(blockIdx.x * kWaves + w, 0);
    // one sequence (no cu_seqlens): the item is the tile and the slots are
    // the n_chunks chunks, with no division; a batch: (sequence, tile) and
    // the sequence's slot range from its token range
    int tile = 0, b = 0, s0 = 0, ns = 0;
    if (!cu_seqlens) {
        tile = item;
        ns = valid ? n_chunks : 0;
    } else if (valid) {
        const int n_tiles = num_heads / 16 * (kDV / 16);
        tile = item % n_tiles;  // (head / 16) * 32 + dim / 16
        b = item / n_tiles;
        const int lo = min(max(cu_seqlens[b], 0), total_tokens);
        const int hi = min(max(cu_seqlens[b + 1], lo), total_tokens);
        if (hi > lo) {
            const long long c = (long long)seq_cost * (b + 1);  // virtual offset of the sequence
            s0 = (int)((lo + c) / chunk) + b;
            ns = (int)((hi - 1 + c) / chunk) + b - s0 + 1;
        }
    }
    const int head = (tile >> 5) * 16 + (lane & 15);
    const int dim0 = (tile & 31) * 16 + 4 * (lane >> 4);

    float m = -INFINITY, l = 0.f;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    if (ns > 0) {  // uniform per wave
        const size_t slot_elems = (size_t)num_heads * kDV;
        const PartT *op = o_part + (size_t)s0 * slot_elems + (size_t)tile * 256 + lane * 4;
        const float *mp = m_part + (size_t)s0 * num_heads + head;
        const float *lp = l_part + (size_t)s0 * num_heads + head;

        // slots k0, k0 + W, ..., k0 + W (kU - 1)
        auto load = [&](Batch &sb, int k0) {
#pragma unroll
            for (int j = 0; j < kU; ++j) {
                const int s = k0 + W * j;
                if (s < ns) {
                    sb.v[j] = *(const V *)(op + (size_t)s * slot_elems);
                    sb.m[j] = mp[(size_t)s * num_heads];
                    sb.l[j] = lp[(size_t)s * num_heads];
                } else {
                    sb.v[j] = V{};
                    sb.m[j] = -INFINITY;
                    sb.l[j] = 0.f;
                }
            }
        };
        auto merge = [&](const Batch &sb) {
            float mx = m;
#pragma unroll
            for (int j = 0; j < kU; ++j)
                mx = fmaxf(mx, sb.m[j]);
            if (mx != -INFINITY) {  // uniform per wave: the first batch holds a slot
                const float sc = fast_exp2(m - mx);
                acc *= sc;
                l *= sc;
#pragma unroll
                for (int j = 0; j < kU; ++j) {
                    const float e = fast_exp2(sb.m[j] - mx);
                    const float el = e * sb.l[j];
                    acc += (kNorm ? el : e) * to_f32(sb.v[j]);
                    l += el;
                }
                m = mx;
            }
        };
        constexpr int kStep = W * kU;
        Batch A, B;
        int k0 = k;
        if (k0 < ns) {
            load(A, k0);
            while (true) {
                bool more = k0 + kStep < ns;
                if (more)
                    load(B, k0 + kStep);
                merge(A);
                if (!more)
                    break;
                k0 += kStep;
                more = k0 + kStep < ns;
                if (more)
                    load(A, k0 + kStep);
                merge(B);
                if (!more)
                    break;
                k0 += kStep;
            }
        }
    }
    MLA_CSTAMP(blockIdx.x * kWaves + w, 1);
    if constexpr (W > 1) {
        s_m[w][lane] = m;
        s_l[w][lane] = l;
        s_o[w][lane] = acc;
        __syncthreads();
        if (k == 0) {
            m = s_m[w][lane];
#pragma unroll
            for (int j = 1; j < W; ++j)
                m = fmaxf(m, s_m[w + j][lane]);
            if (m != -INFINITY) {
                l = 0.f;
                acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    const float e = fast_exp2(s_m[w + j][lane] - m);
                    l += e * s_l[w + j][lane];
                    acc += e * s_o[w + j][lane];
                }
            }
        }
    }
    MLA_CSTAMP(blockIdx.x * kWaves + w, 2);
    if (valid && k == 0) {
        const floatx4 t = (m != -INFINITY) ? acc * (1.0f / l) : floatx4{0.f, 0.f, 0.f, 0.f};
        const size_t o_off = ((size_t)b * num_heads + head) * kDV + dim0;
        if constexpr (std::is_same<OutT, float>::value) {
            *(floatx4 *)((float *)out + o_off) = t;
        } else {
            using V = typename SlotBatch<OutT>::V;
            const V h = {(OutT)t[0], (OutT)t[1], (OutT)t[2], (OutT)t[3]};
            *(V *)((OutT *)out + o_off) = h;
        }
    }
#ifdef MLA_TIMELINE
    __builtin_amdgcn_s_waitcnt(0);
    MLA_CSTAMP(blockIdx.x * kWaves + w, 3);
#endif
}

// Many items (large batches): one wave merges kT consecutive tiles of one
// sequence -- the same 16 heads, dims 16 * kT apart from the next wave's --
// over all the sequence's slots, so the m and l loads serve kT tiles and each
// wave keeps kT loads per slot in flight; 4 waves per workgroup. Slots go in
// batches of kUT, the next batch's loads in flight while the current one
// merges.
constexpr int kT = 4;
constexpr int kUT = 4;

template <typename PartT, typename OutT>
__global__ __launch_bounds__(256)
void combine_tiles_kernel(const PartT *__restrict__ o_part,
                          const float *__restrict__ m_part,
                          const float *__restrict__ l_part,
                          const int *__restrict__ cu_seqlens,
                          void *__restrict__ out,
                          int num_heads, int total_tokens, int chunk, int n_groups, int seq_cost)
{
    constexpr bool kNorm = !std::is_same<OutT, float>::value;
    using V = typename SlotBatch<PartT>::V;
    struct Batch {
        V v[kUT][kT];
        float m[kUT];
        float l[kUT];
    };
    const int lane = threadIdx.x & 63;
    // wave-uniform: the group's index arithmetic runs on the scalar unit
    const int grp = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (grp >= n_groups)  // uniform per wave; no barriers follow
        return;
    MLA_CSTAMP(grp, 0);
    constexpr int kGroupsPerHeads = kDV / 16 / kT;  // tile groups per 16 heads
    const int groups_per_seq = num_heads / 16 * kGroupsPerHeads;
    const int b = grp / groups_per_seq;
    const int g = grp - b * groups_per_seq;
    const int tile0 = (g / kGroupsPerHeads) * 32 + (g % kGroupsPerHeads) * kT;  // (head / 16) * 32 + dim / 16
    const int head = (tile0 >> 5) * 16 + (lane & 15);

    int lo = 0, hi = total_tokens;
    if (cu_seqlens) {
        lo = min(max(cu_seqlens[b], 0), total_tokens);
        hi = min(max(cu_seqlens[b + 1], lo), total_tokens);
    }
    float m = -INFINITY, l = 0.f;
    floatx4 acc[kT];
#pragma unroll
    for (int t = 0; t < kT; ++t)
        acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (hi > lo) {
        const long long c = cu_seqlens ? (long long)seq_cost * (b + 1) : 0;  // virtual offset of the sequence
        const int s0 = (int)((lo + c) / chunk) + b;
        const int ns = (int)((hi - 1 + c) / chunk) + b - s0 + 1;
        const size_t slot_elems = (size_t)num_heads * kDV;
        const PartT *op = o_part + (size_t)s0 * slot_elems + (size_t)tile0 * 256 + lane * 4;
        const float *mp = m_part + (size_t)s0 * num_heads + head;
        const float *lp = l_part + (size_t)s0 * num_heads + head;
        auto load = [&](Batch &sb, int k0) {
#pragma unroll
            for (int j = 0; j < kUT; ++j) {
                const int s = k0 + j;
                if (s < ns) {
#pragma unroll
                    for (int t = 0; t < kT; ++t)
                        sb.v[j][t] = *(const V *)(op + (size_t)s * slot_elems + t * 256);
                    sb.m[j] = mp[(size_t)s * num_heads];
                    sb.l[j] = lp[(size_t)s * num_heads];
                } else {
#pragma unroll
                    for (int t = 0; t < kT; ++t)
                        sb.v[j][t] = V{};
                    sb.m[j] = -INFINITY;
                    sb.l[j] = 0.f;
                }
            }
        };
        auto merge = [&](const Batch &sb) {
            float mx = m;
#pragma unroll
            for (int j = 0; j < kUT; ++j)
                mx = fmaxf(mx, sb.m[j]);
            if (mx != -INFINITY) {  // uniform per wave: the first batch holds a slot
                const float sc = fast_exp2(m - mx);
                l *= sc;
#pragma unroll
                for (int t = 0; t < kT; ++t)
                    acc[t] *= sc;
#pragma unroll
                for (int j = 0; j < kUT; ++j) {
                    const float e = fast_exp2(sb.m[j] - mx);
                    const float el = e * sb.l[j];
#pragma unroll
                    for (int t = 0; t < kT; ++t)
                        acc[t] += (kNorm ? el : e) * to_f32(sb.v[j][t]);
                    l += el;
                }
                m = mx;
            }
        };
        Batch A, B;
        int k0 = 0;
        load(A, 0);
        while (true) {
            bool more = k0 + kUT < ns;
            if (more)
                load(B, k0 + kUT);
            merge(A);
            if (!more)
                break;
            k0 += kUT;
            more = k0 + kUT < ns;
            if (more)
                load(A, k0 + kUT);
            merge(B);
            if (!more)
                break;
            k0 += kUT;
        }
    }
    MLA_CSTAMP(grp, 1);
    MLA_CSTAMP(grp, 2);
    const float inv = (m != -INFINITY) ? 1.0f / l : 0.f;
#pragma unroll
    for (int t = 0; t < kT; ++t) {
        const int dim0 = ((tile0 + t) & 31) * 16 + 4 * (lane >> 4);
        const size_t o_off = ((size_t)b * num_heads + head) * kDV + dim0;
        const floatx4 v = acc[t] * inv;
        if constexpr (std::is_same<OutT, float>::value) {
            *(floatx4 *)((float *)out + o_off) = v;
        } else {
            using VO = typename SlotBatch<OutT>::V;
            const VO h = {(OutT)v[0], (OutT)v[1], (OutT)v[2], (OutT)v[3]};
            *(VO *)((OutT *)out + o_off) = h;
        }
    }
#ifdef MLA_TIMELINE
    __builtin_amdgcn_s_waitcnt(0);
    MLA_CSTAMP(grp, 3);
#endif
}

// Few items (fewer (tile, sequence) items than CUs: one sequence at fewer
// than 128 heads, small batches of few heads), or fp32 partials (up to
// kResidentWaves items): the unit of work is a quarter
// tile -- the 16 heads x 4 dims that lanes 16 q .. 16 q + 15 own in the
// tile's accumulator order, 64 contiguous elements of each slot -- so the
// grid holds four times as many workgroups and spreads the reads over that
// many CUs. One workgroup of W waves per quarter item. Lane (j, h) takes head
// h of slots 4 i + j, so one load instruction reads the quarter of four
// consecutive slots; wave k takes the slot quads k, k + W, ..., kUQ of them
// per load batch, the next batch's loads in flight while it merges the
// current one. The four slot groups of a wave are merged across lanes
// (v_permlane32/16_swap), the W waves through LDS; lanes 0..15 of wave 0
// store the quarter.
constexpr int kUQ = 4;  // slot quads per load batch and wave

template <typename PartT, typename OutT, int W>
__global__ __launch_bounds__(64 * W)
void combine_quarter_kernel(const PartT *__restrict__ o_part,
                            const float *__restrict__ m_part,
                            const float *__restrict__ l_part,
                            const int *__restrict__ cu_seqlens,
                            void *__restrict__ out,
                            int num_heads, int total_tokens, int chunk, int n_chunks, int seq_cost)
{
    constexpr bool kNorm = !std::is_same<OutT, float>::value;
    using V = typename SlotBatch<PartT>::V;
    struct Batch {
        V v[kUQ];
        float m[kUQ];
        float l[kUQ];
    };
    __shared__ float s_m[W][16];
    __shared__ float s_l[W][16];
    __shared__ floatx4 s_o[W][16];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    MLA_CSTAMP(blockIdx.x * W + w, 0);
    const int item = blockIdx.x >> 2;  // (sequence, tile)
    const int q = blockIdx.x & 3;      // dims 4 q .. 4 q + 3 of the tile
    const int j = lane >> 4, h = lane & 15;
    int tile = item, b = 0, s0 = 0, ns = n_chunks;
    if (cu_seqlens) {
        const int n_tiles = num_heads / 16 * (kDV / 16);
        tile = item % n_tiles;  // (head / 16) * 32 + dim / 16
        b = item / n_tiles;
        ns = 0;
        const int lo = min(max(cu_seqlens[b], 0), total_tokens);
        const int hi = min(max(cu_seqlens[b + 1], lo), total_tokens);
        if (hi > lo) {
            const long long c = (long long)seq_cost * (b + 1);  // virtual offset of the sequence
            s0 = (int)((lo + c) / chunk) + b;
            ns = (int)((hi - 1 + c) / chunk) + b - s0 + 1;
        }
    }
    const int head = (tile >> 5) * 16 + h;

    float m = -INFINITY, l = 0.f;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const int n_quads = (ns + 3) / 4;
    if (w < n_quads) {  // uniform per wave
        const size_t slot_elems = (size_t)num_heads * kDV;
        const PartT *op = o_part + (size_t)s0 * slot_elems + (size_t)tile * 256 + q * 64 + h * 4;
        const float *mp = m_part + (size_t)s0 * num_heads + head;
        const float *lp = l_part + (size_t)s0 * num_heads + head;
        // quads k0, k0 + W, ..., k0 + W (kUQ - 1); this lane's slot of each
        auto load = [&](Batch &sb, int k0) {
#pragma unroll
            for (int i = 0; i < kUQ; ++i) {
                const int s = 4 * (k0 + W * i) + j;
                if (s < ns) {
                    sb.v[i] = *(const V *)(op + (size_t)s * slot_elems);
                    sb.m[i] = mp[(size_t)s * num_heads];
                    sb.l[i] = lp[(size_t)s * num_heads];
                } else {
                    sb.v[i] = V{};
                    sb.m[i] = -INFINITY;
                    sb.l[i] = 0.f;
                }
            }
        };
        // per lane: a lane with no slot yet has m = -inf and keeps zeros
        auto merge = [&](const Batch &sb) {
            float mx = m;
#pragma unroll
            for (int i = 0; i < kUQ; ++i)
                mx = fmaxf(mx, sb.m[i]);
            const float mr = mx == -INFINITY ? 0.f : mx;
            const float sc = fast_exp2(m - mr);
            acc *= sc;
            l *= sc;
#pragma unroll
            for (int i = 0; i < kUQ; ++i) {
                const float e = fast_exp2(sb.m[i] - mr);
                const float el = e * sb.l[i];
                acc += (kNorm ? el : e) * to_f32(sb.v[i]);
                l += el;
            }
            m = mx;
        };
        constexpr int kStep = W * kUQ;
        Batch A, B;
        int k0 = w;
        load(A, k0);
        while (true) {
            bool more = k0 + kStep < n_quads;
            if (more)
                load(B, k0 + kStep);
            merge(A);
            if (!more)
                break;
            k0 += kStep;
            more = k0 + kStep < n_quads;
            if (more)
                load(A, k0 + kStep);
            merge(B);
            if (!more)
                break;
            k0 += kStep;
        }
    }
    MLA_CSTAMP(blockIdx.x * W + w, 1);
    // the four slot groups of the wave (lanes h, h + 16, h + 32, h + 48)
    {
        const float mx = max_over_lane_groups(m);
        const float f = fast_exp2(m - (mx == -INFINITY ? 0.f : mx));
        l = sum_over_lane_groups(l * f);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            acc[c] = sum_over_lane_groups(acc[c] * f);
        m = mx;
    }
    if constexpr (W > 1) {
        if (lane < 16) {
            s_m[w][h] = m;
            s_l[w][h] = l;
            s_o[w][h] = acc;
        }
        __syncthreads();
        if (w == 0) {
            m = s_m[0][h];
#pragma unroll
            for (int k = 1; k < W; ++k)
                m = fmaxf(m, s_m[k][h]);
            const float mr = m == -INFINITY ? 0.f : m;
            l = 0.f;
            acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < W; ++k) {
                const float e = fast_exp2(s_m[k][h] - mr);
                l += e * s_l[k][h];
                acc += e * s_o[k][h];
            }
        }
    }
    MLA_CSTAMP(blockIdx.x * W + w, 2);
    if (w == 0 && lane < 16) {
        const floatx4 t = (m != -INFINITY) ? acc * (1.0f / l) : floatx4{0.f, 0.f, 0.f, 0.f};
        const size_t o_off = ((size_t)b * num_heads + head) * kDV + (tile & 31) * 16 + 4 * q;
        if constexpr (std::is_same<OutT, float>::value) {
            *(floatx4 *)((float *)out + o_off) = t;
        } else {
            using VO = typename SlotBatch<OutT>::V;
            *(VO *)((OutT *)out + o_off) = VO{(OutT)t[0], (OutT)t[1], (OutT)t[2], (OutT)t[3]};
        }
    }
#ifdef MLA_TIMELINE
    __builtin_amdgcn_s_waitcnt(0);
    MLA_CSTAMP(blockIdx.x * W + w, 3);
#endif
}

template <typename PartT, typename OutT, int W>
void launch_w(const Problem &pb, const Plan &p, const Partials &w, int n_items, hipStream_t s)
{
    constexpr int kWaves = W > 8 ? W : 8;
    constexpr int kItems = kWaves / W;
    hipLaunchKernelGGL((combine_kernel<PartT, OutT, W>), dim3((n_items + kItems - 1) / kItems),
                       dim3(64 * kWaves), 0, s, static_cast<const PartT *>(w.o), w.m, w.l,
                       pb.cu_seqlens, pb.out, pb.num_heads, pb.total_tokens, p.chunk, n_items, p.n_chunks,
                       p.seq_cost);
}

template <typename PartT, typename OutT, int W>
void launch_quarter(const Problem &pb, const Plan &p, const Partials &w, int n_items, hipStream_t s)
{
    hipLaunchKernelGGL((combine_quarter_kernel<PartT, OutT, W>), dim3(4 * n_items), dim3(64 * W), 0, s,
                       static_cast<const PartT *>(w.o), w.m, w.l, pb.cu_seqlens, pb.out, pb.num_heads,
                       pb.total_tokens, p.chunk, p.n_chunks, p.seq_cost);
}

// waves > 0: combine_kernel with that many waves per item; 0:
// combine_tiles_kernel; < 0: combine_quarter_kernel with -waves waves.
template <typename PartT, typename OutT>
void launch_part(const Problem &pb, const Plan &p, const Partials &w, int waves, int n_items,
                 hipStream_t s)
{
    if (waves < 0) {
        switch (-waves) {
        case 1: launch_quarter<PartT, OutT, 1>(pb, p, w, n_items, s); break;
        case 2: launch_quarter<PartT, OutT, 2>(pb, p, w, n_items, s); break;
        case 4: launch_quarter<PartT, OutT, 4>(pb, p, w, n_items, s); break;
        case 8: launch_quarter<PartT, OutT, 8>(pb, p, w, n_items, s); break;
        default: launch_quarter<PartT, OutT, 16>(pb, p, w, n_items, s); break;
        }
        return;
    }
    if (waves == 0) {  // kT tiles per wave
        const int n_groups = n_items / kT;
        hipLaunchKernelGGL((combine_tiles_kernel<PartT, OutT>), dim3((n_groups + 3) / 4), dim3(256), 0, s,
                           static_cast<const PartT *>(w.o), w.m, w.l, pb.cu_seqlens, pb.out, pb.num_heads,
                           pb.total_tokens, p.chunk, n_groups, p.seq_cost);
        return;
    }
    switch (waves) {
    case 1: launch_w<PartT, OutT, 1>(pb, p, w, n_items, s); break;
    case 2: launch_w<PartT, OutT, 2>(pb, p, w, n_items, s); break;
    case 4: launch_w<PartT, OutT, 4>(pb, p, w, n_items, s); break;
    case 8: launch_w<PartT, OutT, 8>(pb, p, w, n_items, s); break;
    default: launch_w<PartT, OutT, 16>(pb, p, w, n_items, s); break;
    }
}

}  // namespace

#ifdef MLA_TIMELINE
extern "C" int mla_timeline_read_combine(void *dst, size_t bytes)
{
    const size_t n = bytes < sizeof(mla_combine_stamps) ? bytes : sizeof(mla_combine_stamps);
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(mla_combine_stamps), n, 0, hipMemcpyDeviceToHost);
}

// Zeroes the combine stamps (waves of the next launch overwrite theirs; the
// rest stay zero).
extern "C" int mla_timeline_clear_combine()
{
    static unsigned long long zeros[kCombineTimelineWaves * 4];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(mla_combine_stamps), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
#endif

// Waves that share one (tile, sequence) item: enough that each merges about
// 4 slots of an average sequence, at most 16, and no more than keep the grid
// to about kResidentWaves waves, so that it runs in one round. Measured on
// MI355X (rocprofv3 kernel durations): batched B = 32 at n_h = 128 (8192
// items, about 5 slots each) merges in 8.4 us with one wave per item against
// 12.4 us with two; one sequence (256 items) is fastest with the 4-slot
// rule (N = 4096: 8 waves per item).
// With fewer items than CUs, and with fp32 partials, quarter items
// (combine_quarter_kernel, returned as -W): W waves such that each merges
// about kUQ quads of slots, at most 16. fp32 partials read faster that way
// at every slot count measured (one sequence at 128 heads, µs per call,
// items -> quarter items: fp16 path with fp32 partials N = 4096 13.92 ->
// 13.11, N = 16384 22.33 -> 21.01, N = 65536 35.02 -> 34.75; fp32 path
// N = 1024 14.29 -> 13.59, N = 4096 24.78 -> 23.44, N = 8192 36.11 -> 35.62);
// fp16 partials do not (N = 4096 10.79 -> 11.03).
constexpr int kResidentWaves = 4096;

int combine_waves_per_item(const Plan &p, int batch, int n_items, int cu_count)
{
    if (n_items > kResidentWaves)
        return 0;  // more items than resident waves: kT tiles per wave (combine_tiles_kernel)
    const int slots = (p.n_slots + batch - 1) / batch;  // about the slots of one sequence
    if (n_items < cu_count || p.part_bytes == 4) {
        const int quads = (slots + 3) / 4;
        int waves = 1;
        while (waves < 16 && kUQ * waves < quads)
            waves *= 2;
        return -waves;
    }
    int waves = 1;
    while (waves < 16 && 4 * waves < slots && 2 * waves * n_items <= kResidentWaves)
        waves *= 2;
    return waves;
}

int combine_workgroups(const Plan &p, int batch, int num_heads, int cu_count)
{
    const int n_items = num_heads / 16 * (kDV / 16) * batch;
    const int waves = combine_waves_per_item(p, batch, n_items, cu_count);
    if (waves < 0)
        return 4 * n_items;
    if (waves == 0)
        return (n_items / kT + 3) / 4;
    const int items_per_wg = (waves > 8 ? waves : 8) / waves;
    return (n_items + items_per_wg - 1) / items_per_wg;
}

hipError_t launch_combine(const Problem &pb, const Plan &p, const Partials &w,
                          hipStream_t s)
{
    const int n_items = pb.num_heads / 16 * (kDV / 16) * pb.batch;
    const int waves = combine_waves_per_item(p, pb.batch, n_items, current_cu_count());
    if (pb.fp32)
        launch_part<float, float>(pb, p, w, waves, n_items, s);
    else if (p.part_bytes == 4 && !pb.bf16)  // fp32 partials: an option of the fp16 path only
        launch_part<float, _Float16>(pb, p, w, waves, n_items, s);
    else if (p.part_bytes == 4)
        return hipErrorInvalidValue;
    else
        pb.bf16 ? launch_part<__bf16, __bf16>(pb, p, w, waves, n_items, s)
                : launch_part<_Float16, _Float16>(pb, p, w, waves, n_items, s);
    // the launch's own error; hipPeekAtLastError leaves a sticky error from
    // the caller's earlier work in place for the caller to see
    return hipPeekAtLastError();
}

}  // namespace mla
