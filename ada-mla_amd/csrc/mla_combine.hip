// LSE-weighted merge of split-KV partials into the decode output:
//   m = max_s m_s,  l = sum_s l_s 2^(m_s - m),  O* = sum_s O_s 2^(m_s - m) / l
// over the slots s of one (sequence, head); m_s are in log2 units.
//
// Replaces mla_decode_combine (reference csrc/mla_decode_splitk_fwd.cuh:894-939),
// which ran one 128-thread block per head looping serially over the splits
// with the weight e^(m_s - m) recomputed per column. Here:
//  * fp32 partials; the max starts at -inf; an empty sequence writes zeros;
//  * a sequence's slot range follows from the split plan (any number of
//    splits, any batch);
//  * one 512-thread workgroup per (16 x 16 output tile, sequence). The
//    partial O is stored tile by tile in MFMA accumulator order
//    (frag_offset), so a wave reads one slot's tile as 1 KB of contiguous
//    memory; lane (g, h) owns head h, dims 4g..4g+3 of the tile. Each of the
//    8 waves merges every 8th slot online (running max, rescaled sums) with
//    the loads of the next 8 slots in flight while it merges the current 8
//    (128 slots per memory round trip), and the 8 wave results are merged
//    through LDS.
#include "mla_device.hpp"
#include "mla_internal.hpp"

namespace mla {
namespace {

constexpr int kWaves = 8;
constexpr int kU = 8;  // slots per load batch and wave

struct SlotBatch {
    floatx4 v[kU];
    float m[kU];
    float l[kU];
};

template <bool kOutF32>
__global__ __launch_bounds__(64 * kWaves)
void combine_kernel(const float *__restrict__ o_part,
                    const float *__restrict__ m_part,
                    const float *__restrict__ l_part,
                    const int *__restrict__ cu_seqlens,
                    void *__restrict__ out,
                    int num_heads, int total_tokens, int chunk)
{
    __shared__ float s_m[kWaves][64];
    __shared__ float s_l[kWaves][64];
    __shared__ floatx4 s_o[kWaves][64];

    const int tile = blockIdx.x;  // (head / 16) * 32 + dim / 16
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int head = (tile >> 5) * 16 + (lane & 15);
    const int dim0 = (tile & 31) * 16 + 4 * (lane >> 4);

    int lo = 0, hi = total_tokens;
    if (cu_seqlens) {
        lo = min(max(cu_seqlens[b], 0), total_tokens);
        hi = min(max(cu_seqlens[b + 1], lo), total_tokens);
    }
    float m = -INFINITY, l = 0.f;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    if (hi > lo) {  // uniform per workgroup
        const int s0 = lo / chunk + b;
        const int ns = (hi - 1) / chunk + b - s0 + 1;
        const size_t slot_floats = (size_t)num_heads * kDV;
        const float *op = o_part + (size_t)s0 * slot_floats + (size_t)tile * 256 + lane * 4;
        const float *mp = m_part + (size_t)s0 * num_heads + head;
        const float *lp = l_part + (size_t)s0 * num_heads + head;

        // slots k0, k0 + 8, ..., k0 + 8 (kU - 1) of this wave
        auto load = [&](SlotBatch &sb, int k0) {
#pragma unroll
            for (int j = 0; j < kU; ++j) {
                const int s = k0 + kWaves * j;
                if (s < ns) {
                    sb.v[j] = *(const floatx4 *)(op + (size_t)s * slot_floats);
                    sb.m[j] = mp[(size_t)s * num_heads];
                    sb.l[j] = lp[(size_t)s * num_heads];
                } else {
                    sb.v[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                    sb.m[j] = -INFINITY;
                    sb.l[j] = 0.f;
                }
            }
        };
        auto merge = [&](const SlotBatch &sb) {
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
                    acc += e * sb.v[j];
                    l += e * sb.l[j];
                }
                m = mx;
            }
        };
        constexpr int kStep = kWaves * kU;
        SlotBatch A, B;
        int k0 = w;
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
    s_m[w][lane] = m;
    s_l[w][lane] = l;
    s_o[w][lane] = acc;
    __syncthreads();
    if (w == 0) {
        float mm = s_m[0][lane];
#pragma unroll
        for (int k = 1; k < kWaves; ++k)
            mm = fmaxf(mm, s_m[k][lane]);
        floatx4 t = {0.f, 0.f, 0.f, 0.f};
        if (mm != -INFINITY) {
            float ls = 0.f;
#pragma unroll
            for (int k = 0; k < kWaves; ++k) {
                const float e = fast_exp2(s_m[k][lane] - mm);
                ls += e * s_l[k][lane];
                t += e * s_o[k][lane];
            }
            t *= 1.0f / ls;
        }
        const size_t o_off = ((size_t)b * num_heads + head) * kDV + dim0;
        if constexpr (kOutF32) {
            *(floatx4 *)((float *)out + o_off) = t;
        } else {
            const half4 h = {(_Float16)t[0], (_Float16)t[1], (_Float16)t[2], (_Float16)t[3]};
            *(half4 *)((_Float16 *)out + o_off) = h;
        }
    }
}

}  // namespace

hipError_t launch_combine(const Problem &pb, const Plan &p, const Partials &w,
                          bool out_fp32, hipStream_t s)
{
    const dim3 grid(pb.num_heads / 16 * (kDV / 16), pb.batch), block(64 * kWaves);
    if (out_fp32)
        hipLaunchKernelGGL(combine_kernel<true>, grid, block, 0, s, w.o, w.m, w.l,
                           pb.cu_seqlens, pb.out, pb.num_heads, pb.total_tokens, p.chunk);
    else
        hipLaunchKernelGGL(combine_kernel<false>, grid, block, 0, s, w.o, w.m, w.l,
                           pb.cu_seqlens, pb.out, pb.num_heads, pb.total_tokens, p.chunk);
    return hipGetLastError();
}

}  // namespace mla
