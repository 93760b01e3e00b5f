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
//  * one 256-thread workgroup per (head, 128-column quarter, sequence): lanes
//    0..31 of each of 8 slot groups own 4 columns each and stream every 8th
//    slot with independent 16-byte loads, so the partial reads of a head are
//    spread over 4 workgroups and many loads are in flight per thread; the 8
//    group sums are added through LDS.
#include "mla_device.hpp"
#include "mla_internal.hpp"

namespace mla {
namespace {

constexpr int kCols = 128;                 // output columns per workgroup
constexpr int kQuads = kCols / 4;          // 32 threads per slot group
constexpr int kGroups = 256 / kQuads;      // 8 slot groups

// Workgroup-wide reduction of one float (max or sum) over 256 threads.
template <bool kMax>
__device__ __forceinline__ float block_reduce(float v, float *red)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = kMax ? fmaxf(v, o) : v + o;
    }
    const int wave = threadIdx.x >> 6;
    __syncthreads();  // red is reused
    if ((threadIdx.x & 63) == 0)
        red[wave] = v;
    __syncthreads();
    return kMax ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]))
                : (red[0] + red[1]) + (red[2] + red[3]);
}

template <bool kOutF32>
__global__ __launch_bounds__(256)
void combine_kernel(const float *__restrict__ o_part,
                    const float *__restrict__ m_part,
                    const float *__restrict__ l_part,
                    const int *__restrict__ cu_seqlens,
                    void *__restrict__ out,
                    int num_heads, int total_tokens, int chunk)
{
    __shared__ float red[4];
    __shared__ floatx4 part[kGroups][kQuads];

    const int head = blockIdx.x;
    const int col0 = blockIdx.y * kCols;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int quad = tid % kQuads;
    const int grp = tid / kQuads;

    int lo = 0, hi = total_tokens;
    if (cu_seqlens) {
        lo = min(max(cu_seqlens[b], 0), total_tokens);
        hi = min(max(cu_seqlens[b + 1], lo), total_tokens);
    }
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    float inv_l = 0.f;
    if (hi > lo) {  // uniform per workgroup
        const int s0 = lo / chunk + b;
        const int ns = (hi - 1) / chunk + b - s0 + 1;
        const float *mrow = m_part + (size_t)s0 * num_heads + head;
        const float *lrow = l_part + (size_t)s0 * num_heads + head;

        float mx = -INFINITY;
        for (int s = tid; s < ns; s += 256)
            mx = fmaxf(mx, mrow[(size_t)s * num_heads]);
        const float m = block_reduce<true>(mx, red);
        float ls = 0.f;
        for (int s = tid; s < ns; s += 256)
            ls += fast_exp2(mrow[(size_t)s * num_heads] - m) * lrow[(size_t)s * num_heads];
        inv_l = 1.0f / block_reduce<false>(ls, red);

        const float *orow = o_part + ((size_t)s0 * num_heads + head) * kDV + col0 + 4 * quad;
        const size_t ostride = (size_t)num_heads * kDV;
        int s = grp;
        for (; s + 3 * kGroups < ns; s += 4 * kGroups) {
            const floatx4 v0 = *(const floatx4 *)(orow + (size_t)s * ostride);
            const floatx4 v1 = *(const floatx4 *)(orow + (size_t)(s + kGroups) * ostride);
            const floatx4 v2 = *(const floatx4 *)(orow + (size_t)(s + 2 * kGroups) * ostride);
            const floatx4 v3 = *(const floatx4 *)(orow + (size_t)(s + 3 * kGroups) * ostride);
            acc += fast_exp2(mrow[(size_t)s * num_heads] - m) * v0;
            acc += fast_exp2(mrow[(size_t)(s + kGroups) * num_heads] - m) * v1;
            acc += fast_exp2(mrow[(size_t)(s + 2 * kGroups) * num_heads] - m) * v2;
            acc += fast_exp2(mrow[(size_t)(s + 3 * kGroups) * num_heads] - m) * v3;
        }
        for (; s < ns; s += kGroups)
            acc += fast_exp2(mrow[(size_t)s * num_heads] - m) * *(const floatx4 *)(orow + (size_t)s * ostride);
    }
    part[grp][quad] = acc;
    __syncthreads();
    if (grp == 0) {
        floatx4 t = part[0][quad];
#pragma unroll
        for (int k = 1; k < kGroups; ++k)
            t += part[k][quad];
        t *= inv_l;
        const size_t o_off = ((size_t)b * num_heads + head) * kDV + col0 + 4 * quad;
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
    const dim3 grid(pb.num_heads, kDV / kCols, pb.batch), block(256);
    if (out_fp32)
        hipLaunchKernelGGL(combine_kernel<true>, grid, block, 0, s, w.o, w.m, w.l,
                           pb.cu_seqlens, pb.out, pb.num_heads, pb.total_tokens, p.chunk);
    else
        hipLaunchKernelGGL(combine_kernel<false>, grid, block, 0, s, w.o, w.m, w.l,
                           pb.cu_seqlens, pb.out, pb.num_heads, pb.total_tokens, p.chunk);
    return hipGetLastError();
}

}  // namespace mla
