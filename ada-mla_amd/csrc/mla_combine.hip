// LSE-weighted merge of split-KV partials into the decode output:
//   m = max_s m_s,  l = sum_s l_s 2^(m_s - m),  O* = sum_s O_s 2^(m_s - m) / l
// over the slots of one (sequence, head); m_s are in log2 units.
//
// Replaces mla_decode_combine (reference csrc/mla_decode_splitk_fwd.cuh:894-939):
// fp32 partials instead of fp16, the max started at -inf, a sequence's slot
// range derived from the split plan (any number of splits, any batch), two
// heads per 256-thread workgroup with one 16-byte partial read per thread per
// slot, and the weights 2^(m_s - m) computed once per slot instead of once
// per column. An empty sequence writes zeros.
#include "mla_device.hpp"
#include "mla_internal.hpp"

namespace mla {
namespace {

template <bool kOutF32>
__global__ __launch_bounds__(256)
void combine_kernel(const float *__restrict__ o_part,
                    const float *__restrict__ m_part,
                    const float *__restrict__ l_part,
                    const int *__restrict__ cu_seqlens,
                    void *__restrict__ out,
                    int num_heads, int total_tokens, int chunk)
{
    const int b = blockIdx.y;
    const int head = blockIdx.x * 2 + (threadIdx.x >> 7);
    const int d = 4 * (threadIdx.x & 127);

    int lo = 0, hi = total_tokens;
    if (cu_seqlens) {
        lo = min(max(cu_seqlens[b], 0), total_tokens);
        hi = min(max(cu_seqlens[b + 1], lo), total_tokens);
    }
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    if (hi > lo) {
        const int s0 = lo / chunk + b;
        const int s1 = (hi - 1) / chunk + b;
        float m = -INFINITY;
        for (int s = s0; s <= s1; ++s)
            m = fmaxf(m, m_part[(size_t)s * num_heads + head]);
        float l = 0.f;
        for (int s = s0; s <= s1; ++s) {
            const float w = fast_exp2(m_part[(size_t)s * num_heads + head] - m);
            l += w * l_part[(size_t)s * num_heads + head];
            acc += w * *(const floatx4 *)(o_part + ((size_t)s * num_heads + head) * kDV + d);
        }
        acc *= 1.0f / l;
    }
    const size_t o_off = ((size_t)b * num_heads + head) * kDV + d;
    if constexpr (kOutF32) {
        *(floatx4 *)((float *)out + o_off) = acc;
    } else {
        half4 h = {(_Float16)acc[0], (_Float16)acc[1], (_Float16)acc[2], (_Float16)acc[3]};
        *(half4 *)((_Float16 *)out + o_off) = h;
    }
}

}  // namespace

hipError_t launch_combine(const Problem &pb, const Plan &p, const Partials &w,
                          bool out_fp32, hipStream_t s)
{
    const dim3 grid(pb.num_heads / 2, pb.batch), block(256);
    if (out_fp32)
        hipLaunchKernelGGL(combine_kernel<true>, grid, block, 0, s, w.o, w.m, w.l,
                           pb.cu_seqlens, pb.out, pb.num_heads, pb.total_tokens, p.chunk);
    else
        hipLaunchKernelGGL(combine_kernel<false>, grid, block, 0, s, w.o, w.m, w.l,
                           pb.cu_seqlens, pb.out, pb.num_heads, pb.total_tokens, p.chunk);
    return hipGetLastError();
}

}  // namespace mla
