// Device-side helpers for the gfx950 (CDNA4) MLA decode kernels: vector
// types, MFMA wrappers, the LDS transpose read and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

namespace mla {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef short shortx4 __attribute__((__vector_size__(4 * sizeof(short))));

#define MLA_LDS __attribute__((address_space(3)))

// D[16x16] += A[16x32] * B[32x16], fp16 in, fp32 accumulate.
// Lane l supplies A[l % 16][8 * (l / 16) + j] and B[8 * (l / 16) + j][l % 16]
// (j = 0..7) and holds D[4 * (l / 16) + i][l % 16] (i = 0..3).
__device__ __forceinline__ floatx4 mfma16x16x32(half8 a, half8 b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The same product with bf16 operands.
__device__ __forceinline__ floatx4 mfma16x16x32(bf16x8 a, bf16x8 b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef int intx8 __attribute__((ext_vector_type(8)));

// D[16x16] += A[16x128] * B[128x16], OCP fp8 E4M3 in, fp32 accumulate.
// Lane l supplies A[l % 16][32 * (l / 16) + j] and B[32 * (l / 16) + j][l % 16]
// as byte j (0..31) of its 8 registers; D layout as above. (Checked on
// gfx950 against a float64 product of the decoded bytes.)
__device__ __forceinline__ floatx4 mfma16x16x128_fp8(intx8 a, intx8 b, floatx4 c)
{
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// D[16x16] += A[16x32] * B[32x16], OCP fp8 E4M3 in: lane l supplies
// A[l % 16][8 * (l / 16) + j] and B[8 * (l / 16) + j][l % 16] as byte j (0..7).
__device__ __forceinline__ floatx4 mfma16x16x32_fp8(uint2 a, uint2 b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), c,
                                                     0, 0, 0);
}

// Vector types of a 16-bit storage type (fp16 or bf16): 8 elements are one
// MFMA operand, 4 one transpose read or one partial store.
template <typename E>
struct Vec;
template <>
struct Vec<_Float16> {
    using v8 = half8;
    using v4 = half4;
};
template <>
struct Vec<__bf16> {
    using v8 = bf16x8;
    using v4 = bf16x4;
};

// D[16x16] += A[16x4] * B[4x16] in fp32. Lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16]; D layout as above.
__device__ __forceinline__ floatx4 mfma16x16x4f32(float a, float b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane j points at the
// 4 halves [row j / 4][4 * (j % 4) .. +3] of a 4 x 16 block; after the read,
// lane i of the group holds column i of that block (rows 0..3).
template <typename E>
__device__ __forceinline__ typename Vec<E>::v4 lds_read_tr16(const E *p)
{
    const MLA_LDS shortx4 *lp = (const MLA_LDS shortx4 *)(const MLA_LDS E *)p;
    shortx4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<MLA_LDS shortx4 *>(lp));
    return __builtin_bit_cast(typename Vec<E>::v4, r);
}

// ds_read_b64_tr_b8: within each group of 16 lanes, lane j points at the 8
// bytes [row j / 2][8 * (j % 2) .. +7] of an 8 x 16 byte block; after the
// read, lane i of the group holds column i of that block (byte r = row r).
// (Lane layout measured on gfx950.)
__device__ __forceinline__ uint2 lds_read_tr8(const unsigned char *p)
{
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MLA_LDS v2i *)(const MLA_LDS unsigned char *)p);
    return uint2{(unsigned)r[0], (unsigned)r[1]};
}

// 2^x on the hardware exp unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float fast_exp2(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

// max / sum over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48)
// on the VALU lane-swap instructions of gfx950 (v_permlane32_swap,
// v_permlane16_swap), so the reduction does not queue behind LDS traffic.
// With both operands equal, permlane32_swap leaves halves {lo, lo} and
// {hi, hi}; combining the two results gives every lane f(v[l], v[l ^ 32]).
// permlane16_swap does the same for odd/even rows of 16 lanes.
template <typename F>
__device__ __forceinline__ float reduce_over_lane_groups(float v, F f)
{
    const unsigned u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = f(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const unsigned w = __float_as_uint(v);
    const auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return f(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float max_over_lane_groups(float v)
{
    return reduce_over_lane_groups(v, [](float x, float y) { return fmaxf(x, y); });
}

__device__ __forceinline__ float sum_over_lane_groups(float v)
{
    return reduce_over_lane_groups(v, [](float x, float y) { return x + y; });
}

// Global stores with the nontemporal bit, as inline asm: a store the
// compiler knows (__builtin_nontemporal_store) that sits in one branch of a
// runtime choice is merged with a plain store of the same value and address
// in the other branch, and the hint is dropped. No memory clobber: they are
// for results that nothing in the storing kernel reads back, so other
// accesses may move across them.
__device__ __forceinline__ void store_nt(float *p, float v)
{
    asm volatile("global_store_dword %0, %1, off nt" ::"v"(p), "v"(v));
}
// A store of more than 64 bits of data reads its data VGPRs after issue: on
// gfx950 a VALU write to those registers needs two wait states after the
// store. The compiler inserts them for stores it generates but cannot see
// into inline asm, so the asm carries them itself (s_nop 1). Without them a
// VALU that reused the registers right after the store corrupted the first
// two dwords of some lanes' 16 bytes (measured: fp32 partials of a few
// lanes per slot, depending on the schedule).
__device__ __forceinline__ void store_nt(floatx4 *p, floatx4 v)
{
    asm volatile("global_store_dwordx4 %0, %1, off nt\n\ts_nop 1" ::"v"(p), "v"(v));
}
template <typename V4>  // 4 x 16-bit elements
__device__ __forceinline__ void store_nt8(V4 *p, V4 v)
{
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    asm volatile("global_store_dwordx2 %0, %1, off nt" ::"v"(p), "v"(__builtin_bit_cast(u32x2, v)));
}

// Offset (in floats) of O[head][dim] within one slot of the fp32 partial
// output: 16 x 16 tiles (16 heads x 16 value dims) stored in the MFMA
// accumulator order, lane (16 * g + head % 16) holding dims 4g .. 4g+3 of
// the tile, so that one wave writes or reads a tile as 1 KB of contiguous
// memory. Tiles are ordered [head / 16][dim / 16].
__host__ __device__ __forceinline__ size_t frag_offset(int head, int dim)
{
    return ((size_t)(head >> 4) * 32 + (dim >> 4)) * 256 + (((dim & 15) >> 2) * 16 + (head & 15)) * 4 + (dim & 3);
}

// Chunk bounds of a batch (cu_seqlens [batch + 1]), computed by one wave
// (all 64 lanes active). Sequence b's tokens [cu[b], cu[b+1]) take the
// virtual positions [cu[b] + seq_cost (b + 1), cu[b+1] + seq_cost (b + 1)):
// every sequence start adds seq_cost virtual tokens, the measured cost of
// starting a piece in tokens of steady-state work. Returns the first
// sequence whose virtual end exceeds x (batch if none) and sets t to the
// first real token at or after virtual position x (total if none), and
// seq_lo / seq_hi to that sequence's bounds (total if none). cu_seqlens
// entries are clamped as the kernels' piece walks clamp them.
__device__ __forceinline__ int seq_virtual_bound(const int *cu, int batch, int total, int seq_cost, long long x,
                                                 int lane, int &t, int &seq_lo, int &seq_hi)
{
    for (int base = 0; base < batch; base += 64) {
        const int i = base + lane;
        bool past = false;
        int lo_i = 0, hi_i = 0;
        if (i < batch) {
            lo_i = min(max(cu[i], 0), total);
            hi_i = min(max(cu[i + 1], lo_i), total);
            past = (long long)hi_i + (long long)seq_cost * (i + 1) > x;
        }
        const unsigned long long m = __builtin_amdgcn_ballot_w64(past);
        if (m != 0) {
            const int k = __builtin_ctzll(m);
            seq_lo = __builtin_amdgcn_readlane(lo_i, k);
            seq_hi = __builtin_amdgcn_readlane(hi_i, k);
            const long long v = x - (long long)seq_cost * (base + k + 1);
            t = v > seq_lo ? (int)v : seq_lo;
            return base + k;
        }
    }
    t = seq_lo = seq_hi = total;
    return batch;
}

}  // namespace mla
