// The LDS ring of the split-KV decode kernels: slot layout and swizzles,
// the direct global->LDS load, and the barrier and counter waits the
// kernels order those loads with.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mla {

// The O accumulators' reference max (log2 units) is moved only when a
// block's max exceeds it by more than this; P scaled onto the reference is
// then at most 2^8.
constexpr float kLazyRescale = 8.0f;

// Ring slot layout (32 rows: tokens of a block, or heads of Q*): the C_N
// part of row r (chunks 0..63, 16 bytes each) at byte r * 1024, the rope
// part (chunks 64..71) in a separate area at 32 KB + r * 128, so that a
// global->LDS load unit (64 chunks) is exactly one C_N row or 8 rope rows.
// Chunks are XOR-swizzled within a row:
//  - C_N: chunk c of row r sits at c ^ (r mod 16). Rows are 1024 bytes, a
//    multiple of the LDS bank period, so only the swizzle spreads the reads.
//    Measured on gfx950 (rocprofv3 SQ_LDS_BANK_CONFLICT on probe kernels of
//    each access pattern): the first product's 16-byte row reads (lane
//    16g + i: row i, logical chunk 4j + g) are conflict-free when bit 0 of
//    the stored chunk varies with the row's low two bits, and the transpose
//    reads are conflict-free when it is the same for all rows of one
//    instruction. Both hold with this swizzle because the second product
//    takes its K (token) order as 8g + {0,2,4,6} (first transpose read) and
//    8g + {1,3,5,7} (second): each transpose read touches rows of one
//    parity. P's columns follow the same token order (see the P write in the S waves).
//  - rope: chunk 64 + c' of row r sits at c' ^ rope_swizzle(r); rows are
//    128 bytes, so rows r and r+1 share a bank period and the swizzle
//    (r / 2) mod 8 separates the 8 row pairs of 16 consecutive rows.
__device__ __forceinline__ int row_swizzle(int row)
{
    return row & 15;
}

__device__ __forceinline__ int rope_swizzle(int row)
{
    return (row >> 1) & 7;
}

// fp8 cache: byte offset of the rope parts within a ring slot (after 32
// C_N rows of 512 bytes).
constexpr int kF8Rope = 16384;

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
__device__ __forceinline__ void global_to_lds16(const void *base, int off, const void *lds)
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

// The same load with the LDS destination given as a wave-uniform LDS byte
// address, for the steady-state feeding: its lane offsets are formed once and
// kept in registers of their own. Offsets recomputed into one shared register
// before every load made each load's address arithmetic wait until the
// previous load had read that register.
__device__ __forceinline__ void global_to_lds16_at(const void *base, int off, unsigned lds_addr)
{
    unsigned saved_m0;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %3\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved_m0) : "v"(off), "s"(base), "s"(lds_addr) : "memory");
}

}  // namespace mla
