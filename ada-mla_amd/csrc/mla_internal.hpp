// Host-side plan and launch interface shared by the kernel translation units
// and the C ABI (mla_capi.hip). Not installed; callers use include/mla_mi355x.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace mla {

constexpr int kDK = 576;  // latent + rope width of Q* and C
constexpr int kDV = 512;  // value width (C_N = C[:, :512])

// Split-KV schedule. The packed token range [0, total_tokens) is cut into
// n_chunks chunks of `chunk` tokens; workgroup (chunk w, head tile h) handles
// heads [h * head_tile, +head_tile) over the tokens of chunk w. With
// cu_seqlens the cut is over virtual positions: token t of sequence b sits
// at t + seq_cost (b + 1) and chunk w holds the tokens whose virtual
// positions fall in [w chunk, (w + 1) chunk). A chunk that spans sequences
// b..b' emits one partial result per sequence; the partial of (chunk w,
// sequence b) lives in slot w + b, so slots never collide and a sequence's
// partials are the contiguous slots
// [(lo_b + c_b) / chunk + b, (hi_b - 1 + c_b) / chunk + b], c_b = seq_cost (b + 1).
struct Plan {
    int head_tile;     // heads per workgroup
    int n_head_tiles;  // num_heads / head_tile
    int block_tokens;  // tokens per LDS block
    int chunk;         // tokens per split (virtual tokens with cu_seqlens; a multiple of
                       // block_tokens)
    int n_chunks;      // splits over the packed tokens
    int n_slots;       // partial-result slots: n_chunks + batch - 1
    int xcd_remap;     // 1: the head tiles of one chunk share an XCD; the grid then
                       // holds grid_chunks() chunks (n_chunks padded to a multiple of 8)
    int part_bytes;    // bytes per partial O element: 2 (16-bit paths), 4 (fp32 path, or 16-bit
                       // paths with fp32 partials)
    int merge;         // kMergeCombine: combine_kernel merges the partials (a second launch);
                       // kMergeDirect: one chunk, the split kernel writes the output itself
    int part_plain;    // 1: the 16-bit split kernel stores its partials with plain stores,
                       // 0: with nontemporal ones (see choose_part_plain)
    int seq_cost;      // calls with cu_seqlens: virtual tokens each sequence start adds, so
                       // that chunks of `chunk` virtual tokens carry equal work with their
                       // piece starts (seq_virtual_bound in mla_device.hpp); 0 otherwise
};

constexpr int kMergeCombine = 0;
constexpr int kMergeDirect = 1;

// Chunks in the split kernels' launch grid: with xcd_remap, workgroup b
// takes chunk (b / 8 / n_head_tiles) * 8 + b % 8, so the grid is padded to a
// multiple of 8 chunks; the padding workgroups find no tokens and exit.
inline int grid_chunks(const Plan &p) { return p.xcd_remap ? (p.n_chunks + 7) / 8 * 8 : p.n_chunks; }

// Partial results of the split kernels: O in n_slots blocks of
// num_heads x 512 elements, each stored as 16 x 16 tiles in MFMA accumulator
// order (frag_offset in mla_device.hpp), then the running max in log2 units
// and the running sum [n_slots][num_heads] (fp32). The 16-bit paths store O
// normalised by its running sum, in the input type (fp16 or bf16: the
// softmax-weighted mean of the piece's C_N rows, bounded by the largest |C|
// entry); the fp32 path stores O unnormalised, in fp32.
struct Partials {
    void *o;
    float *m;
    float *l;
};

// Paged KV cache: token l of sequence b is row (l mod 2^page_shift) of page
// block_table[b * bt_stride + (l >> page_shift)] of a cache of num_pages
// pages [2^page_shift][576]. block_table == nullptr: the packed layout.
struct Paging {
    const int *block_table;
    int page_shift;
    int bt_stride;
    int num_pages;
};

struct Problem {
    const void *q;          // [batch][num_heads][576]
    const void *c;          // [total_tokens][576]
    const int *cu_seqlens;  // [batch + 1] on device, or nullptr for one sequence
    void *out;              // [batch][num_heads][512]
    int batch;
    int num_heads;
    int total_tokens;
    float scale_log2;       // softmax scale * log2(e)
    bool fp32;              // fp32 path (q, c, out fp32; unnormalised fp32 partials)
    bool bf16;              // 16-bit path: q, c, out (and the partial O) in bf16, not fp16
    Paging paging;          // c is a paged cache when paging.block_table != nullptr
    bool fp8;               // c is OCP fp8 (E4M3FN) with per-tensor scale c_scale (q, out fp16)
    float out_scale;        // multiplies the normalised partial O (c_scale for fp8, else 1)
};

// Layout of the cache the plan is for. kPaged: one extra block per piece in
// the cost model (pieces start page-aligned). kF8: charged the same extra
// block, a stand-in for the operand conversions that lengthen its steps.
enum class CacheKind { kPacked, kPaged, kF8 };

// CUs of the current device (cached per device); 256 if it cannot be queried.
int current_cu_count();

// Records e as this host thread's last HIP error (mla_last_hip_error) and
// returns MLA_STATUS_HIP_ERROR.
int record_hip_error(hipError_t e);

// seqlens: the call passes cu_seqlens (a batch, possibly of one sequence);
// only a single sequence without cu_seqlens can take the one-launch plan.
Plan make_plan(bool fp32, int num_heads, int total_tokens, int batch, bool seqlens,
               int num_splits, int cu_count, CacheKind cache = CacheKind::kPacked,
               bool f32_partials = false);
size_t partials_bytes(const Plan &p, int num_heads);
Partials carve_partials(void *ws, const Plan &p, int num_heads);

hipError_t launch_splitkv_fp16(const Problem &pb, const Plan &p,
                               const Partials &w, bool tr_load, hipStream_t s);
hipError_t launch_splitkv_fp32(const Problem &pb, const Plan &p,
                               const Partials &w, hipStream_t s);
// The output has the partials' type: fp16 / bf16 on the 16-bit path, fp32
// on the fp32 path.
// Workgroups of the combine launch for plan p (batch sequences, num_heads).
int combine_workgroups(const Plan &p, int batch, int num_heads, int cu_count);
// The combine's form for n_items (16 x 16 tile, sequence) items: W > 0 waves
// per item, 0 for tile groups (more items than resident waves), -W for
// quarter items.
int combine_waves_per_item(const Plan &p, int batch, int n_items, int cu_count);

hipError_t launch_combine(const Problem &pb, const Plan &p, const Partials &w,
                          hipStream_t s);

}  // namespace mla
