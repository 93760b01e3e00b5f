/*
 * mla_mi355x.h -- C ABI of the MI355X (gfx950) weight-absorbed MLA decode:
 *
 *     O*[h, :] = softmax_t( Q*[h, :] . C[t, :] / sqrt(192) ) . C[t, :512]
 *
 * with Q* [num_heads x 576], the latent cache C [N x 576] (first 512 columns
 * are C_N, the last 64 the rope part) and O* [num_heads x 512].
 *
 * This is the drop-in boundary below the PyTorch extension: the reference's
 * extension (csrc/mla_api.cpp) calls raw-pointer launchers declared in
 * csrc/mla_decode.hpp; the entry points here are what it would bind instead.
 *
 * Conventions (all entry points):
 *  - Plain device pointers, row-major and contiguous, 16-byte aligned.
 *  - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *    asynchronously; nothing synchronises, nothing allocates.
 *  - The caller owns the workspace; query its size with the matching
 *    *_workspace_size function (same arguments, same current device).
 *    Calls that share one workspace must not overlap in time.
 *  - `num_splits` <= 0 picks the split count from the sequence length and
 *    the device's CU count; > 0 requests that many splits (clamped so every
 *    split holds at least one LDS block).
 *  - Return value: MLA_STATUS_SUCCESS (0) or one of the codes below; nothing
 *    is enqueued when a code other than 0 or MLA_STATUS_HIP_ERROR is
 *    returned. Thread-safe. Shared state: a per-device cache of the CU
 *    count and a per-device cache of the allocation-free entry point's
 *    scratch address (each written once per device). Per host thread: the
 *    last HIP error and the last few split plans.
 *  - num_heads must be a positive multiple of 16.
 */
#ifndef MLA_MI355X_H
#define MLA_MI355X_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLA_HEAD_DIM_K 576 /* mla.py:33 HEAD_DIM_K = HEAD_DIM_C + HEAD_DIM_ROPE */
#define MLA_HEAD_DIM_V 512 /* mla.py:31 HEAD_DIM_C */
#define MLA_ABI_VERSION 2 /* 2: mla_project_output_workspace_size takes d_model; status 5 added */

#define MLA_STATUS_SUCCESS 0
#define MLA_STATUS_INVALID_VALUE 1       /* null pointer or unsupported size */
#define MLA_STATUS_MISALIGNED 2          /* a pointer is not 16-byte aligned */
#define MLA_STATUS_WORKSPACE_TOO_SMALL 3 /* workspace_bytes below the size query */
#define MLA_STATUS_HIP_ERROR 4           /* a HIP launch failed: mla_last_hip_error() */
#define MLA_STATUS_SCRATCH_EXCEEDED 5    /* mla_decode_split_fp16_noalloc: partials exceed its scratch */

/* Size of the device array that holds the split partials of
 * mla_decode_split_fp16_noalloc (one per GPU the library runs on). */
#define MLA_NOALLOC_SCRATCH_BYTES (32u << 20)

/* Testing aid for mla_decode_split_fp16_ex: read the C_N^T operand of the
 * second product with scalar LDS loads instead of the LDS transpose read. */
#define MLA_FLAG_SCALAR_TRANSPOSE 1u

/* mla_decode_split_fp16_ex / _partials / _combine: keep the split partials
 * in fp32 instead of the input type (twice the partial traffic; the combine
 * must be given the same flag as the split phase). The workspace size
 * queries cover both precisions. */
#define MLA_FLAG_FP32_PARTIALS 4u

/* A single-sequence 16-bit call (mla_decode_split_fp16/_ex, _bf16, _fp8 and
 * the allocation-free entry point) whose plan has one split is ONE launch:
 * the split kernel writes the output itself, with no partials and no
 * combine (the planner prefers one split for short sequences, about
 * 200 tokens or fewer at 128 heads, for that reason). This flag keeps the
 * reference's two launches in that case too: split kernel, then the LSE
 * combine (csrc/mla_decode_splitk_fwd.cuh:973-978). */
#define MLA_FLAG_TWO_LAUNCHES 8u

/* Plan queries only (mla_decode_split_num_splits, _head_tile, _launches):
 * report the plan of the fp8-cache entry mla_decode_split_fp8 for these
 * sizes. Its cache streams half the bytes of a 16-bit one, so with few heads
 * and long sequences its plan can take more splits, or another head tile,
 * than the 16-bit plan. The decode entry points ignore it. */
#define MLA_FLAG_FP8_CACHE 16u

int mla_abi_version(void);
const char *mla_status_string(int status);
/* hipError_t of the last failed HIP call on this thread (0 if none). */
int mla_last_hip_error(void);

/* Number of splits (partial results per head) that mla_decode_split_fp16_ex
 * (with MLA_FLAG_FP8_CACHE: mla_decode_split_fp8) uses for these arguments
 * and flags on the current device; 0 for invalid sizes.
 * Replaces the fixed `num_splits = 4` of mla_decode_split
 * (csrc/mla_api.cpp:97). */
int mla_decode_split_num_splits(int num_heads, int seq_length, int num_splits,
                                unsigned flags);

/* Heads per workgroup (16, 32 or 64) of the plan that
 * mla_decode_split_fp16_ex (with MLA_FLAG_FP8_CACHE: mla_decode_split_fp8)
 * uses for these arguments and flags on the current device; 0 for invalid
 * sizes.
 * With an fp8 cache, tiles of 32 or 64 heads run the first product on fp8
 * MFMAs (Q* split in two fp8 parts), tiles of 16 convert C to fp16. No
 * counterpart in the reference. */
int mla_decode_split_head_tile(int num_heads, int seq_length, int num_splits,
                               unsigned flags);

/* Kernel launches (1 or 2, see MLA_FLAG_TWO_LAUNCHES) that
 * mla_decode_split_fp16_ex (with MLA_FLAG_FP8_CACHE: mla_decode_split_fp8)
 * makes for these arguments and flags on the current device; 0 for invalid sizes. No counterpart in the reference, whose
 * launcher always makes two (csrc/mla_decode_splitk_fwd.cuh:973-978). */
int mla_decode_split_launches(int num_heads, int seq_length, int num_splits,
                              unsigned flags);

/* Workspace for mla_decode_split_fp16 (split partials: O normalised by its
 * running sum in fp16, running max and sum in fp32). Replaces the
 * splits_max / splits_sum / splits_out buffers that mla_decode_split_
 * allocates per call (csrc/mla_api.cpp:71-75). Returns 0 for invalid sizes. */
size_t mla_decode_split_workspace_size(int num_heads, int seq_length,
                                       int num_splits);

/* fp16 split-KV decode: query [num_heads x 576] fp16, cache [seq_length x 576]
 * fp16 -> out [num_heads x 512] fp16; fp32 accumulation and softmax state,
 * fp16 normalised partials merged in fp32. Replaces run_mla_decode_splitk<at::Half>
 * (csrc/mla_decode.hpp:25-34; csrc/mla_decode_splitk_fwd_sm89.cu:26-47 ->
 * run_mla_decode_splitk_fp16, csrc/mla_decode_splitk_fwd.cuh:941-985), which
 * took three caller buffers, no stream, and required num_heads == 128 and
 * seq_length % 64 == 0. */
int mla_decode_split_fp16(const void *query, const void *cache, void *out,
                          void *workspace, size_t workspace_bytes,
                          int num_heads, int seq_length, int num_splits,
                          void *stream);

/* mla_decode_split_fp16 with flags (MLA_FLAG_*). */
int mla_decode_split_fp16_ex(const void *query, const void *cache, void *out,
                             void *workspace, size_t workspace_bytes,
                             int num_heads, int seq_length, int num_splits,
                             unsigned flags, void *stream);

/* mla_decode_split_fp16 without a workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The split
 * partials go to a file-scope device array of MLA_NOALLOC_SCRATCH_BYTES
 * (32 MiB) that each GPU holds until the process ends; its device address is
 * looked up (hipGetSymbolAddress) on the first call on each device. The call
 * allocates nothing and launches the same kernels with the same split plan
 * as mla_decode_split_fp16, so the results are identical. Every call on one
 * GPU shares that GPU's array: calls that overlap in time on one GPU (other
 * streams, other threads) race. Nothing in the array needs clearing: each
 * call writes every partial it reads. Returns MLA_STATUS_SCRATCH_EXCEEDED
 * when the plan's partials would not fit (not for any num_splits <= 0 plan
 * on a GPU of up to 256 CUs: those stay below 17 MiB). */
int mla_decode_split_fp16_noalloc(const void *query, const void *cache,
                                  void *out, int num_heads, int seq_length,
                                  int num_splits, void *stream);

/* The two launches of mla_decode_split_fp16, one at a time: the split-KV
 * kernel, which leaves its partials in the workspace, then the LSE combine,
 * which merges them into out. Called back to back on one stream with the
 * same num_heads / seq_length / num_splits they equal mla_decode_split_fp16
 * (the reference's launcher makes the same two launches,
 * csrc/mla_decode_splitk_fwd.cuh:973-978); apart, they let a caller place
 * other work or timing events between the phases. */
int mla_decode_split_fp16_partials(const void *query, const void *cache,
                                   void *workspace, size_t workspace_bytes,
                                   int num_heads, int seq_length,
                                   int num_splits, unsigned flags,
                                   void *stream);
int mla_decode_split_fp16_combine(const void *workspace,
                                  size_t workspace_bytes, void *out,
                                  int num_heads, int seq_length,
                                  int num_splits, unsigned flags,
                                  void *stream);

/* Workspace for mla_decode_fused_fp32. */
size_t mla_decode_fused_workspace_size(int num_heads, int seq_length,
                                       int num_splits);

/* fp32 decode: query [num_heads x head_dim_c] fp32, cache
 * [seq_length x head_dim_c] fp32 -> out [num_heads x 512] fp32, fp32
 * products. head_dim_c must be 576. Replaces run_mla_decode_fused
 * (csrc/mla_decode.hpp:17-22; csrc/mla_decode_fused_fwd_sm89.cu:6-60), which
 * needed num_heads % 16 == 0 and seq_length % 16 == 0 and no workspace. */
int mla_decode_fused_fp32(const float *query, const float *cache, float *out,
                          void *workspace, size_t workspace_bytes,
                          int num_heads, int head_dim_c, int seq_length,
                          int num_splits, void *stream);

/* Workspace for mla_decode_split_batched_fp16. */
size_t mla_decode_split_batched_workspace_size(int batch, int num_heads,
                                               int total_tokens,
                                               int num_splits);

/* Batched variable-length fp16 decode (no reference counterpart: the
 * reference handles one sequence per call, csrc/mla_api.cpp:67-69).
 * query [batch x num_heads x 576] fp16; cache = the sequences' caches packed
 * back to back [total_tokens x 576] fp16; cu_seqlens [batch + 1] int32 on the
 * device with cu_seqlens[0] = 0, non-decreasing, cu_seqlens[batch] =
 * total_tokens (sequence b owns rows cu_seqlens[b] .. cu_seqlens[b+1]-1);
 * out [batch x num_heads x 512] fp16. Empty sequences give zero rows. The
 * splits are cut over the packed tokens, so work is balanced whatever the
 * length mix. Values of cu_seqlens outside [0, total_tokens] are clamped. */
int mla_decode_split_batched_fp16(const void *query, const void *cache,
                                  const int *cu_seqlens, void *out,
                                  void *workspace, size_t workspace_bytes,
                                  int batch, int num_heads, int total_tokens,
                                  int num_splits, void *stream);

/* The two launches of mla_decode_split_batched_fp16, one at a time, as
 * mla_decode_split_fp16_partials / _combine are for one sequence: the
 * split-KV kernel leaves the partials in the workspace, the combine merges
 * them into out. Called back to back on one stream with the same sizes they
 * equal mla_decode_split_batched_fp16. No reference counterpart (the
 * reference decodes one sequence per call). */
int mla_decode_split_batched_fp16_partials(const void *query,
                                           const void *cache,
                                           const int *cu_seqlens,
                                           void *workspace,
                                           size_t workspace_bytes, int batch,
                                           int num_heads, int total_tokens,
                                           int num_splits, void *stream);
int mla_decode_split_batched_fp16_combine(const void *workspace,
                                          size_t workspace_bytes,
                                          const int *cu_seqlens, void *out,
                                          int batch, int num_heads,
                                          int total_tokens, int num_splits,
                                          void *stream);

/* bf16 KV cache: mla_decode_split_fp16 and mla_decode_split_batched_fp16
 * with query, cache and out in bf16 (the same workspace sizes; bf16 MFMAs,
 * fp32 accumulation and softmax state, P and the normalised partials in
 * bf16). No reference counterpart: the reference lists bf16 as future work
 * (README.md:405-408) and its --bf16 flag is commented out (mla.py:163). */
int mla_decode_split_bf16(const void *query, const void *cache, void *out,
                          void *workspace, size_t workspace_bytes,
                          int num_heads, int seq_length, int num_splits,
                          void *stream);
int mla_decode_split_batched_bf16(const void *query, const void *cache,
                                  const int *cu_seqlens, void *out,
                                  void *workspace, size_t workspace_bytes,
                                  int batch, int num_heads, int total_tokens,
                                  int num_splits, void *stream);

/* Paged KV cache (no reference counterpart: the reference reads one
 * contiguous cache per call, csrc/mla_api.cpp:67-69). kv_cache is
 * [num_pages x page_size x 576] (fp16 or bf16); token l of sequence b is row
 * l % page_size of page block_table[b * block_table_stride + l / page_size]
 * (int32 on the device). cu_seqlens [batch + 1] (int32, device) holds the
 * prefix sums of the sequence lengths (cu_seqlens[0] = 0, cu_seqlens[batch]
 * = total_tokens), query [batch x num_heads x 576], out
 * [batch x num_heads x 512]; empty sequences give zero rows. page_size is a
 * power of two >= 32. Page ids outside [0, num_pages) and block-table
 * columns beyond block_table_stride are clamped (the result is then
 * meaningless but every access stays inside the caller's buffers). The same
 * split planner as the packed batched entry (head tiles of 16, 32 or 64).
 * total_tokens is not checked against cu_seqlens[batch] (that would need a
 * device read): every sequence's range is clipped to [0, total_tokens), so a
 * total_tokens below cu_seqlens[batch] silently truncates the trailing
 * sequences (their rows cover only their tokens below total_tokens, zeros if
 * none) and still returns MLA_STATUS_SUCCESS; a larger one only changes the
 * split plan. */
size_t mla_decode_paged_workspace_size(int batch, int num_heads,
                                       int total_tokens, int num_splits);
int mla_decode_paged_fp16(const void *query, const void *kv_cache,
                          const int *block_table, const int *cu_seqlens,
                          void *out, void *workspace, size_t workspace_bytes,
                          int batch, int num_heads, int total_tokens,
                          int page_size, int num_pages,
                          int block_table_stride, int num_splits,
                          void *stream);
int mla_decode_paged_bf16(const void *query, const void *kv_cache,
                          const int *block_table, const int *cu_seqlens,
                          void *out, void *workspace, size_t workspace_bytes,
                          int batch, int num_heads, int total_tokens,
                          int page_size, int num_pages,
                          int block_table_stride, int num_splits,
                          void *stream);

/* fp8 KV cache (no reference counterpart: the reference lists it as future
 * work, README.md:408): query [.. x num_heads x 576] fp16, cache
 * [tokens x 576] OCP fp8 E4M3FN bytes holding C / cache_scale (a per-tensor
 * scale > 0), out fp16. The decode reads the cache at one byte per value
 * (half the HBM traffic of fp16), keeps the bytes as they are in LDS and
 * converts each MFMA operand to fp16 after its LDS read (exact: every E4M3FN
 * value is an fp16 value); products and softmax as on the fp16 path. Workspace from
 * mla_decode_split_fp8_workspace_size(batch, num_heads, total_tokens,
 * num_splits) (batch = 1 for the single-sequence entry). cu_seqlens as for
 * mla_decode_split_batched_fp16. */
size_t mla_decode_split_fp8_workspace_size(int batch, int num_heads,
                                           int total_tokens, int num_splits);
int mla_decode_split_fp8(const void *query, const void *cache_fp8,
                         float cache_scale, void *out, void *workspace,
                         size_t workspace_bytes, int num_heads,
                         int seq_length, int num_splits, void *stream);
int mla_decode_split_batched_fp8(const void *query, const void *cache_fp8,
                                 float cache_scale, const int *cu_seqlens,
                                 void *out, void *workspace,
                                 size_t workspace_bytes, int batch,
                                 int num_heads, int total_tokens,
                                 int num_splits, void *stream);

/* The projections around the decode, completing an MLA attention block's
 * decode step (no reference code: the math is README.md:76-85, 104-110).
 * Weights in torch Linear layout: w_uk, w_uv [num_heads][128][512] (the key
 * and value halves of the latent up-projection), w_o [d_model][num_heads*128].
 *
 * mla_absorb_query_*: q_nope [batch][num_heads][128], q_rope
 *   [batch][num_heads][64] -> q_star [batch][num_heads][576] with
 *   q_star[..., :512] = q_nope W_UK[h] and q_star[..., 512:] = q_rope, the
 *   query of mla_decode_split_batched_* / mla_decode_paged_* (no softmax
 *   scale: the decode applies it).
 * mla_project_output_*: o_star [batch][num_heads][512] (the decode's output)
 *   -> out [batch][d_model] = concat_h(o_star[:, h] W_UV[h]^T) W_O^T, with
 *   the per-head values in a caller workspace of
 *   mla_project_output_workspace_size(batch, num_heads, d_model) bytes
 *   (the per-head values, then the output projection's fp32 K-part sums).
 * All three products are MFMA kernels of this library (fp32 accumulation)
 * and allocate nothing: W_UK and W_UV one workgroup per (head, column
 * slice), W_O streamed once from HBM through an LDS ring by at most one
 * workgroup per CU, in K-parts whose fp32 sums a second small kernel adds. */
size_t mla_project_output_workspace_size(int batch, int num_heads, int d_model);
int mla_absorb_query_fp16(const void *q_nope, const void *q_rope,
                          const void *w_uk, void *q_star, int batch,
                          int num_heads, void *stream);
int mla_absorb_query_bf16(const void *q_nope, const void *q_rope,
                          const void *w_uk, void *q_star, int batch,
                          int num_heads, void *stream);
int mla_project_output_fp16(const void *o_star, const void *w_uv,
                            const void *w_o, void *out, void *workspace,
                            size_t workspace_bytes, int batch, int num_heads,
                            int d_model, void *stream);
int mla_project_output_bf16(const void *o_star, const void *w_uv,
                            const void *w_o, void *out, void *workspace,
                            size_t workspace_bytes, int batch, int num_heads,
                            int d_model, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MLA_MI355X_H */
