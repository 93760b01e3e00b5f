// fp32 split-KV MLA decode for gfx950 (the --fp32 path): same math and the
// same partial tile layout as the fp16 kernel, with O kept unnormalised in
// fp32, on fp32 MFMAs (16x16x4f32) so that products and sums keep fp32
// precision end to end.
//
// Replaces mla_decode_fused (reference csrc/mla_decode_fused_fwd.cuh:50-352,
// launcher csrc/mla_decode_fused_fwd_sm89.cu:6-60), which ran one CTA per 16
// heads over the whole sequence (8 CTAs at 128 heads). Here the sequence is
// split so the grid fills the GPU, and the splits are merged by
// mla_combine.hip.
//
// Workgroup = 4 wave64s, 16 heads, blocks of 16 tokens:
//  * S^T = C Q*^T: wave w owns K-quarter [144w, 144w + 144) of the 16x16 tile
//    (its Q* slice stays in VGPRs); the four partial tiles are summed through
//    LDS. Each lane reads 4 consecutive K of both operands with one 16-byte
//    LDS read and feeds them to 4 MFMAs (the same K permutation on A and B).
//  * every wave then redoes the (tiny) softmax of the 16x16 tile, so all of
//    them hold the running max and sum; wave 0 publishes P.
//  * O^T = C_N^T P^T: wave w owns 128 output columns, read from LDS as
//    16-byte runs: MFMA tile t (0..3) of half h takes as its row i the
//    value dim 128w + 64h + 4i + t, so one ds_read_b128 of dims
//    128w + 64h + 4i .. +3 feeds four MFMAs and the 16 lanes of a token row
//    read 256 contiguous bytes. (Single floats at 16 consecutive dims, four
//    token rows per instruction, put two rows on the same LDS banks.) The
//    store undoes the permutation: lane (head j, g) of the four tiles holds
//    the 16 dims of natural tile 8w + 4h + g.
#include "mla_device.hpp"
#include "mla_internal.hpp"
#include "mla_ring.hpp"

namespace mla {

#ifdef MLA_TIMELINE
// Timeline build only (see mla_splitkv_fp16.hip): per workgroup of the fp32
// kernel, wave 0 records s_memrealtime at entry, at the first block, at the
// end of the block loop and after the partial store (stores complete), and
// s_memtime sums over the blocks of its three phases: the first product (to
// the barrier after the partial logits), the softmax and C staging (to the
// next barrier) and the second product.
constexpr int kTimelineWorkgroupsF32 = 8192;
__device__ unsigned long long mla_timeline_stamps_f32[kTimelineWorkgroupsF32 * 16];
#define MLA_STAMP32(e, v)                                                                  \
    do {                                                                                   \
        if (wave == 0 && lane == 0 && blockIdx.x < kTimelineWorkgroupsF32)                 \
            mla_timeline_stamps_f32[blockIdx.x * 16 + (e)] = (unsigned long long)(v);      \
    } while (0)
#define MLA_MT32() __builtin_amdgcn_s_memtime()
#else
#define MLA_STAMP32(e, v) \
    do {                  \
    } while (0)
#endif

namespace {

constexpr int kHT = 16;                  // heads per workgroup
constexpr int kBT = 16;                  // tokens per block
constexpr int kRow = kDK + 4;            // LDS row stride (floats): 2320 B
constexpr int kRowChunks = kDK / 4;      // 16-byte chunks per row
constexpr int kStage = kBT * kRowChunks / 256;
constexpr int kKQ = kDK / 4;             // K per wave (144)
constexpr int kPRow = kBT + 4;
// partial S^T tiles [wave][token][head] with rows of 20 floats: the four
// token rows a write or read instruction touches then start 16 banks apart
// (rows of 16 put all four on the same 16 banks)
constexpr int kSRow = kHT + 4;
static_assert(kBT * kRowChunks % 256 == 0, "stage split");

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))
void splitkv_fp32_kernel(const float *__restrict__ q,
                         const float *__restrict__ c,
                         const int *__restrict__ cu_seqlens,
                         float *__restrict__ o_part,
                         float *__restrict__ m_part,
                         float *__restrict__ l_part,
                         int num_heads, int batch, int total_tokens, int chunk,
                         int n_head_tiles, int xcd_remap, float scale_log2)
{
    __shared__ __attribute__((aligned(16))) float s_c[2 * kBT * kRow];
    __shared__ __attribute__((aligned(16))) float s_s[4 * kBT * kSRow];
    __shared__ float s_p[kHT * kPRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l16 = lane & 15;
    const int g = lane >> 4;
    MLA_STAMP32(0, __builtin_amdgcn_s_memrealtime());
#ifdef MLA_TIMELINE
    unsigned long long ph_s = 0, ph_x = 0, ph_o = 0, tm = 0;
#endif

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
    if ((long long)split * chunk >= total_tokens)  // a padding workgroup of the grid
        return;
    const int lo = split * chunk;
    const int hi = min(lo + chunk, total_tokens);
    const int head0 = ht * kHT;

    int b = 0;
    const int nseq = cu_seqlens ? batch : 1;
    if (cu_seqlens) {
        int l = 0, r = batch;
        while (r - l > 1) {
            const int mid = (l + r) >> 1;
            if (cu_seqlens[mid] <= lo) l = mid; else r = mid;
        }
        b = l;
    }

    for (; b < nseq; ++b) {
        int seq_lo = 0, seq_hi = total_tokens;
        if (cu_seqlens) {
            seq_lo = min(max(cu_seqlens[b], 0), total_tokens);
            seq_hi = min(max(cu_seqlens[b + 1], seq_lo), total_tokens);
        }
        if (seq_lo >= hi)
            break;
        const int p_lo = max(seq_lo, lo);
        const int p_hi = min(seq_hi, hi);
        if (p_lo >= p_hi)
            continue;
        const int slot = split + b;
        const int nblk = (p_hi - p_lo + kBT - 1) / kBT;

        __syncthreads();

        // Q* slice: head head0 + l16, dims kKQ*wave + 16*kq + 4*g .. +3
        floatx4 qf[kKQ / 16];
        {
            const float *qrow = q + ((size_t)b * num_heads + head0 + l16) * kDK + kKQ * wave + 4 * g;
#pragma unroll
            for (int kq = 0; kq < kKQ / 16; ++kq)
                qf[kq] = *(const floatx4 *)(qrow + 16 * kq);
        }

        floatx4 stage[kStage];
        auto load_stage = [&](int t0) {
#pragma unroll
            for (int s = 0; s < kStage; ++s) {
                const int ci = tid + 256 * s;
                const int tok = ci / kRowChunks;
                const int col = ci - tok * kRowChunks;
                const int gt = t0 + tok;
                if (gt < p_hi)
                    stage[s] = *(const floatx4 *)(c + (size_t)gt * kDK + col * 4);
                else
                    stage[s] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        };
        auto store_stage = [&](int which) {
            float *dst = s_c + which * kBT * kRow;
#pragma unroll
            for (int s = 0; s < kStage; ++s) {
                const int ci = tid + 256 * s;
                const int tok = ci / kRowChunks;
                const int col = ci - tok * kRowChunks;
                *(floatx4 *)(dst + tok * kRow + col * 4) = stage[s];
            }
        };

        load_stage(p_lo);
        store_stage(0);
        if (nblk > 1)
            load_stage(p_lo + kBT);

        float m_run = -INFINITY, l_run = 0.f;
        floatx4 o[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
            o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

        __syncthreads();
        MLA_STAMP32(1, __builtin_amdgcn_s_memrealtime());
        MLA_STAMP32(11, nblk);

        for (int blk = 0; blk < nblk; ++blk) {
#ifdef MLA_TIMELINE
            tm = MLA_MT32();
#endif
            const int cur = blk & 1;
            const int t0 = p_lo + blk * kBT;
            const float *cs = s_c + cur * kBT * kRow;

            // ---- partial S^T over this wave's K-quarter
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            {
                const float *arow = cs + l16 * kRow + kKQ * wave + 4 * g;
#pragma unroll
                for (int kq = 0; kq < kKQ / 16; ++kq) {
                    const floatx4 a = *(const floatx4 *)(arow + 16 * kq);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc = mfma16x16x4f32(a[j], qf[kq][j], acc);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                s_s[(wave * kBT + 4 * g + i) * kSRow + l16] = acc[i];
            __syncthreads();
#ifdef MLA_TIMELINE
            { const unsigned long long t2 = MLA_MT32(); ph_s += t2 - tm; tm = t2; }
#endif

            // ---- full tile, softmax (every wave, identical results)
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = (4 * g + i) * kSRow + l16;
                const float sdot = ((s_s[r] + s_s[kBT * kSRow + r]) + s_s[2 * kBT * kSRow + r]) + s_s[3 * kBT * kSRow + r];
                sv[i] = (t0 + 4 * g + i) < p_hi ? sdot * scale_log2 : -INFINITY;
                mx = fmaxf(mx, sv[i]);
            }
            mx = max_over_lane_groups(mx);
            const float mn = fmaxf(m_run, mx);
            const float alpha = fast_exp2(m_run - mn);
            m_run = mn;
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = fast_exp2(sv[i] - mn);
                psum += p;
                if (wave == 0)
                    s_p[l16 * kPRow + 4 * g + i] = p;
            }
            l_run = l_run * alpha + psum;

            if (blk + 1 < nblk)
                store_stage(cur ^ 1);
            if (blk + 2 < nblk)
                load_stage(t0 + 2 * kBT);
            __syncthreads();
#ifdef MLA_TIMELINE
            { const unsigned long long t2 = MLA_MT32(); ph_x += t2 - tm; tm = t2; }
#endif

            // ---- O^T[dims 128*wave .. +128][heads] += C_N^T P^T; o[4h + t]
            // row i is dim 128*wave + 64h + 4i + t
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                o[dt] *= alpha;
#pragma unroll
            for (int ks = 0; ks < kBT / 4; ++ks) {
                const float pbv = s_p[l16 * kPRow + 4 * ks + g];
                const float *crow = cs + (4 * ks + g) * kRow + 128 * wave + 4 * l16;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const floatx4 a = *(const floatx4 *)(crow + 64 * h);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        o[4 * h + t] = mfma16x16x4f32(a[t], pbv, o[4 * h + t]);
                }
            }
#ifdef MLA_TIMELINE
            { const unsigned long long t2 = MLA_MT32(); ph_o += t2 - tm; }
#endif
        }
        MLA_STAMP32(2, __builtin_amdgcn_s_memrealtime());
#ifdef MLA_TIMELINE
        MLA_STAMP32(6, ph_s);
        MLA_STAMP32(7, ph_x);
        MLA_STAMP32(8, ph_o);
#endif

        const float lsum = sum_over_lane_groups(l_run);
        if (tid < kHT) {
            __builtin_nontemporal_store(m_run, m_part + (size_t)slot * num_heads + head0 + tid);
            __builtin_nontemporal_store(lsum, l_part + (size_t)slot * num_heads + head0 + tid);
        }
        // in the MFMA accumulator order of natural 16 x 16 tiles (frag_offset):
        // lane (head j, g) holds, over o[4h .. 4h+3], dims 16g .. 16g+15 of
        // tile 8*wave + 4h + g, element r of o[4h + t] being dim 4r + t of
        // it; each store writes 4 runs of 256 contiguous bytes. Nontemporal,
        // as the partials are read once, by the combine (see
        // mla_splitkv_fp16.hip)
        float *obase = o_part + (size_t)slot * num_heads * kDV;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const floatx4 v = {o[4 * h][r], o[4 * h + 1][r], o[4 * h + 2][r], o[4 * h + 3][r]};
                __builtin_nontemporal_store(
                    v, (floatx4 *)(obase + frag_offset(head0 + l16, 128 * wave + 64 * h + 16 * g + 4 * r)));
            }
#ifdef MLA_TIMELINE
        MLA_WAIT_VMCNT(0);
#endif
        MLA_STAMP32(3, __builtin_amdgcn_s_memrealtime());
    }
}

}  // namespace

hipError_t launch_splitkv_fp32(const Problem &pb, const Plan &p, const Partials &w, hipStream_t s)
{
    if (p.n_chunks == 0)
        return hipSuccess;
    const dim3 grid(grid_chunks(p) * p.n_head_tiles), block(256);
    hipLaunchKernelGGL(splitkv_fp32_kernel, grid, block, 0, s,
                       (const float *)pb.q, (const float *)pb.c, pb.cu_seqlens,
                       static_cast<float *>(w.o), w.m, w.l, pb.num_heads, pb.batch, pb.total_tokens,
                       p.chunk, p.n_head_tiles, p.xcd_remap, pb.scale_log2);
    // the launch's own error; hipPeekAtLastError leaves a sticky error from
    // the caller's earlier work in place for the caller to see
    return hipPeekAtLastError();
}

}  // namespace mla

#ifdef MLA_TIMELINE
extern "C" int mla_timeline_read_f32(void *dst, size_t bytes)
{
    const size_t n = bytes < sizeof(mla::mla_timeline_stamps_f32) ? bytes : sizeof(mla::mla_timeline_stamps_f32);
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(mla::mla_timeline_stamps_f32), n, 0, hipMemcpyDeviceToHost);
}
#endif
