// A C++ caller of the C ABI (include/mla_mi355x.h) with no Python and no
// torch: plain hipMalloc'd buffers, a HIP stream, and the entry points a
// C/C++ host (the reference's own extension, csrc/mla_api.cpp, or any other
// native caller) would bind. Test infrastructure: it checks the decode
// against the CPU oracle (oracle/mla_naive_cpu.c, the restatement of the
// reference's run_mla_decode_cpu with the decode contract's scale and 512
// value columns) and times the headline call without an interpreter around it.
//
//   abi_client --abi     ABI version and status strings only (no GPU call)
//   abi_client --to-half float bit patterns (hex, stdin) -> binary16 bits and
//                        the float they convert back to (checks the helpers)
//   abi_client           parity cases; prints PASS/FAIL per case, exit 0 if all pass
//   abi_client --bench   us per mla_decode_split_fp16 call, n_h = 128, N = 4096
//
// Exit codes: 0 pass, 1 a case failed, 2 a HIP call failed, 77 no GPU.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "mla_mi355x.h"

extern "C" int oracle_mla_decode_cpu(const float *query, const float *cache, float *out, int num_heads,
                                     int head_dim_c, int seq_length, int dv, double divisor);

namespace {

constexpr int kDK = MLA_HEAD_DIM_K;
constexpr int kDV = MLA_HEAD_DIM_V;

// ---- IEEE binary16 <-> binary32 on the host (round to nearest even).
uint16_t to_half(float f)
{
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int exp = (int)((x >> 23) & 0xff) - 127 + 15;
    uint32_t mant = x & 0x7fffffu;
    if (((x >> 23) & 0xff) == 0xff)  // inf / nan
        return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    if (exp >= 31)
        return (uint16_t)(sign | 0x7c00u);
    if (exp <= 0) {  // subnormal or zero in binary16
        if (exp < -10)
            return (uint16_t)sign;
        mant |= 0x800000u;
        const int shift = 14 - exp;
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u)))
            ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)exp << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
        ++h;  // a carry into the exponent is the correct rounding
    return (uint16_t)(sign | h);
}

float from_half(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ffu;
    float f;
    if (exp == 0) {
        f = std::ldexp((float)mant, -24);
    } else if (exp == 31) {
        f = mant ? NAN : INFINITY;
    } else {
        f = std::ldexp((float)(mant | 0x400u), exp - 25);
    }
    uint32_t x;
    std::memcpy(&x, &f, 4);
    x |= sign;
    std::memcpy(&f, &x, 4);
    return f;
}

// ---- seeded N(0, 1) values: splitmix64 -> uniform -> Box-Muller.
struct Rng {
    uint64_t s;
    uint64_t next()
    {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    float normal()
    {
        const double u = uniform(), v = uniform();
        return (float)(std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v));
    }
};

int g_failures = 0;

#define HIP_OK(call)                                                                   \
    do {                                                                               \
        const hipError_t e_ = (call);                                                  \
        if (e_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "HIP error %d (%s) at %s:%d\n", (int)e_,              \
                         hipGetErrorString(e_), __FILE__, __LINE__);                   \
            std::exit(2);                                                              \
        }                                                                              \
    } while (0)

template <typename T>
struct DevBuf {
    T *p = nullptr;
    size_t n = 0;
    explicit DevBuf(size_t count) : n(count) { HIP_OK(hipMalloc((void **)&p, count * sizeof(T) + 16)); }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    void put(const std::vector<T> &v) { HIP_OK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice)); }
    std::vector<T> get() const
    {
        std::vector<T> v(n);
        HIP_OK(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
        return v;
    }
};

void report(const std::string &name, bool ok, const std::string &detail)
{
    std::printf("%s %s%s%s\n", ok ? "PASS" : "FAIL", name.c_str(), detail.empty() ? "" : ": ", detail.c_str());
    std::fflush(stdout);
    if (!ok)
        ++g_failures;
}

void expect_status(const std::string &name, int got, int want)
{
    report(name, got == want,
           "status " + std::to_string(got) + " (" + mla_status_string(got) + "), expected " + std::to_string(want));
}

std::vector<float> halves_to_float(const std::vector<uint16_t> &h)
{
    std::vector<float> f(h.size());
    for (size_t i = 0; i < h.size(); ++i)
        f[i] = from_half(h[i]);
    return f;
}

std::vector<uint16_t> random_halves(Rng &rng, size_t n)
{
    std::vector<uint16_t> h(n);
    for (auto &x : h)
        x = to_half(rng.normal());
    return h;
}

// the decode contract on the CPU: divisor sqrt(192), 512 value columns
std::vector<float> oracle(const float *q, const float *c, int n_h, int n)
{
    std::vector<float> out((size_t)n_h * kDV, 0.f);
    if (n > 0 && oracle_mla_decode_cpu(q, c, out.data(), n_h, kDK, n, kDV, std::sqrt(192.0)) != 0) {
        std::fprintf(stderr, "oracle failed\n");
        std::exit(2);
    }
    return out;
}

// max |got - ref| and whether |got - ref| <= atol + rtol |ref| everywhere
std::string compare(const float *got, const float *ref, size_t n, double tol, bool *ok, double *worst_out = nullptr)
{
    double worst = 0.0;
    *ok = true;
    for (size_t i = 0; i < n; ++i) {
        const double d = std::fabs((double)got[i] - (double)ref[i]);
        if (!(d <= tol + tol * std::fabs((double)ref[i])))
            *ok = false;
        if (!std::isnan(worst) && (std::isnan(d) || d > worst))
            worst = d;  // a NaN, once seen, is what is reported
    }
    if (worst_out)
        *worst_out = worst;
    char buf[96];
    std::snprintf(buf, sizeof buf, "max |err| %.3e (atol = rtol = %.0e)", worst, tol);
    return buf;
}

void case_single(hipStream_t s, int n_h, int n, int splits, uint64_t seed)
{
    Rng rng{seed};
    const auto qh = random_halves(rng, (size_t)n_h * kDK), ch = random_halves(rng, (size_t)n * kDK);
    DevBuf<uint16_t> q(qh.size()), c(ch.size()), out((size_t)n_h * kDV);
    q.put(qh);
    c.put(ch);
    const size_t ws_bytes = mla_decode_split_workspace_size(n_h, n, splits);
    DevBuf<unsigned char> ws(ws_bytes);
    const int st = mla_decode_split_fp16(q.p, c.p, out.p, ws.p, ws_bytes, n_h, n, splits, s);
    const std::string name = "split_fp16 n_h=" + std::to_string(n_h) + " N=" + std::to_string(n) +
                             " splits=" + std::to_string(splits);
    if (st != MLA_STATUS_SUCCESS) {
        expect_status(name, st, MLA_STATUS_SUCCESS);
        return;
    }
    HIP_OK(hipStreamSynchronize(s));
    const auto got = halves_to_float(out.get());
    const auto ref = oracle(halves_to_float(qh).data(), halves_to_float(ch).data(), n_h, n);
    bool ok;
    const std::string d = compare(got.data(), ref.data(), got.size(), 1e-2, &ok);
    report(name, ok, d);

    // the same decode as two launches with fp32 partials
    DevBuf<uint16_t> out2((size_t)n_h * kDV);
    int st2 = mla_decode_split_fp16_partials(q.p, c.p, ws.p, ws_bytes, n_h, n, splits, MLA_FLAG_FP32_PARTIALS, s);
    if (st2 == MLA_STATUS_SUCCESS)
        st2 = mla_decode_split_fp16_combine(ws.p, ws_bytes, out2.p, n_h, n, splits, MLA_FLAG_FP32_PARTIALS, s);
    if (st2 != MLA_STATUS_SUCCESS) {
        expect_status(name + " (partials + combine, fp32 partials)", st2, MLA_STATUS_SUCCESS);
        return;
    }
    HIP_OK(hipStreamSynchronize(s));
    const auto got2 = halves_to_float(out2.get());
    const std::string d2 = compare(got2.data(), ref.data(), got2.size(), 1e-2, &ok);
    report(name + " (partials + combine, fp32 partials)", ok, d2);
}

void case_batched(hipStream_t s, int n_h, const std::vector<int> &lens, uint64_t seed)
{
    Rng rng{seed};
    const int batch = (int)lens.size();
    std::vector<int> cu(batch + 1, 0);
    for (int b = 0; b < batch; ++b)
        cu[b + 1] = cu[b] + lens[b];
    const int total = cu[batch];
    const auto qh = random_halves(rng, (size_t)batch * n_h * kDK), ch = random_halves(rng, (size_t)total * kDK);
    DevBuf<uint16_t> q(qh.size()), c(std::max<size_t>(ch.size(), 1)), out((size_t)batch * n_h * kDV);
    DevBuf<int> cu_d(cu.size());
    q.put(qh);
    if (!ch.empty())
        c.put(ch);
    cu_d.put(cu);
    const size_t ws_bytes = mla_decode_split_batched_workspace_size(batch, n_h, total, 0);
    DevBuf<unsigned char> ws(ws_bytes);
    std::string name = "split_batched_fp16 n_h=" + std::to_string(n_h) + " lengths=";
    for (int b = 0; b < batch; ++b)
        name += (b ? "," : "") + std::to_string(lens[b]);
    const int st = mla_decode_split_batched_fp16(q.p, c.p, cu_d.p, out.p, ws.p, ws_bytes, batch, n_h, total, 0, s);
    if (st != MLA_STATUS_SUCCESS) {
        expect_status(name, st, MLA_STATUS_SUCCESS);
        return;
    }
    HIP_OK(hipStreamSynchronize(s));
    const auto got = halves_to_float(out.get());
    const auto qf = halves_to_float(qh), cf = halves_to_float(ch);
    bool all_ok = true;
    std::string detail;
    double worst = 0.0;
    for (int b = 0; b < batch; ++b) {
        const float *gb = got.data() + (size_t)b * n_h * kDV;
        bool ok;
        if (lens[b] == 0) {
            ok = true;
            for (int i = 0; i < n_h * kDV; ++i)
                ok = ok && gb[i] == 0.f;
            if (!ok)
                detail = "empty sequence " + std::to_string(b) + " not zero";
        } else {
            const auto ref = oracle(qf.data() + (size_t)b * n_h * kDK, cf.data() + (size_t)cu[b] * kDK, n_h, lens[b]);
            double w = 0.0;
            const std::string d = compare(gb, ref.data(), ref.size(), 1e-2, &ok, &w);
            if (!ok && detail.empty())
                detail = "sequence " + std::to_string(b) + " " + d;
            if (std::isnan(w) || w > worst)
                worst = w;
        }
        all_ok = all_ok && ok;
    }
    if (detail.empty()) {
        char buf[96];
        std::snprintf(buf, sizeof buf, "max |err| %.3e over the sequences (atol = rtol = 1e-02)", worst);
        detail = buf;
    }
    report(name, all_ok, detail);
}

void case_fp32(hipStream_t s, int n_h, int n, uint64_t seed)
{
    Rng rng{seed};
    std::vector<float> qf((size_t)n_h * kDK), cf((size_t)n * kDK);
    for (auto &x : qf)
        x = rng.normal();
    for (auto &x : cf)
        x = rng.normal();
    DevBuf<float> q(qf.size()), c(cf.size()), out((size_t)n_h * kDV);
    q.put(qf);
    c.put(cf);
    const size_t ws_bytes = mla_decode_fused_workspace_size(n_h, n, 0);
    DevBuf<unsigned char> ws(ws_bytes);
    const std::string name = "fused_fp32 n_h=" + std::to_string(n_h) + " N=" + std::to_string(n);
    const int st = mla_decode_fused_fp32(q.p, c.p, out.p, ws.p, ws_bytes, n_h, kDK, n, 0, s);
    if (st != MLA_STATUS_SUCCESS) {
        expect_status(name, st, MLA_STATUS_SUCCESS);
        return;
    }
    HIP_OK(hipStreamSynchronize(s));
    const auto got = out.get();
    const auto ref = oracle(qf.data(), cf.data(), n_h, n);
    bool ok;
    const std::string d = compare(got.data(), ref.data(), got.size(), 1e-4, &ok);
    report(name, ok, d);
}

void case_errors(hipStream_t s)
{
    const int n_h = 16, n = 64;
    DevBuf<uint16_t> q((size_t)n_h * kDK), c((size_t)n * kDK + 8), out((size_t)n_h * kDV);
    const size_t ws_bytes = mla_decode_split_workspace_size(n_h, n, 0);
    DevBuf<unsigned char> ws(ws_bytes);
    expect_status("error: null query", mla_decode_split_fp16(nullptr, c.p, out.p, ws.p, ws_bytes, n_h, n, 0, s),
                  MLA_STATUS_INVALID_VALUE);
    expect_status("error: num_heads 17", mla_decode_split_fp16(q.p, c.p, out.p, ws.p, ws_bytes, 17, n, 0, s),
                  MLA_STATUS_INVALID_VALUE);
    // the size query covers fp32 partials, the larger of the two precisions
    expect_status("error: workspace one byte short (fp32 partials)",
                  mla_decode_split_fp16_ex(q.p, c.p, out.p, ws.p, ws_bytes - 1, n_h, n, 0, MLA_FLAG_FP32_PARTIALS, s),
                  MLA_STATUS_WORKSPACE_TOO_SMALL);
    expect_status("error: empty workspace", mla_decode_split_fp16(q.p, c.p, out.p, ws.p, 0, n_h, n, 0, s),
                  MLA_STATUS_WORKSPACE_TOO_SMALL);
    expect_status("error: misaligned cache",
                  mla_decode_split_fp16(q.p, (const char *)c.p + 2, out.p, ws.p, ws_bytes, n_h, n, 0, s),
                  MLA_STATUS_MISALIGNED);
    expect_status("error: head_dim_c 512 on the fp32 entry",
                  mla_decode_fused_fp32((const float *)q.p, (const float *)c.p, (float *)out.p, ws.p, ws_bytes, n_h,
                                        512, n, 0, s),
                  MLA_STATUS_INVALID_VALUE);
    HIP_OK(hipStreamSynchronize(s));
}

int bench(hipStream_t s)
{
    // ~1 s of warm-up calls first: the GPU's clocks reach their steady state
    const int n_h = 128, n = 4096, warmup = 90000, steps = 200;
    // 224 (Q*, C) device pairs (1.09 GB: nothing a call reads is still in the
    // L2 or the 256 MB MALL when it comes round again) rotated per call,
    // filled from 8 host draws
    const int pool = 224, draws = 8;
    Rng rng{42};
    std::vector<std::vector<uint16_t>> hq, hc;
    for (int i = 0; i < draws; ++i) {
        hq.push_back(random_halves(rng, (size_t)n_h * kDK));
        hc.push_back(random_halves(rng, (size_t)n * kDK));
    }
    std::vector<DevBuf<uint16_t> *> qs, cs;
    for (int i = 0; i < pool; ++i) {
        qs.push_back(new DevBuf<uint16_t>((size_t)n_h * kDK));
        cs.push_back(new DevBuf<uint16_t>((size_t)n * kDK));
        qs.back()->put(hq[i % draws]);
        cs.back()->put(hc[i % draws]);
    }
    DevBuf<uint16_t> out((size_t)n_h * kDV);
    const size_t ws_bytes = mla_decode_split_workspace_size(n_h, n, 0);
    DevBuf<unsigned char> ws(ws_bytes);
    auto call = [&](int i) {
        const int st = mla_decode_split_fp16(qs[i % pool]->p, cs[i % pool]->p, out.p, ws.p, ws_bytes, n_h, n, 0, s);
        if (st != MLA_STATUS_SUCCESS) {
            std::fprintf(stderr, "mla_decode_split_fp16: %s\n", mla_status_string(st));
            std::exit(2);
        }
    };
    for (int i = 0; i < warmup; ++i)
        call(i);
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a));
    HIP_OK(hipEventCreate(&b));
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipEventRecord(a, s));
    for (int i = 0; i < steps; ++i)
        call(i);
    HIP_OK(hipEventRecord(b, s));
    HIP_OK(hipEventSynchronize(b));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, a, b));
    const double us = ms * 1e3 / steps;
    const double bytes = 2.0 * ((double)n_h * kDK + (double)n * kDK + (double)n_h * kDV);
    std::printf("{\"client\": \"abi_client (C++, no Python)\", \"call\": \"mla_decode_split_fp16\", \"num_heads\": %d, "
                "\"seq_len\": %d, \"splits\": %d, \"steps\": %d, \"warmup\": %d, \"us_per_call\": %.3f, "
                "\"call_TBps\": %.4f}\n",
                n_h, n, mla_decode_split_num_splits(n_h, n, 0, 0), steps, warmup, us, bytes / (us * 1e-6) / 1e12);
    HIP_OK(hipEventDestroy(a));
    HIP_OK(hipEventDestroy(b));
    for (auto *p : qs)
        delete p;
    for (auto *p : cs)
        delete p;
    return 0;
}

}  // namespace

int main(int argc, char **argv)
{
    const std::string mode = argc > 1 ? argv[1] : "";
    if (mode == "--abi") {
        std::printf("abi_version %d\n", mla_abi_version());
        for (int st = 0; st <= 5; ++st)
            std::printf("status %d: %s\n", st, mla_status_string(st));
        std::printf("workspace n_h=128 N=4096: %zu bytes\n", mla_decode_split_workspace_size(128, 4096, 0));
        return mla_abi_version() == MLA_ABI_VERSION ? 0 : 1;
    }
    if (mode == "--to-half") {  // float bit patterns (hex) on stdin -> binary16 bits and back (hex)
        unsigned x;
        while (std::scanf("%x", &x) == 1) {
            float f;
            std::memcpy(&f, &x, 4);
            const uint16_t h = to_half(f);
            const float back = from_half(h);
            uint32_t bb;
            std::memcpy(&bb, &back, 4);
            std::printf("%04x %08x\n", (unsigned)h, (unsigned)bb);
        }
        return 0;
    }
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        std::printf("no GPU\n");
        return 77;
    }
    HIP_OK(hipSetDevice(0));
    hipStream_t s;
    HIP_OK(hipStreamCreate(&s));
    int rc = 0;
    if (mode == "--bench") {
        rc = bench(s);
    } else {
        case_single(s, 128, 4096, 0, 1);
        case_single(s, 16, 1, 0, 2);
        case_single(s, 48, 777, 5, 3);
        case_batched(s, 32, {5, 0, 1000, 33, 2048}, 4);
        case_fp32(s, 32, 300, 5);
        case_errors(s);
        std::printf("%d failure(s)\n", g_failures);
        rc = g_failures ? 1 : 0;
    }
    HIP_OK(hipStreamDestroy(s));
    return rc;
}
