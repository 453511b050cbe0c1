// Bench harness for the flash-GQA C++ operator API (MI355X / gfx950).
//
// Counterpart of the reference's C++ harness
// examples/cplusplus/test_decode_flash_gqa.cu: seeded inputs, single-launch
// GPU timing with events (:295-310), bandwidth and TFLOPS from the tensor
// sizes (:311-319), and the CPU reference attention timed on the host with
// omp_get_wtime (:180-255).  It covers the five BASELINE configurations:
// decode (1, 2), ragged decode (3) and causal prefill (4, 5), through the
// drop-in entry points LaunchFlashGqaBf16Kernel, LaunchFlashGqaBf16KernelVarlen
// and LaunchFlashGqaForwardBf16Kernel.
//
// The CPU reference is the oracle library (oracle/fgqa_oracle.c): it is both
// the parity checker (max-abs 2e-2 and mean-abs 2e-3 on bf16 outputs, LSE
// within 1e-3) and the reported CPU baseline, with the thread count stated.
// Config 5 is checked and timed on a row sample (all heads of batch 0, the
// first and the last 128 query rows), and the sample is named in the output.
//
// GPU time: `queued` is the average of the timed launches issued back to
// back (the roofline fraction uses it); `single` is the median of launches
// timed one at a time, as the reference harness does, which includes the host
// side of each call.
//
// Output: one table row and one JSON line per configuration; exit status 1
// when a launch fails or a configuration misses the tolerance.
//
//   bench_flash_gqa [--configs 1,2,4] [--iters 20] [--warmup 5] [--seed 2024] [--threads 0]
#include <hip/hip_runtime_api.h>
#include <omp.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "FlashGQA/decode_flash_gqa_kernel.h"
#include "FlashGQA/flash_gqa_forward_kernel.h"
#include "Utils/utils.h"
#include "fgqa_oracle.h"

namespace {

constexpr double kHbmPeakGBs = 8000.0;        // MI355X HBM3E
constexpr double kBf16PeakTFlops = 2516.6;    // 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
constexpr double kMaxAbsTol = 2e-2;
constexpr double kMeanAbsTol = 2e-3;
constexpr double kLseTol = 1e-3;
constexpr int kHeadDim = 128;

#define HIP_CHECK(x)                                                                          \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            std::exit(2);                                                                     \
        }                                                                                     \
    } while (0)

struct Config {
    int id;
    bool prefill;
    bool ragged;
    int batch, seq, hq, hkv;
    float sigma;
};

// The BASELINE configurations.
const Config kConfigs[] = {
    {1, false, false, 2, 512, 16, 2, 1.0f},
    {2, false, false, 60, 4096, 128, 8, 1.0f},
    {3, false, true, 64, 32768, 64, 8, 1.0f},
    {4, true, false, 1, 4096, 16, 1, 1.0f},
    {5, true, false, 4, 16384, 32, 8, 0.5f},
};

// Counter-based N(0, sigma^2) bf16 values: SplitMix64 (Steele, Lea and Flood,
// "Fast splittable pseudorandom number generators", 2014) keyed by (seed,
// tensor) and indexed by element, two uniforms per value, Box-Muller.  The
// value of element i does not depend on the thread count.
uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

double uniform01(uint64_t key, uint64_t i) { return (double)(splitmix64(key + i) >> 11) * 0x1.0p-53; }

void fill_normal(std::vector<uint16_t>& dst, uint64_t seed, uint64_t tensor, float sigma) {
    const uint64_t key = splitmix64(seed ^ (tensor << 56));
    const int64_t n = (int64_t)dst.size();
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const double u1 = uniform01(key, 2 * (uint64_t)i);
        const double u2 = uniform01(key, 2 * (uint64_t)i + 1);
        const double z = std::sqrt(-2.0 * std::log1p(-u1)) * std::cos(2.0 * M_PI * u2);
        dst[i] = fgqa_oracle_f32_to_bf16((float)(sigma * z));
    }
}

// Single launches bracketed by events (the reference harness's timing, which
// includes the host side of each call), and the same launches queued back to
// back between one pair of events (the GPU's own rate).
struct Stats {
    double median_us, min_us, mean_us, queued_us;
};

template <typename F>
Stats time_launches(F&& launch, int warmup, int iters) {
    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    // at least `warmup` launches, and at least 150 ms of them: the CPU check
    // of the previous configuration leaves the GPU idle for seconds, and the
    // clock under a compute-bound kernel settles only after about 60 ms
    // (config 4's prefill: 73-85 us per launch in the first 10 ms, 68 us from
    // 60 ms on)
    for (int i = 0; i < warmup; ++i) launch();
    HIP_CHECK(hipDeviceSynchronize());
    {
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < 40000; ++i) {
            launch();
            if ((i & 7) == 7) {
                HIP_CHECK(hipDeviceSynchronize());
                if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(150)) break;
            }
        }
        HIP_CHECK(hipDeviceSynchronize());
    }
    std::vector<double> us;
    for (int i = 0; i < iters; ++i) {
        HIP_CHECK(hipEventRecord(e0, nullptr));
        launch();
        HIP_CHECK(hipEventRecord(e1, nullptr));
        HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0.f;
        HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        us.push_back(ms * 1e3);
    }
    HIP_CHECK(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; ++i) launch();
    HIP_CHECK(hipEventRecord(e1, nullptr));
    HIP_CHECK(hipEventSynchronize(e1));
    float qms = 0.f;
    HIP_CHECK(hipEventElapsedTime(&qms, e0, e1));
    HIP_CHECK(hipEventDestroy(e0));
    HIP_CHECK(hipEventDestroy(e1));
    std::vector<double> s = us;
    std::sort(s.begin(), s.end());
    double sum = 0.0;
    for (double x : us) sum += x;
    return {s[s.size() / 2], s.front(), sum / (double)us.size(), qms * 1e3 / iters};
}

struct ErrStats {
    double max_abs = 0.0, sum_abs = 0.0;
    int64_t n = 0;
    bool finite = true;
    void add(uint16_t out, uint16_t ref) {
        const double d = std::fabs((double)fgqa_oracle_bf16_to_f32(out) - (double)fgqa_oracle_bf16_to_f32(ref));
        if (!std::isfinite(d)) finite = false;
        max_abs = std::max(max_abs, d);
        sum_abs += d;
        ++n;
    }
    double mean_abs() const { return n ? sum_abs / (double)n : 0.0; }
    bool ok() const { return finite && n > 0 && max_abs <= kMaxAbsTol && mean_abs() <= kMeanAbsTol; }
};

template <typename T>
T* to_device(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_CHECK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <typename T>
std::vector<T> to_host(const T* d, size_t n) {
    std::vector<T> h(n);
    HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

struct Options {
    std::vector<int> configs{1, 2, 4};
    int iters = 20, warmup = 5, threads = 0;
    uint64_t seed = 2024;
};

bool run_decode(const Config& c, const Options& opt, int threads) {
    const int B = c.batch, S = c.seq, Hq = c.hq, Hkv = c.hkv, D = kHeadDim;
    const float scale = 1.0f / std::sqrt((float)D);
    const size_t nq = (size_t)B * Hq * D, nkv = (size_t)B * S * Hkv * D;
    std::vector<uint16_t> q(nq), k(nkv), v(nkv);
    fill_normal(q, opt.seed + c.id, 0, c.sigma);
    fill_normal(k, opt.seed + c.id, 1, c.sigma);
    fill_normal(v, opt.seed + c.id, 2, c.sigma);
    std::vector<int32_t> lens(B, S);
    if (c.ragged) {
        const uint64_t key = splitmix64((opt.seed + c.id) ^ (3ull << 56));
        for (int b = 0; b < B; ++b) lens[b] = 1 + (int)(splitmix64(key + b) % (uint64_t)S);
        // padding past each length is NaN: it must never be read
#pragma omp parallel for schedule(dynamic)
        for (int b = 0; b < B; ++b)
            for (int64_t i = GET_1D_INDEX_FROM_4D(b, lens[b], 0, 0, S, Hkv, D);
                 i < GET_1D_INDEX_FROM_4D(b + 1, 0, 0, 0, S, Hkv, D); ++i)
                k[i] = v[i] = 0x7FC0;
    }
    int64_t valid = 0;
    for (int b = 0; b < B; ++b) valid += lens[b];

    uint16_t *dq = to_device(q), *dk = to_device(k), *dv = to_device(v), *dout = nullptr;
    float* dinter = nullptr;
    int32_t* dlens = c.ragged ? to_device(lens) : nullptr;
    HIP_CHECK(hipMalloc(&dout, nq * 2));
    HIP_CHECK(hipMalloc(&dinter, nq * sizeof(float)));
    auto launch = [&] {
        if (c.ragged)
            LaunchFlashGqaBf16KernelVarlen(reinterpret_cast<const bf16_t*>(dq), reinterpret_cast<const bf16_t*>(dk),
                                           reinterpret_cast<const bf16_t*>(dv), scale, reinterpret_cast<bf16_t*>(dout),
                                           dlens, B, S, Hq, Hkv, D);
        else
            LaunchFlashGqaBf16Kernel(reinterpret_cast<const bf16_t*>(dq), reinterpret_cast<const bf16_t*>(dk),
                                     reinterpret_cast<const bf16_t*>(dv), scale, reinterpret_cast<bf16_t*>(dout),
                                     dinter, B, S, Hq, Hkv, D);
    };
    launch();
    const int st = FlashGqaGetLastStatus();
    if (st != 0) {
        std::fprintf(stderr, "config %d: launch status %d\n", c.id, st);
        return false;
    }
    const Stats t = time_launches(launch, opt.warmup, opt.iters);
    std::vector<uint16_t> out = to_host(dout, nq);

    // CPU reference: the C++ reference's loop (bf16 P, 128-token tiles), all rows
    std::vector<uint16_t> ref(nq);
    const double c0 = omp_get_wtime();
    const int rc = fgqa_oracle_decode_bf16(q.data(), k.data(), v.data(), scale, ref.data(), nullptr, B, S, Hq, Hkv, D,
                                           c.ragged ? lens.data() : nullptr, 128, 1, threads);
    const double cpu_s = omp_get_wtime() - c0;
    ErrStats err;
    for (size_t i = 0; i < nq; ++i) err.add(out[i], ref[i]);

    const double kv_bytes = 2.0 * (double)valid * Hkv * D * 2;
    const double all_bytes = kv_bytes + 2.0 * (double)nq * 2;
    const double gbs = kv_bytes / (t.queued_us * 1e-6) / 1e9;
    const bool ok = rc == 0 && err.ok();
    std::printf("%-3d %-8s B=%-3d S=%-6d Hq=%-4d Hkv=%-2d  GPU %9.1f us queued (single %9.1f)  %8.1f GB/s  %5.1f %% of HBM"
                "  | CPU %8.3f s (%d threads)  max-abs %.2e mean-abs %.2e  %s\n",
                c.id, c.ragged ? "ragged" : "decode", B, S, Hq, Hkv, t.queued_us, t.median_us, gbs,
                100.0 * gbs / kHbmPeakGBs, cpu_s, threads, err.max_abs, err.mean_abs(), ok ? "PASS" : "FAIL");
    std::printf("{\"config\": %d, \"kind\": \"%s\", \"batch\": %d, \"seq\": %d, \"num_q_heads\": %d, "
                "\"num_kv_heads\": %d, \"gpu_us_queued\": %.2f, \"gpu_us_median\": %.2f, \"gpu_us_min\": %.2f, "
                "\"gpu_us_mean\": %.2f, \"kv_bytes\": %.0f, \"GBs\": %.2f, \"all_tensor_GBs\": %.2f, "
                "\"roofline\": {\"bound\": \"hbm\", \"peak\": %.1f, \"unit\": \"GB/s\", \"frac\": %.4f}, "
                "\"cpu_s\": %.4f, \"cpu_threads\": %d, "
                "\"cpu_sample\": \"all rows\", \"cpu_GBs\": %.3f, \"max_abs\": %.3e, \"mean_abs\": %.3e, \"pass\": %s}\n",
                c.id, c.ragged ? "ragged decode" : "decode", B, S, Hq, Hkv, t.queued_us, t.median_us, t.min_us,
                t.mean_us, kv_bytes, gbs, all_bytes / (t.queued_us * 1e-6) / 1e9, kHbmPeakGBs, gbs / kHbmPeakGBs,
                cpu_s, threads,
                kv_bytes / cpu_s / 1e9, err.max_abs, err.mean_abs(), ok ? "true" : "false");
    std::fflush(stdout);
    HIP_CHECK(hipFree(dq));
    HIP_CHECK(hipFree(dk));
    HIP_CHECK(hipFree(dv));
    HIP_CHECK(hipFree(dout));
    HIP_CHECK(hipFree(dinter));
    if (dlens) HIP_CHECK(hipFree(dlens));
    return ok;
}

bool run_prefill(const Config& c, const Options& opt, int threads) {
    const int B = c.batch, S = c.seq, Hq = c.hq, Hkv = c.hkv, D = kHeadDim;
    const float scale = 1.0f / std::sqrt((float)D);
    const size_t nq = (size_t)B * S * Hq * D, nkv = (size_t)B * S * Hkv * D, nl = (size_t)B * Hq * S;
    std::vector<uint16_t> q(nq), k(nkv), v(nkv);
    fill_normal(q, opt.seed + c.id, 0, c.sigma);
    fill_normal(k, opt.seed + c.id, 1, c.sigma);
    fill_normal(v, opt.seed + c.id, 2, c.sigma);

    uint16_t *dq = to_device(q), *dk = to_device(k), *dv = to_device(v), *dout = nullptr;
    float* dlse = nullptr;
    HIP_CHECK(hipMalloc(&dout, nq * 2));
    HIP_CHECK(hipMalloc(&dlse, nl * sizeof(float)));
    auto launch = [&] {
        LaunchFlashGqaForwardBf16Kernel(reinterpret_cast<const bf16_t*>(dq), reinterpret_cast<const bf16_t*>(dk),
                                        reinterpret_cast<const bf16_t*>(dv), scale, reinterpret_cast<bf16_t*>(dout),
                                        dlse, B, S, S, Hq, Hkv, D, true);
    };
    launch();
    const int st = FlashGqaGetLastStatus();
    if (st != 0) {
        std::fprintf(stderr, "config %d: launch status %d\n", c.id, st);
        return false;
    }
    const Stats t = time_launches(launch, opt.warmup, opt.iters);
    std::vector<uint16_t> out = to_host(dout, nq);
    std::vector<float> lse = to_host(dlse, nl);

    // CPU reference on row blocks [r0, r0 + n) of batch 0..nb-1 (all heads):
    // the whole problem for config 4, a sample for config 5.
    struct Block {
        int b, r0, n;
    };
    std::vector<Block> blocks;
    std::string sample;
    if (c.id == 5) {
        blocks = {{0, 0, 128}, {0, S - 128, 128}};
        sample = "batch 0, all heads, query rows [0,128) and [S-128,S)";
    } else {
        for (int b = 0; b < B; ++b) blocks.push_back({b, 0, S});
        sample = "all rows";
    }
    const int64_t qs[3] = {(int64_t)S * Hq * D, (int64_t)Hq * D, D};
    const int64_t ks[3] = {(int64_t)S * Hkv * D, (int64_t)Hkv * D, D};
    ErrStats err;
    double lse_max = 0.0, cpu_s = 0.0, sample_flops = 0.0;
    bool rc_ok = true, lse_ok = true;
    for (const Block& bl : blocks) {
        std::vector<uint16_t> ref((size_t)bl.n * Hq * D);
        std::vector<float> lref((size_t)Hq * bl.n);
        const int64_t os[3] = {(int64_t)bl.n * Hq * D, (int64_t)Hq * D, D};
        const uint16_t* qb = q.data() + (size_t)bl.b * qs[0] + (size_t)bl.r0 * qs[1];
        const uint16_t* kb = k.data() + (size_t)bl.b * ks[0];
        const uint16_t* vb = v.data() + (size_t)bl.b * ks[0];
        const double c0 = omp_get_wtime();
        rc_ok = rc_ok && fgqa_oracle_prefill_bf16(qb, kb, vb, scale, ref.data(), lref.data(), 1, bl.n, S, Hq, Hkv, D,
                                                  qs, ks, ks, os, 1, bl.r0, threads) == 0;
        cpu_s += omp_get_wtime() - c0;
        // keys each row sees: r + 1 (causal, top-left)
        for (int r = bl.r0; r < bl.r0 + bl.n; ++r) sample_flops += (double)Hq * 2.0 * (r + 1) * (D + D);
        for (int r = 0; r < bl.n; ++r)
            for (int h = 0; h < Hq; ++h)
                for (int d = 0; d < D; ++d)
                    err.add(out[GET_1D_INDEX_FROM_4D(bl.b, bl.r0 + r, h, d, S, Hq, D)],
                            ref[GET_1D_INDEX_FROM_3D(r, h, d, Hq, D)]);
        for (int h = 0; h < Hq; ++h)
            for (int r = 0; r < bl.n; ++r) {
                const double g = lse[((size_t)bl.b * Hq + h) * S + bl.r0 + r];
                const double d = std::fabs(g - (double)lref[(size_t)h * bl.n + r]);
                if (!std::isfinite(d)) lse_ok = false;
                lse_max = std::max(lse_max, d);
            }
    }
    lse_ok = lse_ok && lse_max <= kLseTol;

    // the reference's causal-halved count (test_flash_gqa_kernel.py:282-301)
    const double flops = (double)B * Hq * 2.0 * S * S * (D + D) / 2.0;
    const double tflops = flops / (t.queued_us * 1e-6) / 1e12;
    const bool ok = rc_ok && err.ok() && lse_ok;
    std::printf("%-3d %-8s B=%-3d S=%-6d Hq=%-4d Hkv=%-2d  GPU %9.1f us queued (single %9.1f)  %8.1f TFLOP/s %5.1f %% of bf16"
                "  | CPU %8.3f s (%d threads, %s)  max-abs %.2e mean-abs %.2e lse %.1e  %s\n",
                c.id, "prefill", B, S, Hq, Hkv, t.queued_us, t.median_us, tflops, 100.0 * tflops / kBf16PeakTFlops, cpu_s,
                threads, sample.c_str(), err.max_abs, err.mean_abs(), lse_max, ok ? "PASS" : "FAIL");
    std::printf("{\"config\": %d, \"kind\": \"causal prefill\", \"batch\": %d, \"seq\": %d, \"num_q_heads\": %d, "
                "\"num_kv_heads\": %d, \"gpu_us_queued\": %.2f, \"gpu_us_median\": %.2f, \"gpu_us_min\": %.2f, "
                "\"gpu_us_mean\": %.2f, \"flops\": %.0f, \"TFLOPs\": %.2f, \"roofline\": {\"bound\": \"mfma\", \"peak\": %.1f, "
                "\"unit\": \"TFLOP/s\", \"frac\": %.4f}, \"cpu_s\": %.4f, \"cpu_threads\": %d, \"cpu_sample\": \"%s\", "
                "\"cpu_GFLOPs\": %.3f, \"max_abs\": %.3e, \"mean_abs\": %.3e, \"lse_max_abs\": %.3e, \"pass\": %s}\n",
                c.id, B, S, Hq, Hkv, t.queued_us, t.median_us, t.min_us, t.mean_us, flops, tflops, kBf16PeakTFlops,
                tflops / kBf16PeakTFlops, cpu_s, threads, sample.c_str(), sample_flops / cpu_s / 1e9, err.max_abs,
                err.mean_abs(), lse_max, ok ? "true" : "false");
    std::fflush(stdout);
    HIP_CHECK(hipFree(dq));
    HIP_CHECK(hipFree(dk));
    HIP_CHECK(hipFree(dv));
    HIP_CHECK(hipFree(dout));
    HIP_CHECK(hipFree(dlse));
    return ok;
}

Options parse(int argc, char** argv) {
    Options o;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&]() -> const char* {
            if (i + 1 >= argc) {
                std::fprintf(stderr, "%s needs a value\n", a.c_str());
                std::exit(2);
            }
            return argv[++i];
        };
        if (a == "--configs") {
            o.configs.clear();
            std::string s = next();
            size_t p = 0;
            while (p < s.size()) {
                const size_t e = s.find(',', p);
                o.configs.push_back(std::atoi(s.substr(p, e == std::string::npos ? std::string::npos : e - p).c_str()));
                if (e == std::string::npos) break;
                p = e + 1;
            }
        } else if (a == "--iters") {
            o.iters = std::max(1, std::atoi(next()));
        } else if (a == "--warmup") {
            o.warmup = std::max(0, std::atoi(next()));
        } else if (a == "--seed") {
            o.seed = std::strtoull(next(), nullptr, 10);
        } else if (a == "--threads") {
            o.threads = std::atoi(next());
        } else {
            std::fprintf(stderr, "usage: %s [--configs 1,2,4] [--iters N] [--warmup N] [--seed N] [--threads N]\n",
                         argv[0]);
            std::exit(2);
        }
    }
    return o;
}

}  // namespace

int main(int argc, char** argv) {
    const Options opt = parse(argc, argv);
    if (opt.threads > 0) omp_set_num_threads(opt.threads);
    const int threads = opt.threads > 0 ? opt.threads : omp_get_max_threads();
    int dev_count = 0;
    HIP_CHECK(hipGetDeviceCount(&dev_count));
    hipDeviceProp_t prop;
    HIP_CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("# device 0: %s, %d CUs; host: %u hardware threads, CPU reference on %d OpenMP threads; seed %llu\n",
                prop.gcnArchName, prop.multiProcessorCount, std::thread::hardware_concurrency(), threads,
                (unsigned long long)opt.seed);
    std::fflush(stdout);
    bool all_ok = true;
    for (int id : opt.configs) {
        const Config* c = nullptr;
        for (const Config& x : kConfigs)
            if (x.id == id) c = &x;
        if (c == nullptr) {
            std::fprintf(stderr, "unknown config %d\n", id);
            return 2;
        }
        std::printf("# config %d ...\n", id);
        std::fflush(stdout);
        all_ok = (c->prefill ? run_prefill(*c, opt, threads) : run_decode(*c, opt, threads)) && all_ok;
    }
    return all_ok ? 0 : 1;
}
