// main.cpp -- task1 harness: one binary per (dtype, version).
// Reference: results/ralph_loop_fable/src/main.cpp:10-127.
//
// Same command line (-m -n -k -w/--n_warmup -t/--n_test -h/--help, defaults
// 4096/4096/4096/10/100), the same loop (GPU: warm-up launches, then each
// timed launch bracketed by its own event pair on the null stream and a host
// sync; CPU v0: the loop forced to 10 rounds timed with a steady clock), the
// same TFLOPS formula and the same three stdout lines, so logs stay parseable
// by the reference's tooling.  Additions: --dist/--seed (reproducible
// inputs), --err-legacy (abort on GT == 0 as the original statistic does),
// --json (one machine-readable line with per-iteration statistics, the SCLK,
// memory clock and socket power sampled over the timed loop, the CU count,
// the host cores and the fraction of peak), --dump (A, B, GT and C of the
// run to a file, so the printed statistic can be recomputed elsewhere).
#include <hip/hip_runtime.h>
#include <sched.h>

#include <algorithm>
#include <charconv>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

#include "playground/matmul.hpp"
#include "playground/system.hpp"
#include "playground/test_data.hpp"
#include "vk_bench.h"

// If CPU matmul is used; otherwise GPU matmul.
constexpr bool USING_CPU_MATMUL = playground::params::MatmulVersion == playground::PG_MATMUL_FP32_CBLAS ||
                                  playground::params::MatmulVersion == playground::PG_MATMUL_FP16_CBLAS;

namespace playground {
PLAYGROUND_MATMUL_DEC(params::DataType, params::MatmulVersion, M, N, K, A, B, C);
}

#ifndef TARGET_BIN_OUTPUT_NAME
#define TARGET_BIN_OUTPUT_NAME "task1"
#endif

namespace {

// Shortest round-trip decimal form (what std::format("{}") prints).
template <typename T>
std::string shortest(T v) {
    char buf[64];
    auto r = std::to_chars(buf, buf + sizeof(buf), v);
    return std::string(buf, r.ptr);
}

struct Options {
    uint32_t m = 4096, n = 4096, k = 4096, w = 10, t = 100;
    playground::TestConfig cfg;
    bool json = false;
    std::string dump;
};

void usage() {
    std::printf(
        "Playground Task1: General Matrix Multiplication\n"
        "Usage:\n  %s [OPTION...]\n\n"
        "  -m arg            Num of rows of A and C (default: 4096)\n"
        "  -n arg            Num of columns of B and C (default: 4096)\n"
        "  -k arg            Num of columns of A and rows of B (default: 4096)\n"
        "  -w, --n_warmup arg  Num of warmup rounds (default: 10)\n"
        "  -t, --n_test arg    Num of test rounds (default: 100)\n"
        "      --dist arg      normal | uniform | normal0.5 | int (default: normal)\n"
        "      --seed arg      input seed (default: 20261201)\n"
        "      --err-legacy    GT == 0 aborts the error statistic (original rule)\n"
        "      --json          also print one JSON line\n"
        "      --dump arg      write m, n, k, A, B, GT and C of the run to this file\n"
        "  -h, --help        Print usage\n",
        TARGET_BIN_OUTPUT_NAME);
}

bool parse_u32(const char* s, uint32_t& out) {
    char* end = nullptr;
    unsigned long v = std::strtoul(s, &end, 10);
    if (!s[0] || *end || v > 0xffffffffUL) return false;
    out = uint32_t(v);
    return true;
}

int parse(int argc, const char* argv[], Options& o) {
    for (int i = 1; i < argc; i++) {
        std::string a = argv[i];
        std::string val;
        auto eq = a.find('=');
        if (a.rfind("--", 0) == 0 && eq != std::string::npos) {
            val = a.substr(eq + 1);
            a = a.substr(0, eq);
        }
        auto next = [&](const char* name) -> const char* {
            if (!val.empty()) return val.c_str();
            if (i + 1 >= argc) {
                std::fprintf(stderr, "Option '%s' is missing an argument\n", name);
                std::exit(EXIT_FAILURE);
            }
            return argv[++i];
        };
        uint32_t* target = nullptr;
        if (a == "-m" || a == "--m") target = &o.m;
        else if (a == "-n" || a == "--n") target = &o.n;
        else if (a == "-k" || a == "--k") target = &o.k;
        else if (a == "-w" || a == "--n_warmup") target = &o.w;
        else if (a == "-t" || a == "--n_test") target = &o.t;
        if (target) {
            const char* s = next(a.c_str());
            if (!parse_u32(s, *target)) {
                std::fprintf(stderr, "Argument '%s' failed to parse\n", s);
                std::exit(EXIT_FAILURE);
            }
        } else if (a == "--dist") {
            o.cfg.dist = playground::parse_dist(next("--dist"));
        } else if (a == "--seed") {
            o.cfg.seed = std::strtoull(next("--seed"), nullptr, 10);
        } else if (a == "--err-legacy") {
            o.cfg.legacy_err = true;
        } else if (a == "--json") {
            o.json = true;
        } else if (a == "--dump") {
            o.dump = next("--dump");
        } else if (a == "-h" || a == "--help") {
            usage();
            return 1;
        } else {
            std::fprintf(stderr, "Option '%s' does not exist\n", a.c_str());
            std::exit(EXIT_FAILURE);
        }
    }
    return 0;
}

// Host threads this process may run on (the affinity mask), and the machine's.
int host_cores() {
    cpu_set_t set;
    CPU_ZERO(&set);
    if (sched_getaffinity(0, sizeof(set), &set) == 0) return CPU_COUNT(&set);
    return int(std::thread::hardware_concurrency());
}

// --dump: uint32 m, n, k, element size, then A, B, GT and C row-major in the
// binary's data type.
void dump_run(const std::string& path, uint32_t m, uint32_t n, uint32_t k, playground::TestData& td) {
    using playground::params::DataType;
    FILE* f = std::fopen(path.c_str(), "wb");
    PLAYGROUND_CHECK(f != nullptr);
    const uint32_t hdr[4] = {m, n, k, uint32_t(sizeof(DataType))};
    bool ok = std::fwrite(hdr, sizeof(hdr), 1, f) == 1;
    auto put = [&](const DataType* p, size_t count) {
        if (count) ok = ok && std::fwrite(p, sizeof(DataType), count, f) == count;
    };
    put(td.get_mutable_A_ptr(), size_t(m) * k);
    put(td.get_mutable_B_ptr(), size_t(k) * n);
    put(td.get_mutable_GT_ptr(), size_t(m) * n);
    put(td.get_mutable_C_ptr(), size_t(m) * n);
    ok = std::fclose(f) == 0 && ok;
    PLAYGROUND_CHECK(ok);
}

}  // namespace

void test(uint32_t m, uint32_t n, uint32_t k, uint32_t nWarmupRound, uint32_t nTestRound, const Options& o) {
    using namespace playground;

    auto testData = TestData(m, n, k, o.cfg);
    float32_t totalMilliSecs = 0.0F;
    std::vector<float32_t> perIter;
    vkb_clock_stats clk{};
    bool clockOn = false;

    std::printf("[Playground] Start Testing for GEMM Version %u with DType %s ...\n",
                unsigned(params::MatmulVersion), params::DataTypeName.data());
    std::fflush(stdout);

    params::DataType* Aptr = nullptr;
    params::DataType* Bptr = nullptr;
    params::DataType* Cptr = nullptr;

    auto matmulFn = [&Aptr, &Bptr, &Cptr, m, n, k]() {
        PLAYGOUND_MATMUL_CALL(params::MatmulVersion, m, n, k, Aptr, Bptr, Cptr);
    };

    if constexpr (!USING_CPU_MATMUL) {
        hipEvent_t start, stop;
        PLAYGROUND_HIP_CHECK(hipEventCreate(&start));
        PLAYGROUND_HIP_CHECK(hipEventCreate(&stop));
        float32_t runtime = 0.0F;
        testData.initDeviceData();
        Aptr = testData.get_mutable_d_A_ptr();
        Bptr = testData.get_mutable_d_B_ptr();
        Cptr = testData.get_mutable_d_C_ptr();
        for (size_t i = 0; i < nWarmupRound; ++i) matmulFn();
        if (o.json) clockOn = vkb_clock_start(500) == VK_OK;
        for (auto i = 0ULL; i < nTestRound; ++i) {
            PLAYGROUND_HIP_CHECK(hipEventRecord(start, nullptr));
            matmulFn();
            PLAYGROUND_HIP_CHECK(hipEventRecord(stop, nullptr));
            PLAYGROUND_HIP_CHECK(hipEventSynchronize(stop));
            PLAYGROUND_HIP_CHECK(hipEventElapsedTime(&runtime, start, stop));
            totalMilliSecs += runtime;
            perIter.push_back(runtime);
        }
        if (clockOn) clockOn = vkb_clock_stop(&clk) == VK_OK || clk.window_ms > 0;
        testData.copyResultD2H();
        PLAYGROUND_HIP_CHECK(hipEventDestroy(start));
        PLAYGROUND_HIP_CHECK(hipEventDestroy(stop));
    } else {
        Aptr = testData.get_mutable_A_ptr();
        Bptr = testData.get_mutable_B_ptr();
        Cptr = testData.get_mutable_C_ptr();
        nTestRound = 10;  // 10 rounds for CPU matmul to avoid long runtime.
        for (auto i = 0ULL; i < nTestRound; ++i) {
            auto t0 = std::chrono::steady_clock::now();
            matmulFn();
            auto t1 = std::chrono::steady_clock::now();
            const float32_t ms = std::chrono::duration<float32_t, std::milli>(t1 - t0).count();
            totalMilliSecs += ms;
            perIter.push_back(ms);
        }
    }
    if constexpr (!USING_CPU_MATMUL) PLAYGROUND_HIP_CHECK(hipDeviceSynchronize());
    std::printf("[Playground] Calculating Finished\n");

    if (!o.dump.empty()) dump_run(o.dump, m, n, k, testData);
    float32_t avgErr = testData.calculateAvgErr();

    float32_t msecPerMatrixMul = totalMilliSecs / float32_t(nTestRound);
    float64_t flopsPerMatrixMul = 2.0 * m * n * k;
    float64_t tflops = (flopsPerMatrixMul * 1.0e-12F) / (msecPerMatrixMul / 1000.0F);

    std::printf("[Playground] Result >>> TFLOPS: %s; Average Error: %s\n", shortest(tflops).c_str(),
                shortest(avgErr).c_str());
    if (o.json && !perIter.empty()) {
        float mn = *std::min_element(perIter.begin(), perIter.end());
        float mx = *std::max_element(perIter.begin(), perIter.end());
        // Peak per CU and clock: dense fp16 MFMA 4096 FLOP, fp32 256 FLOP
        // (vector FMA and fp32 MFMA alike); spec peaks at 2.4 GHz and 256 CUs.
        const bool f16 = std::is_same_v<params::DataType, float16_t>;
        const double flopPerClkCu = f16 ? 4096.0 : 256.0;
        const double specPeak = f16 ? 2516.6 : 157.3;
        int cus = 0;
        if constexpr (!USING_CPU_MATMUL) {
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
                cus = 0;
        }
        std::string clock = "null";
        if (clockOn && clk.samples > 0) {
            char b[512];
            const double clockPeak = cus * flopPerClkCu * clk.gfx_mhz_mean * 1e6 / 1e12;
            std::snprintf(b, sizeof(b),
                          "{\"sclk_mhz\": %.1f, \"sclk_mhz_min\": %.1f, \"sclk_mhz_max\": %.1f, \"mclk_mhz\": %.1f, "
                          "\"socket_w\": %.1f, \"samples\": %d, \"source\": \"amd-smi gpu_metrics refreshed during the timed loop\", "
                          "\"peak_at_sclk_tflops\": %.1f, \"frac_clock\": %.4f}",
                          clk.gfx_mhz_mean, clk.gfx_mhz_min, clk.gfx_mhz_max, clk.uclk_mhz_mean, clk.socket_w_mean,
                          clk.samples, clockPeak, clockPeak > 0 ? tflops / clockPeak : 0.0);
            clock = b;
        } else if (!USING_CPU_MATMUL && o.json) {
            const char* why = clockOn ? "no metrics refresh during the timed loop (the table refreshes about once per second)"
                                      : vkb_clock_error();
            clock = std::string("{\"error\": \"") + why + "\"}";
        }
        std::printf("{\"binary\": \"%s\", \"version\": %u, \"dtype\": \"%s\", \"m\": %u, \"n\": %u, \"k\": %u, "
                    "\"warmup\": %u, \"iters\": %u, \"mean_ms\": %.6f, \"min_ms\": %.6f, \"max_ms\": %.6f, "
                    "\"tflops\": %s, \"avg_err\": %s, \"seed\": %llu, \"pct_peak\": %.2f, \"cus\": %d, "
                    "\"host_cores\": %d, \"clock\": %s}\n",
                    TARGET_BIN_OUTPUT_NAME, unsigned(params::MatmulVersion), params::DataTypeName.data(), m, n, k,
                    nWarmupRound, nTestRound, double(msecPerMatrixMul), double(mn), double(mx),
                    shortest(tflops).c_str(), shortest(avgErr).c_str(), (unsigned long long)o.cfg.seed,
                    USING_CPU_MATMUL ? 0.0 : 100.0 * tflops / specPeak, cus, host_cores(), clock.c_str());
    }
    std::fflush(stdout);
}

auto main(int argc, const char* argv[]) -> int {
    Options o;
    try {
        if (parse(argc, argv, o)) return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "%s\n", e.what());
        return EXIT_FAILURE;
    }
    test(o.m, o.n, o.k, o.w, o.t, o);
    return 0;
}
