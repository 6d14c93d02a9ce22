// Runs the task1 harness's own error statistic, TestData::calculateAvgErr
// (include/playground/test_data.hpp; the reference's is
// results/naive_cycle4/include/playground/test_data.hpp:145-162), on GT and C
// arrays read from a file, so that a CPU test can compare what the harness
// prints with the oracle's restatement bit for bit.
//
// Built twice by the test: -DTEST_FLOAT16 (fp16 GT/C) and without (fp32).
// Usage: stat_check <file> [--legacy]
//   file: uint64 count, then count GT values, then count C values, each in
//   the binary's DataType (little-endian, as written by numpy's tofile).
// Prints "ok <hex bits of the float statistic>"; the statistic's own aborts
// (non-finite C, an infinite or NaN sum, GT == 0 in legacy mode, no valid
// term) exit with EXIT_FAILURE after "[Playground] Check failed ...".
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "playground/test_data.hpp"

int main(int argc, char** argv) {
    using namespace playground;
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s <file> [--legacy]\n", argv[0]);
        return 2;
    }
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    uint64_t count = 0;
    if (std::fread(&count, sizeof(count), 1, f) != 1 || count == 0 || count > (1u << 26)) return 2;
    std::vector<params::DataType> gt(count), c(count);
    if (std::fread(gt.data(), sizeof(params::DataType), count, f) != count) return 2;
    if (std::fread(c.data(), sizeof(params::DataType), count, f) != count) return 2;
    std::fclose(f);

    TestConfig cfg;
    cfg.legacy_err = argc > 2 && std::strcmp(argv[2], "--legacy") == 0;
    // A count x 1 x 1 problem: the constructor's ground truth (version 0) is
    // then replaced by the file's arrays through the harness accessors.
    TestData td(uint32_t(count), 1, 1, cfg);
    std::memcpy(td.get_mutable_GT_ptr(), gt.data(), count * sizeof(params::DataType));
    std::memcpy(td.get_mutable_C_ptr(), c.data(), count * sizeof(params::DataType));
    const float32_t err = td.calculateAvgErr();
    uint32_t bits = 0;
    std::memcpy(&bits, &err, sizeof(bits));
    std::printf("ok %08x\n", bits);
    return 0;
}
