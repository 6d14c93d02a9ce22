// copy_calib.cpp -- a plain device-to-device copy of a known size, used to
// calibrate the FETCH_SIZE / WRITE_SIZE counters (the copy reads and writes
// exactly `MiB` MiB).  Usage: copy_calib [MiB] [repeats]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "playground/utils.hpp"

int main(int argc, char** argv) {
    const size_t mib = argc > 1 ? std::strtoul(argv[1], nullptr, 10) : 256;
    const int reps = argc > 2 ? std::atoi(argv[2]) : 3;
    const size_t bytes = mib << 20;
    void *a = nullptr, *b = nullptr;
    PLAYGROUND_HIP_CHECK(hipMalloc(&a, bytes));
    PLAYGROUND_HIP_CHECK(hipMalloc(&b, bytes));
    PLAYGROUND_HIP_CHECK(hipMemset(a, 1, bytes));
    for (int i = 0; i < reps; i++) PLAYGROUND_HIP_CHECK(hipMemcpy(b, a, bytes, hipMemcpyDeviceToDevice));
    PLAYGROUND_HIP_CHECK(hipDeviceSynchronize());
    std::printf("copied %zu MiB x %d\n", mib, reps);
    PLAYGROUND_HIP_CHECK(hipFree(a));
    PLAYGROUND_HIP_CHECK(hipFree(b));
    return 0;
}
