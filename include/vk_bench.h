/*
 * vk_bench.h -- timing loops of the playground harness as a C ABI
 * (libvk_bench.so), so the Python benchmark measures exactly what the task1
 * binary measures without interpreter overhead between the event records and
 * the launch.
 *
 * Reference: results/ralph_loop_fable/src/main.cpp:52-62 -- warm-up launches,
 * then for each timed launch: event record, matmul, event record, event
 * synchronize, elapsed time.
 */
#ifndef VK_BENCH_H
#define VK_BENCH_H

#include <stddef.h>

#include "vk_gemm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The reference loop on `stream`: `warmup` untimed calls, then `iters` calls
 * each between its own event pair with a host sync; per_iter_ms[i] receives
 * each elapsed time.  Returns VK_OK or the first error. */
int vkb_reference_loop(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n,
                       size_t k, const void* A, const void* B, void* C, void* stream, int warmup,
                       int iters, float* per_iter_ms);

/* `iters` calls back to back between one event pair; *total_ms receives the
 * elapsed time. */
int vkb_back_to_back(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n,
                     size_t k, const void* A, const void* B, void* C, void* stream, int iters,
                     float* total_ms);

/* The benchmark's timed region on `stream`: `warmup` untimed calls, a device
 * synchronisation, then `iters` calls back to back between one event pair (no
 * host sync in between), then a device synchronisation; *total_ms receives
 * the elapsed time between the events.  An event recorded between every pair
 * of calls would not do: on ROCm each such record lengthens the launch that
 * follows it.  Not in the reference, whose loop syncs the host after every
 * call (vkb_reference_loop). */
int vkb_stream_loop(int version, vk_dtype in_dtype, vk_dtype out_dtype, size_t m, size_t n,
                    size_t k, const void* A, const void* B, void* C, void* stream, int warmup,
                    int iters, float* total_ms);

#ifdef __cplusplus
}
#endif
#endif
