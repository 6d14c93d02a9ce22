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

/* GPU clocks and socket power over a region, sampled on a host thread from
 * the driver's metrics table (amd-smi; no GPU work is issued).  The table is
 * refreshed about once per second, so only a region of a few seconds holds
 * samples; the refreshes seen during the region count, the table as it stood
 * when the region began does not.  SCLK is the mean over XCDs of
 * current_gfxclks, averaged over those samples.  Not in the reference, whose
 * post-mortem asks that every run log the clock (README.md:160 of the
 * reference). */
typedef struct vkb_clock_stats {
  int samples;          /* distinct metric-table samples in the region */
  double window_ms;     /* host time between start and stop */
  double gfx_mhz_mean;  /* SCLK */
  double gfx_mhz_min;
  double gfx_mhz_max;
  double uclk_mhz_mean; /* memory clock (0: not reported) */
  double socket_w_mean; /* socket power in W (0: not reported) */
  double gfx_activity_mean; /* GFX busy percentage (-1: not reported) */
} vkb_clock_stats;

/* One refresh of the metrics table seen by the sampler. */
typedef struct vkb_clock_sample {
  double t_ms;          /* host steady-clock time (CLOCK_MONOTONIC, ms) of the read that saw the refresh */
  double gfx_mhz;       /* SCLK, mean over XCDs */
  double uclk_mhz;      /* memory clock (0: not reported) */
  double socket_w;      /* socket power in W (0: not reported) */
  double gfx_activity;  /* GFX busy percentage (-1: not reported) */
  double xcd_mhz[8];    /* SCLK of each XCD (current_gfxclks[0..7]; 0: not reported) */
} vkb_clock_sample;

/* Open the sampler for the current HIP device (VK_OK, or VK_ERR_HIP with the
 * reason in vkb_clock_error()). */
int vkb_clock_open(void);
/* Start sampling every interval_us microseconds. */
int vkb_clock_start(int interval_us);
/* Stop and fill *out; VK_ERR_HIP when no sample was taken. */
int vkb_clock_stop(vkb_clock_stats* out);
const char* vkb_clock_error(void);
/* The refreshes seen so far in the current (or last) region, oldest first:
 * copies up to `max` into out (may be NULL) and returns how many there are.
 * Safe to call while sampling. */
int vkb_clock_samples(vkb_clock_sample* out, int max);
/* The sampler's time base now (CLOCK_MONOTONIC, ms), to place a region's
 * start among the samples. */
double vkb_clock_now_ms(void);

#ifdef __cplusplus
}
#endif
#endif
