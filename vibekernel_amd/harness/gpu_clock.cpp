// gpu_clock.cpp -- part of libvk_bench.so: the GPU's clocks and socket power
// sampled from the driver's metrics table while a timed region runs
// (include/vk_bench.h, vkb_clock_*).
//
// Why: a sustained GEMM holds MI355X at its power limit, and the clock the
// power manager settles on (not the 2.4 GHz of the spec peak) sets how many
// MFMA cycles a launch gets.  The reference learned the same on its A100
// (the SM clock stuck at 1155 MHz; its post-mortem asks that every run log
// the clock).  The clock-true fraction of peak is achieved / (CUs x 4096 FLOP
// x SCLK).
//
// How: the amd-smi library (libamd_smi.so, opened with dlopen so the
// harness still runs where it is absent) reads the driver's gpu_metrics
// table: current_gfxclks[] (one SCLK per XCD), current_uclk (the memory
// clock), current_socket_power and average_gfx_activity.  A host thread polls
// it; the GPU is not touched (no kernel, no HIP call), so the sampler cannot
// perturb the launches it measures beyond one host core.  Measured on
// MI355X: the table is refreshed about once per second (its firmware
// timestamp advances by 0.999 s), so a region needs to last a few seconds to
// hold samples.  Only refreshes seen during the region count: the table read
// at the start predates it and is dropped, and repeated timestamps are
// counted once.
#include <hip/hip_runtime.h>

#include <amd_smi/amdsmi.h>
#include <dlfcn.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "vk_bench.h"

namespace {

using fn_init = amdsmi_status_t (*)(uint64_t);
using fn_sockets = amdsmi_status_t (*)(uint32_t*, amdsmi_socket_handle*);
using fn_procs = amdsmi_status_t (*)(amdsmi_socket_handle, uint32_t*, amdsmi_processor_handle*);
using fn_bdf = amdsmi_status_t (*)(amdsmi_processor_handle, amdsmi_bdf_t*);
using fn_metrics = amdsmi_status_t (*)(amdsmi_processor_handle, amdsmi_gpu_metrics_t*);

struct Sampler {
    std::mutex mu;
    bool opened = false;
    std::string error = "not opened";
    void* lib = nullptr;
    fn_metrics metrics = nullptr;
    amdsmi_processor_handle handle = nullptr;
    int device = -1;

    std::thread th;
    std::atomic<bool> stop{false};
    bool running = false;
    int interval_us = 1000;
    // accumulated over the window
    int samples = 0;
    double gfx_sum = 0, gfx_min = 1e30, gfx_max = 0, uclk_sum = 0, pwr_sum = 0;
    int uclk_n = 0, pwr_n = 0;
    double busy_sum = 0;
    int busy_n = 0;
    uint64_t last_ts = 0;
    bool primed = false;  // the table as the region began has been read
    // Every refresh seen in the region, with the host time of the read that
    // saw it; guarded by dmu (read by vkb_clock_samples while sampling).
    std::mutex dmu;
    std::vector<vkb_clock_sample> log;
    std::chrono::steady_clock::time_point t0;
    double window_ms = 0;

    bool open_for(int dev) {
        if (opened && dev == device) return true;
        opened = false;
        if (!lib) {
            lib = dlopen("libamd_smi.so", RTLD_NOW | RTLD_LOCAL);
            if (!lib) lib = dlopen("/opt/rocm/lib/libamd_smi.so", RTLD_NOW | RTLD_LOCAL);
            if (!lib) {
                error = "libamd_smi.so not found";
                return false;
            }
            auto init = reinterpret_cast<fn_init>(dlsym(lib, "amdsmi_init"));
            if (!init || init(AMDSMI_INIT_AMD_GPUS) != AMDSMI_STATUS_SUCCESS) {
                error = "amdsmi_init failed";
                return false;
            }
        }
        auto sockets = reinterpret_cast<fn_sockets>(dlsym(lib, "amdsmi_get_socket_handles"));
        auto procs = reinterpret_cast<fn_procs>(dlsym(lib, "amdsmi_get_processor_handles"));
        auto bdf = reinterpret_cast<fn_bdf>(dlsym(lib, "amdsmi_get_gpu_device_bdf"));
        metrics = reinterpret_cast<fn_metrics>(dlsym(lib, "amdsmi_get_gpu_metrics_info"));
        if (!sockets || !procs || !bdf || !metrics) {
            error = "amd-smi entry points missing";
            return false;
        }
        // The HIP device's PCI address, matched against amd-smi's processors.
        int dom = 0, bus = 0, devn = 0;
        if (hipDeviceGetAttribute(&dom, hipDeviceAttributePciDomainID, dev) != hipSuccess ||
            hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, dev) != hipSuccess ||
            hipDeviceGetAttribute(&devn, hipDeviceAttributePciDeviceId, dev) != hipSuccess) {
            error = "PCI address of the HIP device unavailable";
            return false;
        }
        uint32_t ns = 0;
        if (sockets(&ns, nullptr) != AMDSMI_STATUS_SUCCESS || ns == 0) {
            error = "no amd-smi sockets";
            return false;
        }
        std::vector<amdsmi_socket_handle> sk(ns);
        if (sockets(&ns, sk.data()) != AMDSMI_STATUS_SUCCESS) {
            error = "amd-smi sockets";
            return false;
        }
        for (uint32_t s = 0; s < ns; s++) {
            uint32_t np = 0;
            if (procs(sk[s], &np, nullptr) != AMDSMI_STATUS_SUCCESS || np == 0) continue;
            std::vector<amdsmi_processor_handle> ph(np);
            if (procs(sk[s], &np, ph.data()) != AMDSMI_STATUS_SUCCESS) continue;
            for (uint32_t p = 0; p < np; p++) {
                amdsmi_bdf_t b{};
                if (bdf(ph[p], &b) != AMDSMI_STATUS_SUCCESS) continue;
                if ((int)b.domain_number == dom && (int)b.bus_number == bus && (int)b.device_number == devn) {
                    handle = ph[p];
                    device = dev;
                    opened = true;
                    error.clear();
                    return true;
                }
            }
        }
        error = "HIP device not found among amd-smi processors";
        return false;
    }

    void sample_once() {
        amdsmi_gpu_metrics_t m;
        std::memset(&m, 0, sizeof(m));
        if (metrics(handle, &m) != AMDSMI_STATUS_SUCCESS) return;
        if (!primed) {  // the table as it stood when the region began
            primed = true;
            last_ts = m.firmware_timestamp;
            return;
        }
        if (m.firmware_timestamp == last_ts) return;
        last_ts = m.firmware_timestamp;
        double s = 0;
        int n = 0;
        for (int x = 0; x < AMDSMI_MAX_NUM_GFX_CLKS; x++) {
            const uint16_t c = m.current_gfxclks[x];
            if (c != 0 && c != 0xffff) {
                s += c;
                n++;
            }
        }
        if (n == 0 && m.current_gfxclk != 0 && m.current_gfxclk != 0xffff) {
            s = m.current_gfxclk;
            n = 1;
        }
        if (n == 0) return;
        const double g = s / n;
        vkb_clock_sample rec{};
        rec.t_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch())
                       .count();
        rec.gfx_mhz = g;
        rec.uclk_mhz = (m.current_uclk != 0 && m.current_uclk != 0xffff) ? m.current_uclk : 0.0;
        rec.socket_w = (m.current_socket_power != 0 && m.current_socket_power != 0xffff) ? m.current_socket_power
                                                                                          : 0.0;
        rec.gfx_activity = m.average_gfx_activity != 0xffff ? m.average_gfx_activity : -1.0;
        for (int x = 0; x < 8 && x < AMDSMI_MAX_NUM_GFX_CLKS; x++) {
            const uint16_t c = m.current_gfxclks[x];
            rec.xcd_mhz[x] = (c != 0 && c != 0xffff) ? c : 0.0;
        }
        {
            std::lock_guard<std::mutex> lk(dmu);
            log.push_back(rec);
        }
        samples++;
        gfx_sum += g;
        gfx_min = std::fmin(gfx_min, g);
        gfx_max = std::fmax(gfx_max, g);
        if (m.current_uclk != 0 && m.current_uclk != 0xffff) {
            uclk_sum += m.current_uclk;
            uclk_n++;
        }
        if (m.current_socket_power != 0 && m.current_socket_power != 0xffff) {
            pwr_sum += m.current_socket_power;
            pwr_n++;
        }
        if (m.average_gfx_activity != 0xffff) {
            busy_sum += m.average_gfx_activity;
            busy_n++;
        }
    }

    void loop() {
        while (!stop.load(std::memory_order_relaxed)) {
            sample_once();
            std::this_thread::sleep_for(std::chrono::microseconds(interval_us));
        }
        sample_once();  // the table as the region ends
    }
};

Sampler& sampler() {
    static Sampler s;
    return s;
}

}  // namespace

extern "C" int vkb_clock_open(void) {
    Sampler& s = sampler();
    std::lock_guard<std::mutex> lk(s.mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        s.error = "hipGetDevice failed";
        return VK_ERR_HIP;
    }
    return s.open_for(dev) ? VK_OK : VK_ERR_HIP;
}

extern "C" const char* vkb_clock_error(void) { return sampler().error.c_str(); }

extern "C" int vkb_clock_start(int interval_us) {
    Sampler& s = sampler();
    std::lock_guard<std::mutex> lk(s.mu);
    if (s.running) return VK_ERR_HIP;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || !s.open_for(dev)) return VK_ERR_HIP;
    s.interval_us = interval_us > 0 ? interval_us : 1000;
    s.samples = 0;
    s.gfx_sum = s.uclk_sum = s.pwr_sum = 0;
    s.gfx_min = 1e30;
    s.gfx_max = 0;
    s.uclk_n = s.pwr_n = 0;
    s.busy_sum = 0;
    s.busy_n = 0;
    s.last_ts = 0;
    s.primed = false;
    {
        std::lock_guard<std::mutex> dl(s.dmu);
        s.log.clear();
    }
    s.stop.store(false);
    s.t0 = std::chrono::steady_clock::now();
    s.th = std::thread([&s] { s.loop(); });
    s.running = true;
    return VK_OK;
}

extern "C" int vkb_clock_stop(vkb_clock_stats* out) {
    Sampler& s = sampler();
    std::lock_guard<std::mutex> lk(s.mu);
    if (!s.running) return VK_ERR_HIP;
    s.stop.store(true);
    s.th.join();
    s.running = false;
    s.window_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - s.t0).count();
    if (out) {
        std::memset(out, 0, sizeof(*out));
        out->samples = s.samples;
        out->window_ms = s.window_ms;
        if (s.samples) {
            out->gfx_mhz_mean = s.gfx_sum / s.samples;
            out->gfx_mhz_min = s.gfx_min;
            out->gfx_mhz_max = s.gfx_max;
        }
        if (s.uclk_n) out->uclk_mhz_mean = s.uclk_sum / s.uclk_n;
        if (s.pwr_n) out->socket_w_mean = s.pwr_sum / s.pwr_n;
        out->gfx_activity_mean = s.busy_n ? s.busy_sum / s.busy_n : -1.0;
    }
    return s.samples ? VK_OK : VK_ERR_HIP;
}

extern "C" double vkb_clock_now_ms(void) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

extern "C" int vkb_clock_samples(vkb_clock_sample* out, int max) {
    Sampler& s = sampler();
    std::lock_guard<std::mutex> lk(s.dmu);
    const int n = (int)s.log.size();
    if (out)
        for (int i = 0; i < n && i < max; i++) out[i] = s.log[i];
    return n;
}
