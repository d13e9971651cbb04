// Library runtime: refusal messages, launch probes, the device capability probe and the host
// form of the attention visibility intervals.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "dm_common.h"

namespace dm {

static thread_local std::string g_error;
static std::atomic<uint64_t> g_probes[DM_PROBE_COUNT];

void set_error(const std::string &msg) { g_error = msg; }

int refuse(const std::string &msg) {
    g_error = msg;
    return DM_ERR_REFUSED;
}

int hip_status(hipError_t e, const char *what) {
    g_error = std::string(what) + ": " + hipGetErrorString(e);
    return DM_ERR_HIP;
}

void probe_add(int probe, uint64_t n) {
    if (probe >= 0 && probe < DM_PROBE_COUNT) g_probes[probe].fetch_add(n);
}

// Kernel timers: event pairs still to be read, per kernel, and the totals read so far. Events are
// pooled; at most kMaxPending pairs are kept per kernel (older ones are read first).
static std::mutex g_timing_mu;
static std::atomic<bool> g_timing{false};
struct TimerSlot {
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
    double ms = 0.0;
    uint64_t launches = 0;
};
static TimerSlot g_timers[DM_KERNEL_COUNT];
static std::vector<hipEvent_t> g_event_pool;
constexpr size_t kMaxPending = 4096;

static hipEvent_t take_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

static void drain(TimerSlot &t) {
    for (auto &pr : t.pending) {
        float ms = 0.f;
        if (hipEventSynchronize(pr.second) == hipSuccess &&
            hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) {
            t.ms += ms;
            t.launches += 1;
        }
        g_event_pool.push_back(pr.first);
        g_event_pool.push_back(pr.second);
    }
    t.pending.clear();
}

KernelTimer::KernelTimer(int kernel, hipStream_t stream) : kernel_(kernel), stream_(stream) {
    if (!g_timing.load(std::memory_order_relaxed) || kernel < 0 || kernel >= DM_KERNEL_COUNT)
        return;
    std::lock_guard<std::mutex> lock(g_timing_mu);
    start_ = take_event();
    if (start_ && hipEventRecord(start_, stream_) != hipSuccess) {
        g_event_pool.push_back(start_);
        start_ = nullptr;
    }
}

KernelTimer::~KernelTimer() {
    if (!start_) return;
    std::lock_guard<std::mutex> lock(g_timing_mu);
    hipEvent_t end = take_event();
    if (!end || hipEventRecord(end, stream_) != hipSuccess) {
        g_event_pool.push_back(start_);
        if (end) g_event_pool.push_back(end);
        return;
    }
    TimerSlot &t = g_timers[kernel_];
    if (t.pending.size() >= kMaxPending) drain(t);
    t.pending.emplace_back(start_, end);
}

// The kernels are built for gfx950 (wave64, MFMA with the 16-deep bf16 forms, 160 KiB of LDS);
// the requirement gate of crates/dash-ops/src/cube.rs:27-151.
bool device_ok(std::string *why) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        *why = "no HIP device";
        return false;
    }
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
        *why = "cannot read the device's properties";
        return false;
    }
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        *why = std::string("the kernels are built for gfx950, the device is ") + p.gcnArchName;
        return false;
    }
    return true;
}

}  // namespace dm

extern "C" {

const char *dm_last_error(void) { return dm::g_error.c_str(); }

uint64_t dm_probe_count(int probe) {
    if (probe < 0 || probe >= DM_PROBE_COUNT) return 0;
    return dm::g_probes[probe].load();
}

void dm_probe_reset(void) {
    for (auto &p : dm::g_probes) p.store(0);
}

int dm_kernel_timing(int enable) {
    std::lock_guard<std::mutex> lock(dm::g_timing_mu);
    for (auto &t : dm::g_timers) {
        dm::drain(t);
        t.ms = 0.0;
        t.launches = 0;
    }
    dm::g_timing.store(enable != 0);
    return DM_OK;
}

int dm_kernel_time(int kernel, double *ms, uint64_t *launches) {
    if (kernel < 0 || kernel >= DM_KERNEL_COUNT) return dm::refuse("kernel_time: no such kernel");
    std::lock_guard<std::mutex> lock(dm::g_timing_mu);
    dm::drain(dm::g_timers[kernel]);
    if (ms) *ms = dm::g_timers[kernel].ms;
    if (launches) *launches = dm::g_timers[kernel].launches;
    return DM_OK;
}

int dm_describe(char *buf, size_t len) {
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) {
        std::snprintf(buf, len, "no HIP device");
        return dm::refuse("dm_describe: no HIP device");
    }
    std::snprintf(buf, len, "%s, %d CUs, wave%d, %zu KiB LDS per workgroup, %.1f GiB HBM, %d MHz",
                  p.gcnArchName, p.multiProcessorCount, p.warpSize, p.sharedMemPerBlock / 1024,
                  p.totalGlobalMem / 1073741824.0, p.clockRate / 1000);
    std::string why;
    return dm::device_ok(&why) ? DM_OK : dm::refuse("dm_describe: " + why);
}

int dm_device_alloc(size_t bytes, void **ptr) {
    if (!ptr) return dm::refuse("device_alloc: null result pointer");
    *ptr = nullptr;
    if (bytes == 0) return DM_OK;
    const hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        *ptr = nullptr;
        return dm::hip_status(e, ("device_alloc: " + std::to_string(bytes) + " bytes").c_str());
    }
    return DM_OK;
}

int dm_device_free(void *ptr) {
    if (!ptr) return DM_OK;
    const hipError_t e = hipFree(ptr);
    return e == hipSuccess ? DM_OK : dm::hip_status(e, "device_free");
}

// (the copies wait for their own completion: a host source or destination may be pageable)
static int dm_copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, void *stream,
                   const char *what) {
    if (bytes == 0) return DM_OK;
    if (!dst || !src) return dm::refuse(std::string(what) + ": null pointer");
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? DM_OK : dm::hip_status(e, what);
}

int dm_copy_to_device(void *dst, const void *src, size_t bytes, void *stream) {
    return dm_copy(dst, src, bytes, hipMemcpyHostToDevice, stream, "copy_to_device");
}

int dm_copy_to_host(void *dst, const void *src, size_t bytes, void *stream) {
    return dm_copy(dst, src, bytes, hipMemcpyDeviceToHost, stream, "copy_to_host");
}

int dm_stream_synchronize(void *stream) {
    const hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    return e == hipSuccess ? DM_OK : dm::hip_status(e, "stream_synchronize");
}

int dm_attention_row_bounds(const dm_attention_desc *desc, int64_t b, int64_t i, int64_t *lo,
                            int64_t *hi) {
    (void)b;
    if (!desc || !lo || !hi) return dm::refuse("attention: null argument");
    if (i < 0 || i >= desc->tq) return dm::refuse("attention: query index out of range");
    dm::MaskInfo m = dm::mask_info(desc);
    dm::row_bounds(m, i, lo, hi);
    return DM_OK;
}

}  // extern "C"
