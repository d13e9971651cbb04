// Library runtime: refusal messages, launch probes, the device capability probe and the host
// form of the attention visibility intervals.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

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
