// ABI plumbing of libpiton_mi355x.so: version, thread-local error messages, the device
// check every entry makes before its first HIP call, and device properties for rooflines.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace piton {

static thread_local char g_msg[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_msg[0] = '\0'; }

static thread_local int g_cu_count = 0;

int device_cu_count() { return g_cu_count; }

int require_device() {
    // the architecture check is cached per thread and device: later calls cost one
    // hipGetDevice
    static thread_local int checked_dev = -1;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && dev == checked_dev) return PITON_OK;
    int count = 0;
    hipError_t ec = hipGetDeviceCount(&count);
    if (ec != hipSuccess || count <= 0)
        return set_error(PITON_ENODEV, "no HIP device (%s)", ec == hipSuccess ? "count 0" : hipGetErrorString(ec));
    if (e != hipSuccess) return set_error(PITON_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return set_error(PITON_EHIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return set_error(PITON_ENODEV, "device %d is %s; this library is built for gfx950", dev, p.gcnArchName);
    checked_dev = dev;
    g_cu_count = p.multiProcessorCount;
    return PITON_OK;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(PITON_EHIP, "%s launch: %s", what, hipGetErrorString(e));
    return PITON_OK;
}

}  // namespace piton

extern "C" {

int32_t piton_mi355x_abi_version(void) { return PITON_MI355X_ABI_VERSION; }

const char *piton_mi355x_last_error(void) { return piton::g_msg; }

int32_t piton_mi355x_device_info(piton_device_info_t *out) {
    using namespace piton;
    PITON_REQUIRE(out != nullptr, PITON_EINVAL, "device_info: null output");
    memset(out, 0, sizeof *out);
    int rc = require_device();
    if (rc) return rc;
    int dev = 0;
    hipGetDevice(&dev);
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return set_error(PITON_EHIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    out->cu_count = p.multiProcessorCount;
    out->max_clock_khz = p.clockRate;
    out->mem_clock_khz = p.memoryClockRate;
    out->mem_bus_width = p.memoryBusWidth;
    out->hbm_bytes = (int64_t)p.totalGlobalMem;
    out->lds_per_cu = (int32_t)p.maxSharedMemoryPerMultiProcessor;
    out->l2_bytes = p.l2CacheSize;
    out->wavefront_size = p.warpSize;
    out->xcd_count = kXcdCount;
    strncpy(out->arch, p.gcnArchName, sizeof out->arch - 1);
    clear_error();
    return PITON_OK;
}

}  // extern "C"
