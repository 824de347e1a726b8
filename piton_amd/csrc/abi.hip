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

struct LaunchNote {
    const void *fn;
    const char *name;
    dim3 grid, block;
    uint32_t dyn_lds;
};
constexpr int kMaxNotes = 8;
static thread_local LaunchNote g_notes[kMaxNotes];
static thread_local int g_note_count = 0;

void note_launch(const void *fn, const char *name, dim3 grid, dim3 block, uint32_t dyn_lds) {
    if (g_note_count < kMaxNotes) g_notes[g_note_count] = LaunchNote{fn, name, grid, block, dyn_lds};
    g_note_count++;
}

void reset_launches() { g_note_count = 0; }

static thread_local int g_cu_count = 0;

int device_cu_count() { return g_cu_count; }

int require_device() {
    // the architecture check is cached per thread and device: later calls cost one
    // hipGetDevice
    static thread_local int checked_dev = -1;
    reset_launches();
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

int32_t piton_mi355x_last_launches(piton_launch_info_t *out, int32_t max, int32_t *count) {
    using namespace piton;
    PITON_REQUIRE(count != nullptr && max >= 0 && (max == 0 || out != nullptr), PITON_EINVAL,
                  "last_launches: null output or negative max");
    const int n = g_note_count < kMaxNotes ? g_note_count : kMaxNotes;
    *count = g_note_count;
    for (int i = 0; i < n && i < max; i++) {
        const LaunchNote &note = g_notes[i];
        piton_launch_info_t &o = out[i];
        memset(&o, 0, sizeof o);
        // the source spelling, without the parentheses a template kernel is launched in
        const char *nm = note.name;
        size_t len = strlen(nm);
        if (len >= 2 && nm[0] == '(' && nm[len - 1] == ')') {
            nm++;
            len -= 2;
        }
        if (len > sizeof o.kernel - 1) len = sizeof o.kernel - 1;
        memcpy(o.kernel, nm, len);
        o.grid[0] = note.grid.x, o.grid[1] = note.grid.y, o.grid[2] = note.grid.z;
        o.block[0] = note.block.x, o.block[1] = note.block.y, o.block[2] = note.block.z;
        // a kernel's attributes do not change: looked up once per kernel and thread
        static thread_local const void *cached_fn[32];
        static thread_local hipFuncAttributes cached_attr[32];
        static thread_local int n_cached = 0;
        int slot = -1;
        for (int c = 0; c < n_cached; c++)
            if (cached_fn[c] == note.fn) slot = c;
        if (slot < 0) {
            hipFuncAttributes attr;
            if (hipFuncGetAttributes(&attr, note.fn) != hipSuccess)
                return set_error(PITON_EHIP, "last_launches: hipFuncGetAttributes failed for %s", o.kernel);
            slot = n_cached < 32 ? n_cached++ : 31;
            cached_fn[slot] = note.fn;
            cached_attr[slot] = attr;
        }
        const hipFuncAttributes &attr = cached_attr[slot];
        o.lds_bytes = (uint32_t)attr.sharedSizeBytes + note.dyn_lds;
        o.vgprs = attr.numRegs;
        o.scratch_bytes = (uint32_t)attr.localSizeBytes;
    }
    clear_error();
    return PITON_OK;
}

}  // extern "C"
