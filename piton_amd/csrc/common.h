// Shared helpers of libpiton_mi355x.so: status codes and the thread-local error message,
// argument checks, wavefront reductions built from DPP lane moves, and the XCD-aware
// workgroup order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "piton_mi355x.h"

namespace piton {

// native 4 x float vector (the nontemporal builtins take native vector pointers)
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------
// status and messages (host)
// ------------------------------------------------------------------------------------------
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// PITON_OK when a gfx950 device is current, else PITON_ENODEV / PITON_EHIP with a message.
int require_device();
// Compute units of the device the last successful require_device() on this thread checked.
int device_cu_count();
// Turns the last launch's status into PITON_OK or PITON_EHIP naming `what`.
int check_launch(const char *what);

// Launch notes for piton_mi355x_last_launches: every kernel launch goes through PITON_LAUNCH,
// which records the kernel, its grid, block and dynamic LDS in this thread's list (cleared by
// require_device(), which every entry calls before its first launch).
void note_launch(const void *fn, const char *name, dim3 grid, dim3 block, uint32_t dyn_lds);
void reset_launches();
// the same with the kernel's recorded name given (a template's parameter values)
#define PITON_LAUNCH_NAMED(kernel, name, grid, block, lds, stream, ...)                                       \
    do {                                                                                                      \
        ::piton::note_launch(reinterpret_cast<const void *>(&kernel), (name), dim3(grid), dim3(block),        \
                             (uint32_t)(lds));                                                                \
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                                   \
    } while (0)
#define PITON_LAUNCH(kernel, grid, block, lds, stream, ...)                                                   \
    do {                                                                                                      \
        ::piton::note_launch(reinterpret_cast<const void *>(&kernel), #kernel, dim3(grid), dim3(block),       \
                             (uint32_t)(lds));                                                                \
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                                   \
    } while (0)

// ------------------------------------------------------------------------------------------
// Phase trace (diagnostics builds only, -DPITON_PHASE_TRACE; piton_amd/phase_trace.py): a traced
// wave keeps up to four s_memrealtime stamps (a 100 MHz clock shared by the whole chip) in
// registers and, at its end, lane 0 stores them into the wave's own record of the launch's
// record area (no atomics, so waves do not wait on each other). The host hands each launch its
// own area (phase_slot(), a kernel argument that is null in the product build, where every
// macro below is empty); PITON_PHASE_TU(name) exports piton_phase_attach_<name>(log, launches)
// for the source file's launches, which cycle through `launches` areas of kPhaseWaves records.
// ------------------------------------------------------------------------------------------
struct PhaseRecord {
    unsigned long long t[4];
    uint32_t kernel, block;
};
constexpr uint32_t kPhaseWaves = 1u << 16;  // records per launch: waves past it are not traced
#ifdef PITON_PHASE_TRACE
static PhaseRecord *g_phase_base = nullptr;
static unsigned int g_phase_launches = 0, g_phase_seq = 0;
static inline PhaseRecord *phase_slot() {
    return g_phase_base ? g_phase_base + (size_t)(g_phase_seq++ % g_phase_launches) * kPhaseWaves : nullptr;
}
#define PITON_PHASE_VARS unsigned long long _phase_t[4] = {0ull, 0ull, 0ull, 0ull}
#define PITON_PHASE(i)                                        \
    do {                                                      \
        __builtin_amdgcn_sched_barrier(0);                    \
        _phase_t[i] = __builtin_amdgcn_s_memrealtime();       \
        __builtin_amdgcn_sched_barrier(0);                    \
    } while (0)
// the wave's loads in flight have landed (the stamp after it marks the first data)
#define PITON_PHASE_WAIT_LOADS() __builtin_amdgcn_s_waitcnt(0x0F70)
#define PITON_PHASE_END(kid, area)                                                                   \
    do {                                                                                             \
        const uint32_t _w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);                     \
        if ((area) && (threadIdx.x & 63) == 0 && _w < ::piton::kPhaseWaves) {                        \
            ::piton::PhaseRecord *_r = (area) + _w;                                                  \
            for (int _k = 0; _k < 4; _k++) _r->t[_k] = _phase_t[_k];                                 \
            _r->kernel = (kid);                                                                      \
            _r->block = _w;                                                                          \
        }                                                                                            \
    } while (0)
#define PITON_PHASE_TU(name)                                                                             \
    extern "C" __attribute__((visibility("default"))) int piton_phase_attach_##name(void *log,           \
                                                                                     unsigned int launches) { \
        ::piton::g_phase_base = launches ? (::piton::PhaseRecord *)log : nullptr;                        \
        ::piton::g_phase_launches = launches;                                                            \
        ::piton::g_phase_seq = 0;                                                                        \
        return 0;                                                                                        \
    }
#else
static inline PhaseRecord *phase_slot() { return nullptr; }
#define PITON_PHASE_VARS
#define PITON_PHASE(i)
#define PITON_PHASE_WAIT_LOADS()
#define PITON_PHASE_END(kid, area)
#define PITON_PHASE_TU(name)
#endif
// kernel ids of the trace records
constexpr uint32_t kPhaseSoftmaxRows = 1, kPhaseSoftmaxWg = 2, kPhaseAttnFast = 3, kPhaseAttnDecodeShort = 4,
                   kPhaseDecodeLayer = 5, kPhaseMlp = 6, kPhaseGemmSplit = 7;

// numpy's argmax rule on (value, index) pairs: a NaN beats any number, the larger value beats
// the smaller, equal values and two NaNs go to the lower index. The combine is associative and
// commutative, so a reduction in any order gives the first index of the maximum.
__device__ __forceinline__ void argmax_combine(float &v, int &i, float v2, int i2) {
    const bool n1 = v != v, n2 = v2 != v2;
    const bool take = (n1 && n2) ? i2 < i : n2 ? true : n1 ? false : (v2 > v || (v2 == v && i2 < i));
    if (take) {
        v = v2;
        i = i2;
    }
}

// Holds a kernel argument in a scalar register from this point on. Without it the compiler may
// load an argument from the kernarg segment where it is first used, and a load late in a short
// kernel is one more memory round trip on its critical path.
template <class T>
__device__ __forceinline__ T sgpr_keep(T v) {
    asm volatile("" : "+s"(v));
    return v;
}

// a < b ? x : 0 for wave-uniform values, as a scalar compare and select. Written out so that
// the compiler cannot turn it into a branch: one inside a loop whose accumulators live in AGPRs
// makes it copy them to VGPRs and back each iteration.
__device__ __forceinline__ int scalar_lt_select(int a, int b, int x) {
    int r;
    asm("s_cmp_lt_i32 %1, %2\n\ts_cselect_b32 %0, %3, 0" : "=s"(r) : "s"(a), "s"(b), "s"(x) : "scc");
    return r;
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
// a * b and a + b for the host's size checks on caller-supplied extents and strides: INT64_MAX
// where the result overflows, so that a check against any bound fails instead of wrapping
inline int64_t sat_mul(int64_t a, int64_t b) {
    int64_t r;
    return __builtin_mul_overflow(a, b, &r) ? INT64_MAX : r;
}
inline int64_t sat_add(int64_t a, int64_t b) {
    int64_t r;
    return __builtin_add_overflow(a, b, &r) ? INT64_MAX : r;
}

#define PITON_REQUIRE(cond, code, ...)                  \
    do {                                                \
        if (!(cond)) return ::piton::set_error((code), __VA_ARGS__); \
    } while (0)

// ------------------------------------------------------------------------------------------
// device helpers
// ------------------------------------------------------------------------------------------

// DPP lane move of a float within rows of 16 lanes (dpp_ctrl: quad_perm, row mirrors).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// DPP control words (GFX9 encoding).
constexpr int DPP_QUAD_XOR1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

struct MaxOp {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct SumOp {
    __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};

// Reduction over one 64-lane wavefront, result in every lane: four DPP steps combine each row
// of 16 lanes, then the four row results are read out of lanes 0, 16, 32, 48.
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = op(v, dpp_f<DPP_QUAD_XOR1>(v));
    v = op(v, dpp_f<DPP_QUAD_XOR2>(v));
    v = op(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    v = op(v, dpp_f<DPP_ROW_MIRROR>(v));
    float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return op(op(a, b), op(c, d));
}

// s_waitcnt immediates (GFX9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
// waitcnt_vm(n): wait until at most n vector-memory operations are in flight, nothing else.
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
// wait until every LDS / scalar-memory operation has completed, nothing else
constexpr int kWaitcntLgkm0 = 0xC07F;

// Orders LDS traffic between the lanes of one wavefront: stores before the fence are visible
// to loads after it in every lane of the wave. The hardware already runs a wave's LDS
// operations in order; the fences stop the compiler from moving a load above a store that
// another lane made (per thread the addresses differ, so it would otherwise be free to).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup order for an XCD-partitioned chip: the dispatcher hands workgroup b to XCD
// b % n_xcd, so renumber to give each XCD a contiguous run of logical ids (neighbouring tiles
// then share that XCD's L2). A bijection on [0, n) for any n.
__device__ __forceinline__ int xcd_logical_id(int b, int n, int n_xcd) {
    int q = n / n_xcd, r = n % n_xcd;
    int x = b % n_xcd, i = b / n_xcd;
    return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

constexpr int kXcdCount = 8;  // MI355X: 8 XCDs of 32 CUs

}  // namespace piton
