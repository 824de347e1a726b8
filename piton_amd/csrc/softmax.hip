// Row softmax: softmax_kernel (examples/kernels.py:60-76), HBM-bound.
//
// Design (gfx950):
//   * the row is loaded once into registers (CH float4 chunks per thread), reduced twice
//     (max, then sum), and written once: 8 bytes of HBM traffic per element, the minimum;
//   * rows of up to 1024 columns: one 64-lane wavefront per row, four per 256-thread
//     workgroup, reductions by DPP lane moves only (no LDS, no barriers);
//   * rows of up to 16K columns: one 256-thread workgroup per row, reductions by DPP within
//     each wave and then through LDS across the four. Many short-lived workgroups keep reads
//     and writes interleaved across the chip; at 4096 x 4096 this streams ~8 % faster than
//     a single generation of row-per-wave waves, which read together and then write together;
//   * loads and stores are nontemporal: the row is touched once. (Cached loads look faster
//     only while the inputs fit the 256 MB last-level cache; from HBM they are ~3 % slower);
//   * rows need not be 16-byte aligned (n = 1823): each row is read through the aligned
//     float4 window that covers it, and elements outside [0, n) of the row are masked to
//     -inf. An aligned 16-byte block lies inside one page, so the window never touches an
//     unmapped address. Stores use float4 where the output row has the same alignment as the
//     input row and the chunk is whole, scalar stores at the row's two ends;
//   * exp is v_exp_f32 on (x - max) * log2(e): about 1e-7 relative on the entries that carry
//     the row's weight; the row sum's reciprocal is correctly rounded;
//   * special values: a +inf or +NaN entry, or an all -inf row, makes the whole row NaN, as
//     in numpy and in the QPU emulator; a -inf entry in a finite row gives exactly 0; a -NaN
//     entry gives exactly 0 and the rest of the row is a normal softmax, as in the emulator,
//     whose fmax orders -NaN lowest and whose float ALUs read it as -inf
//     (piton/qpu/emulator.py:139-147, 173-177, 201-205, 224-225); numpy makes that row NaN;
//   * longer rows take a workgroup-per-row kernel that reads the row three times (max, sum,
//     write).
#include "common.h"

// kernel per row class (float4 chunks per lane: short <= 4, mid 5..8, long 9..16):
// 0 = one wave per row, one row each; 1 = one wave per row, persistent, as many workgroups
// per CU as fit at once; 2 = one workgroup per row (mid and long only)
#ifndef PITON_SM_SHORT
#define PITON_SM_SHORT 0
#endif
#ifndef PITON_SM_MID
#define PITON_SM_MID 1
#endif
#ifndef PITON_SM_LONG
#define PITON_SM_LONG 2
#endif
// chunks per thread of the workgroup kernel: mid class 2 (256 threads) or 1 (512); long
// class 4 (256 threads) or 2 (512)
#ifndef PITON_SM_MID_CH
#define PITON_SM_MID_CH 2
#endif
#ifndef PITON_SM_LONG_CH
#define PITON_SM_LONG_CH 2
#endif

namespace piton {

// e^d as 2^(d * log2 e) with v_exp_f32. The product's rounding (half an ulp of t) costs a
// relative error of |t| * 2^-24 * ln 2 in e^d: about 1e-7 on the entries that carry a row's
// weight (|t| < 4), growing only on entries below e^-16 of the row maximum. d = -inf gives
// exactly 0 and NaN passes.
__device__ __forceinline__ float exp_row(float d) {
    const float kL2E = 1.44269502162933349609375f;  // float(log2 e)
    return __builtin_amdgcn_exp2f(d * kL2E);
}

// The emulator's view of an operand of the subtraction x - max: a NaN with the sign bit set
// (bits above 0xFF800000 as an unsigned integer) is -inf, every other value is itself (a +NaN
// stays NaN, so its row still comes out NaN): one v_min_u32. The row maximum needs no mapping:
// IEEE max returns the other operand of a NaN, as max over the mapped values would (a row of
// -NaN and -inf only has maximum -inf either way).
__device__ __forceinline__ float qpu_neg_nan(float x) {
    return __uint_as_float(min(__float_as_uint(x), 0xFF800000u));
}

// Loads row r's aligned float4 window into b: T threads share the row, thread t holding
// chunks t, t + T, ... (CH of them); elements of the window outside the row are masked when
// the row is processed.
template <int CH, int T, bool ALIGNED>
__device__ __forceinline__ void load_row(const float *in, int64_t in_rs, int64_t r, int n, int lane,
                                         f32x4 (&b)[CH], int &off) {
    const float *rp = in + r * in_rs;
    off = ALIGNED ? 0 : (int)((reinterpret_cast<uintptr_t>(rp) >> 2) & 3);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(rp - off);
    const int nch = (off + n + 3) >> 2;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ci = lane + T * c;
        f32x4 f = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (ci < nch) f = __builtin_nontemporal_load(src + ci);
        b[c] = f;
    }
}

// Reduction over the T threads that share a row: one wavefront by DPP lane moves; T/64 of
// them by DPP, then the wave results through LDS (each use has its own T/64 LDS slots, so one
// barrier per reduction suffices; the waves combine in a fixed pairwise order).
template <int T, class Op>
__device__ __forceinline__ float row_reduce(float v, Op op, float *red) {
    v = wave_reduce(v, op);
    if (T == 64) return v;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    if (T == 256) return op(op(red[0], red[1]), op(red[2], red[3]));
    return op(op(op(red[0], red[1]), op(red[2], red[3])), op(op(red[4], red[5]), op(red[6], red[7])));
}

// Masks row `row` (held in b, window offset off) to [0, n), normalises it and stores it.
// lane: this thread's index among the T threads of the row; red: 2 * T / 64 floats of LDS.
template <int CH, int T, bool ALIGNED>
__device__ __forceinline__ void softmax_store_row(float *out, int64_t out_rs, int64_t row, int n, int lane,
                                                  f32x4 (&b)[CH], int off, float *red) {
    const int nch = (off + n + 3) >> 2;
    // first window chunk of this wave's share of slot c is wbase + T * c (the same in every
    // lane): only the slots holding the row's first or last chunk need per-element masks;
    // chunks past the window were loaded as -inf
    const int wbase = __builtin_amdgcn_readfirstlane(lane & ~63);
    auto edge_slot = [&](int c) {
        const int first = wbase + T * c;
        return first == 0 || (first <= nch - 1 && nch - 1 <= first + 63);
    };
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        if (!ALIGNED && edge_slot(c)) {
            const int e0 = 4 * (lane + T * c) - off;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (!(e0 + j >= 0 && e0 + j < n)) b[c][j] = -INFINITY;
        }
        mx = fmaxf(mx, fmaxf(fmaxf(b[c].x, b[c].y), fmaxf(b[c].z, b[c].w)));
    }
    const float m = row_reduce<T>(mx, MaxOp(), red);

    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // masked entries hold -inf, and so do -NaN entries (qpu_neg_nan): exactly 0 here
            // unless the row itself is NaN
            const float e = exp_row(qpu_neg_nan(b[c][j]) - m);
            b[c][j] = e;
            s += e;
        }
    }
    s = row_reduce<T>(s, SumOp(), red + T / 64);
    const float inv = 1.0f / s;

    float *op = out + row * out_rs;
    const int ooff = ALIGNED ? 0 : (int)((reinterpret_cast<uintptr_t>(op) >> 2) & 3);
    if (ooff == off) {
        // same alignment as the input row: whole chunks as float4, the two end chunks by element
        f32x4 *dst = reinterpret_cast<f32x4 *>(op - off);
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int ci = lane + T * c;
            if (wbase + T * c >= nch) continue;  // the whole slot lies past the window
            if (ALIGNED || !edge_slot(c)) {
                if (ci < nch) __builtin_nontemporal_store(b[c] * inv, dst + ci);
            } else if (ci < nch) {
                const int e0 = 4 * ci - off;
                if (e0 >= 0 && e0 + 3 < n) {
                    __builtin_nontemporal_store(b[c] * inv, dst + ci);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (e0 + j >= 0 && e0 + j < n) op[e0 + j] = b[c][j] * inv;
                }
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int e0 = 4 * (lane + T * c) - off;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (e0 + j >= 0 && e0 + j < n) op[e0 + j] = b[c][j] * inv;
        }
    }
}

// Persistent wavefronts: wave w of W = 4 * gridDim.x handles rows w, w + W, w + 2W, ... and
// issues the loads of its next row before it reduces and stores the current one, so every
// wave keeps reads in flight while it writes and the chip never splits into a read phase
// and a write phase. Two register buffers alternate (the loop is unrolled by two).
// ALIGNED: every row of in and out starts 16-byte aligned and n % 4 == 0, so windows are the
// rows themselves and only whole chunks need a bound. Rows here are <= 2048 columns.
template <int CH, bool ALIGNED>
__global__ __launch_bounds__(256) void softmax_rows_kernel(float *out, const float *in, int64_t in_rs, int64_t out_rs,
                                                           int n, int64_t rows, PhaseRecord *phase) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t W = (int64_t)gridDim.x * 4;
    int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= rows) return;  // whole wavefront leaves together

    f32x4 a[CH], b[CH];
    int off_a, off_b = 0;
    PITON_PHASE_VARS;
    PITON_PHASE(0);
    load_row<CH, 64, ALIGNED>(in, in_rs, row, n, lane, a, off_a);
    PITON_PHASE_WAIT_LOADS();
    PITON_PHASE(1);
    while (true) {
        if (row + W < rows) load_row<CH, 64, ALIGNED>(in, in_rs, row + W, n, lane, b, off_b);
        softmax_store_row<CH, 64, ALIGNED>(out, out_rs, row, n, lane, a, off_a, nullptr);
        row += W;
        if (row >= rows) break;
        if (row + W < rows) load_row<CH, 64, ALIGNED>(in, in_rs, row + W, n, lane, a, off_a);
        softmax_store_row<CH, 64, ALIGNED>(out, out_rs, row, n, lane, b, off_b, nullptr);
        row += W;
        if (row >= rows) break;
    }
    PITON_PHASE(2);
    PITON_PHASE_END(kPhaseSoftmaxRows, phase);
}

// One T-thread workgroup per row (T = 256 or 512, CH chunks per thread): many short-lived
// workgroups keep the chip's reads and writes interleaved, which streams faster than a single
// generation of row-per-wave waves.
template <int CH, int T, bool ALIGNED>
__global__ __launch_bounds__(T) void softmax_wg_kernel(float *out, const float *in, int64_t in_rs, int64_t out_rs,
                                                       int n, PhaseRecord *phase) {
    __shared__ float red[2 * T / 64];
    f32x4 b[CH];
    int off;
    PITON_PHASE_VARS;
    PITON_PHASE(0);
    load_row<CH, T, ALIGNED>(in, in_rs, blockIdx.x, n, threadIdx.x, b, off);
    PITON_PHASE_WAIT_LOADS();
    PITON_PHASE(1);
    softmax_store_row<CH, T, ALIGNED>(out, out_rs, blockIdx.x, n, threadIdx.x, b, off, red);
    PITON_PHASE(2);
    PITON_PHASE_END(kPhaseSoftmaxWg, phase);
}

// Rows too long for registers: one workgroup per row, three passes over the row.
__device__ __forceinline__ float block_reduce(float v, float *red, bool is_max) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    v = is_max ? wave_reduce(v, MaxOp()) : wave_reduce(v, SumOp());
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < 4; w++) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(256) void softmax_long_kernel(float *out, const float *in, int64_t in_rs, int64_t out_rs,
                                                           int64_t n) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float *rp = in + row * in_rs;
    float *op = out + row * out_rs;
    float mx = -INFINITY;
    for (int64_t i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, rp[i]);
    const float m = block_reduce(mx, red, true);
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += 256) s += exp_row(qpu_neg_nan(rp[i]) - m);
    s = block_reduce(s, red, false);
    const float inv = 1.0f / s;
    for (int64_t i = threadIdx.x; i < n; i += 256) op[i] = exp_row(qpu_neg_nan(rp[i]) - m) * inv;
}

// Launches the wave-per-row kernel: one row per wave (mode 0), or persistent waves, as many
// workgroups as the device holds at once (mode 1; the occupancy query is made once per
// kernel and device).
template <int CH, bool ALIGNED>
void launch_rows(int mode, int64_t wgs, hipStream_t st, float *out, const float *in, int64_t in_rs, int64_t out_rs,
                 int n, int64_t rows) {
    int64_t grid = wgs;
    if (mode == 1) {
        static thread_local int per_cu = 0, dev_seen = -1;
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (dev != dev_seen) {
            int blocks = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, softmax_rows_kernel<CH, ALIGNED>, 256, 0) !=
                    hipSuccess || blocks < 1)
                blocks = 1;
            per_cu = blocks;
            dev_seen = dev;
        }
        const int64_t cap = (int64_t)device_cu_count() * per_cu;
        grid = wgs < cap ? wgs : cap;
    }
    PITON_LAUNCH((softmax_rows_kernel<CH, ALIGNED>), dim3((unsigned)grid), dim3(256), 0, st, out, in, in_rs,
                       out_rs, n, rows, phase_slot());
}

}  // namespace piton

PITON_PHASE_TU(softmax)

extern "C" int32_t piton_mi355x_softmax(float *out, const float *in, int64_t in_row_stride, int64_t out_row_stride,
                                        int64_t n_cols, int64_t n_rows, int64_t block_size, void *stream) {
    using namespace piton;
    PITON_REQUIRE(n_rows >= 0 && n_cols >= 0, PITON_EINVAL, "softmax: negative size rows=%lld n_cols=%lld",
                  (long long)n_rows, (long long)n_cols);
    PITON_REQUIRE(block_size >= 1, PITON_EINVAL, "softmax: BLOCK_SIZE must be >= 1, got %lld", (long long)block_size);
    const int64_t n = n_cols < block_size ? n_cols : block_size;
    PITON_REQUIRE(n_rows == 0 || n == 0 || (out && in), PITON_EINVAL, "softmax: null pointer");
    PITON_REQUIRE(aligned4(out) && aligned4(in), PITON_EINVAL, "softmax: pointers must be 4-byte aligned");
    PITON_REQUIRE(n_rows <= 1 || (in_row_stride >= n && out_row_stride >= n), PITON_EINVAL,
                  "softmax: row strides (%lld, %lld) shorter than the %lld columns", (long long)in_row_stride,
                  (long long)out_row_stride, (long long)n);
    int rc = require_device();
    if (rc) return rc;
    if (n_rows == 0 || n == 0) return PITON_OK;
    hipStream_t st = (hipStream_t)stream;
    // worst-case float4 chunks of a row's aligned window
    const bool all_aligned = aligned16(in) && (in_row_stride % 4 == 0 || n_rows == 1);
    const int64_t nch = (n + 3 + (all_aligned ? 0 : 3)) / 4;
    const int64_t per_lane = (nch + 63) / 64;
    const dim3 block(256);
    const bool aligned = aligned16(in) && aligned16(out) && n % 4 == 0 &&
                         ((in_row_stride % 4 == 0 && out_row_stride % 4 == 0) || n_rows == 1);
    const int mode = per_lane <= 4 ? PITON_SM_SHORT : per_lane <= 8 ? PITON_SM_MID : per_lane <= 16 ? PITON_SM_LONG : 2;
    const int64_t wgs = (n_rows + 3) / 4;
#define PITON_SM(CH)                                                                                                \
    do {                                                                                                            \
        if (aligned)                                                                                                \
            launch_rows<CH, true>(mode, wgs, st, out, in, in_row_stride, out_row_stride, (int)n, n_rows);          \
        else                                                                                                        \
            launch_rows<CH, false>(mode, wgs, st, out, in, in_row_stride, out_row_stride, (int)n, n_rows);         \
    } while (0)
#define PITON_SM_WG(CH, T)                                                                                          \
    do {                                                                                                            \
        if (aligned)                                                                                                \
            PITON_LAUNCH((softmax_wg_kernel<CH, T, true>), dim3((unsigned)n_rows), dim3(T), 0, st, out, in,   \
                               in_row_stride, out_row_stride, (int)n, phase_slot());                                \
        else                                                                                                        \
            PITON_LAUNCH((softmax_wg_kernel<CH, T, false>), dim3((unsigned)n_rows), dim3(T), 0, st, out, in,  \
                               in_row_stride, out_row_stride, (int)n, phase_slot());                                \
    } while (0)
    PITON_REQUIRE(mode != 2 || n_rows <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "softmax: too many rows");
    PITON_REQUIRE(mode == 2 || wgs <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "softmax: too many rows");
    if (per_lane <= 1) PITON_SM(1);
    else if (per_lane <= 2) PITON_SM(2);
    else if (per_lane <= 4) PITON_SM(4);
    else if (per_lane <= 8 && mode != 2) PITON_SM(8);
    else if (per_lane <= 8) PITON_SM_WG(PITON_SM_MID_CH, PITON_SM_MID_CH == 2 ? 256 : 512);
    else if (per_lane <= 16 && mode != 2) PITON_SM(16);
    else if (per_lane <= 16) PITON_SM_WG(PITON_SM_LONG_CH, 64 * PITON_SM_LONG_CH == 256 ? 256 : 512);
    else if (per_lane <= 32) PITON_SM_WG(8, 256);
    else if (per_lane <= 64) PITON_SM_WG(16, 256);
    else
        PITON_LAUNCH(softmax_long_kernel, dim3((unsigned)n_rows), block, 0, st, out, in, in_row_stride,
                           out_row_stride, n);
#undef PITON_SM_WG
#undef PITON_SM
    rc = check_launch("softmax");
    if (rc == PITON_OK) clear_error();
    return rc;
}
