// The perf suite's primitives (perf/suite.py:323-351) on gfx950: copy, mul, fma, scaled_relu,
// the special functions of sfu_kernel (examples/sfu_tests.py:6-22) and log, exact int32 //
// and %, row sums and maxima, and the tiled transpose (examples/primitive_kernels.py:13-76,
// examples/kernels.py:80-96, examples/elementwise.py:6-9).
//
// Every one of them moves more bytes than it computes, so each is shaped for HBM:
//   * elementwise: one 16-byte vector per thread on an exact grid (many short workgroups keep
//     reads and writes interleaved), nontemporal loads and stores, a scalar tail for n % 4;
//   * special functions use the device math library (expf, exp2f, logf, log2f, sqrtf) and an
//     IEEE division for the reciprocal and 1/sqrt: within a few ulp, inside the suite's 4e-6;
//   * row reductions: one wavefront per row, float4 loads along the row, DPP reductions;
//   * transpose: 128 x 128 tiles through LDS, 1024 threads, 16-byte nontemporal loads and
//     stores when rows, strides and pointers allow it (LDS row pitch 129), else 64 x 64 scalar
//     tiles (row stride 65); reads and writes are coalesced rows either way. Measured at
//     8192 x 8192: 64 x 64 scalar 130 us, 64 x 128 float4 113 us, 128 x 128 float4 with 256 /
//     512 / 1024 threads 106 / 99 / 98 us, and 90 us with the tiles walked down the columns
//     (a copy of the same bytes: 81 us).
#include <math.h>

#include "common.h"

namespace piton {

struct CopyOp { __device__ float operator()(float x, float, float) const { return x; } };
struct MulOp { __device__ float operator()(float x, float y, float) const { return x * y; } };
struct FmaOp { __device__ float operator()(float x, float y, float a) const { return x * a + y; } };
struct ScaledReluOp { __device__ float operator()(float x, float, float a) const { return x > 0.f ? x * a : 0.f; } };
struct Exp2Op { __device__ float operator()(float x, float, float) const { return exp2f(x); } };
struct Log2Op { __device__ float operator()(float x, float, float) const { return log2f(x); } };
struct RecipOp { __device__ float operator()(float x, float, float) const { return 1.0f / x; } };
struct RsqrtOp { __device__ float operator()(float x, float, float) const { return 1.0f / sqrtf(x); } };
struct ExpOp { __device__ float operator()(float x, float, float) const { return expf(x); } };
struct SqrtOp { __device__ float operator()(float x, float, float) const { return sqrtf(x); } };
struct LogOp { __device__ float operator()(float x, float, float) const { return logf(x); } };

// out[i] = op(x[i], y[i], alpha) for i < n; y may be null for one-input ops
template <class Op, bool TWO>
__global__ __launch_bounds__(256) void map_vec4_kernel(const f32x4 *x, const f32x4 *y, f32x4 *out, int64_t n4,
                                                       float alpha) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const f32x4 a = __builtin_nontemporal_load(x + i);
    const f32x4 b = TWO ? __builtin_nontemporal_load(y + i) : a;
    Op op;
    __builtin_nontemporal_store(f32x4{op(a.x, b.x, alpha), op(a.y, b.y, alpha), op(a.z, b.z, alpha),
                                      op(a.w, b.w, alpha)}, out + i);
}

template <class Op, bool TWO>
__global__ __launch_bounds__(256) void map_scalar_kernel(const float *x, const float *y, float *out, int64_t begin,
                                                         int64_t n, float alpha) {
    const int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    Op op;
    out[i] = op(x[i], TWO ? y[i] : 0.f, alpha);
}

template <class Op, bool TWO>
static int launch_map(const float *x, const float *y, float *out, int64_t n, float alpha, hipStream_t st,
                      const char *what) {
    if (n == 0) return PITON_OK;
    const bool vec = aligned16(x) && aligned16(out) && (!TWO || aligned16(y));
    const int64_t n4 = vec ? n / 4 : 0;
    PITON_REQUIRE((n4 + 255) / 256 <= 0x7FFFFFFF && (n - 4 * n4 + 255) / 256 <= 0x7FFFFFFF, PITON_EUNSUPPORTED,
                  "%s: n=%lld too large", what, (long long)n);
    if (n4 > 0)
        PITON_LAUNCH((map_vec4_kernel<Op, TWO>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                           reinterpret_cast<const f32x4 *>(x), reinterpret_cast<const f32x4 *>(y),
                           reinterpret_cast<f32x4 *>(out), n4, alpha);
    if (4 * n4 < n)
        PITON_LAUNCH((map_scalar_kernel<Op, TWO>), dim3((unsigned)((n - 4 * n4 + 255) / 256)), dim3(256), 0,
                           st, x, y, out, 4 * n4, n, alpha);
    return check_launch(what);
}

// C-style (truncating) quotient and remainder: q = trunc(x / y), r = x - q y. VEC: four
// elements per thread through 16-byte vectors (i indexes vectors), else one.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

template <bool VEC>
__global__ __launch_bounds__(256) void idiv_kernel(const int32_t *x, const int32_t *y, int32_t *q, int32_t *r,
                                                   int64_t begin, int64_t n) {
    const int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    if constexpr (VEC) {
        const i32x4 a = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(x) + i);
        const i32x4 b = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(y) + i);
        const i32x4 qq = a / b;
        __builtin_nontemporal_store(qq, reinterpret_cast<i32x4 *>(q) + i);
        __builtin_nontemporal_store(a - qq * b, reinterpret_cast<i32x4 *>(r) + i);
    } else {
        const int32_t a = x[i], b = y[i];
        const int32_t qq = a / b;
        q[i] = qq;
        r[i] = a - qq * b;
    }
}

// out[r] = sum / max of x[r, 0:n_cols] (row stride `stride`), one wave per row
template <bool MAX>
__global__ __launch_bounds__(256) void row_reduce_kernel(const float *x, float *out, int64_t rows, int64_t n_cols,
                                                         int64_t stride, int vec) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wavefront leaves together
    const float *p = x + row * stride;
    float acc = MAX ? -3.4028234663852886e+38f : 0.f;
    int64_t c0 = 0;
    if (vec) {
        const int64_t n4 = n_cols / 4;
        auto fold = [&](const f32x4 &v) {
            return MAX ? fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)) : (v.x + v.y) + (v.z + v.w);
        };
        int64_t i = lane;
        // four 16-byte loads in flight per lane, folded in a fixed order
        for (; i + 192 < n4; i += 256) {
            const f32x4 *q = reinterpret_cast<const f32x4 *>(p) + i;
            const f32x4 v0 = __builtin_nontemporal_load(q), v1 = __builtin_nontemporal_load(q + 64);
            const f32x4 v2 = __builtin_nontemporal_load(q + 128), v3 = __builtin_nontemporal_load(q + 192);
            const float f = MAX ? fmaxf(fmaxf(fold(v0), fold(v1)), fmaxf(fold(v2), fold(v3)))
                                : (fold(v0) + fold(v1)) + (fold(v2) + fold(v3));
            acc = MAX ? fmaxf(acc, f) : acc + f;
        }
        for (; i < n4; i += 64) {
            const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p) + i);
            acc = MAX ? fmaxf(acc, fold(v)) : acc + fold(v);
        }
        c0 = 4 * n4;
    }
    for (int64_t c = c0 + lane; c < n_cols; c += 64) acc = MAX ? fmaxf(acc, p[c]) : acc + p[c];
    acc = MAX ? wave_reduce(acc, MaxOp()) : wave_reduce(acc, SumOp());
    if (lane == 0) out[row] = acc;
}

// out[c, r] = x[r, c]: 64 x 64 tiles, 256 threads, through LDS
__global__ __launch_bounds__(256) void transpose_kernel(const float *x, float *out, int64_t n_rows, int64_t n_cols,
                                                        int64_t stride_x, int64_t stride_out, int64_t tiles_n) {
    __shared__ float tile[64][65];
    const int64_t tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int64_t r0 = tm * 64, c0 = tn * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int rr = ty + 4 * k;
        const int64_t r = r0 + rr, c = c0 + tx;
        if (r < n_rows && c < n_cols) tile[rr][tx] = x[r * stride_x + c];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int cc = ty + 4 * k;
        const int64_t c = c0 + cc, r = r0 + tx;
        if (c < n_cols && r < n_rows) out[c * stride_out + r] = tile[tx][cc];
    }
}

// Aligned transpose: x 16-byte aligned with stride_x % 4 == 0 and n_cols % 4 == 0, out
// likewise with n_rows % 4 == 0. A workgroup moves a kTrR-row x kTrC-column tile: the threads
// load float4 along the input rows, and store float4 along the output rows, each the 4 input
// rows 4q..4q+3 of one input column (LDS row pitch kTrC + 1).
#ifndef PITON_TR_R
#define PITON_TR_R 128
#endif
#ifndef PITON_TR_C
#define PITON_TR_C 128
#endif
#ifndef PITON_TR_T
#define PITON_TR_T 1024
#endif
constexpr int kTrR = PITON_TR_R, kTrC = PITON_TR_C, kTrT = PITON_TR_T;
__global__ __launch_bounds__(kTrT) void transpose_vec_kernel(const float *x, float *out, int64_t n_rows, int64_t n_cols,
                                                             int64_t stride_x, int64_t stride_out, int64_t tiles_r) {
    constexpr int LPR = kTrC / 4, LP = kTrR * kTrC / (4 * kTrT);  // load: threads per input row, passes
    constexpr int SPR = kTrR / 4, SP = LP;                         // store: threads per output row, passes
    __shared__ float tile[kTrR][kTrC + 1];
    // consecutive workgroups walk down a column band of tiles: the workgroups in flight write
    // long runs of the same output rows (8192^2: 0.69 -> 0.74 of HBM; across 8192^2, 4096^2,
    // 16384 x 4096 and 4096 x 16384 0.63 -> 0.68 on average, where groups of 4-32 row tiles
    // measured 0.64-0.675 and the XCD-contiguous order 0.63)
    const int64_t r0 = (int64_t)(blockIdx.x % tiles_r) * kTrR, c0 = (int64_t)(blockIdx.x / tiles_r) * kTrC;
    const int t = threadIdx.x;
    const int cq = t % LPR, rb = t / LPR;
    f32x4 v[LP];
#pragma unroll
    for (int k = 0; k < LP; k++) {
        const int64_t r = r0 + rb + (kTrT / LPR) * k, c = c0 + 4 * cq;
        v[k] = (r < n_rows && c < n_cols) ? __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x + r * stride_x + c))
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < LP; k++)
#pragma unroll
        for (int e = 0; e < 4; e++) tile[rb + (kTrT / LPR) * k][4 * cq + e] = v[k][e];
    __syncthreads();
    const int oq = t % SPR, ob = t / SPR;
#pragma unroll
    for (int k = 0; k < SP; k++) {
        const int oc = ob + (kTrT / SPR) * k;
        const int64_t c = c0 + oc, r = r0 + 4 * oq;
        if (c < n_cols && r < n_rows)
            __builtin_nontemporal_store(f32x4{tile[4 * oq][oc], tile[4 * oq + 1][oc], tile[4 * oq + 2][oc],
                                              tile[4 * oq + 3][oc]},
                                        reinterpret_cast<f32x4 *>(out + c * stride_out + r));
    }
}

}  // namespace piton

using namespace piton;

#define PITON_MAP_ENTRY_CHECKS(what, two)                                                                   \
    PITON_REQUIRE(n >= 0, PITON_EINVAL, what ": negative n=%lld", (long long)n);                            \
    PITON_REQUIRE(n == 0 || (x && out && (!(two) || y)), PITON_EINVAL, what ": null pointer");              \
    PITON_REQUIRE(aligned4(x) && aligned4(out) && aligned4(y), PITON_EINVAL, what ": pointers must be 4-byte aligned"); \
    int rc = require_device();                                                                              \
    if (rc) return rc

static int32_t finish(int rc) {
    if (rc == PITON_OK) clear_error();
    return rc;
}

extern "C" {

int32_t piton_mi355x_copy(const float *x, float *out, int64_t n, void *stream) {
    const float *y = nullptr;
    PITON_MAP_ENTRY_CHECKS("copy", false);
    return finish(launch_map<CopyOp, false>(x, nullptr, out, n, 0.f, (hipStream_t)stream, "copy"));
}

int32_t piton_mi355x_mul(const float *x, const float *y, float *out, int64_t n, void *stream) {
    PITON_MAP_ENTRY_CHECKS("mul", true);
    return finish(launch_map<MulOp, true>(x, y, out, n, 0.f, (hipStream_t)stream, "mul"));
}

int32_t piton_mi355x_fma(const float *x, const float *y, float *out, int64_t n, float alpha, void *stream) {
    PITON_MAP_ENTRY_CHECKS("fma", true);
    return finish(launch_map<FmaOp, true>(x, y, out, n, alpha, (hipStream_t)stream, "fma"));
}

int32_t piton_mi355x_scaled_relu(const float *x, float *out, int64_t n, float alpha, void *stream) {
    const float *y = nullptr;
    PITON_MAP_ENTRY_CHECKS("scaled_relu", false);
    return finish(launch_map<ScaledReluOp, false>(x, nullptr, out, n, alpha, (hipStream_t)stream, "scaled_relu"));
}

int32_t piton_mi355x_sfu(const float *x, float *out, int64_t n, int32_t op, void *stream) {
    const float *y = nullptr;
    PITON_REQUIRE(op >= 0 && op <= 5, PITON_EINVAL, "sfu: OP %d not in 0..5", op);
    PITON_MAP_ENTRY_CHECKS("sfu", false);
    hipStream_t st = (hipStream_t)stream;
    switch (op) {
        case 0: return finish(launch_map<Exp2Op, false>(x, nullptr, out, n, 0.f, st, "sfu exp2"));
        case 1: return finish(launch_map<Log2Op, false>(x, nullptr, out, n, 0.f, st, "sfu log2"));
        case 2: return finish(launch_map<RecipOp, false>(x, nullptr, out, n, 0.f, st, "sfu recip"));
        case 3: return finish(launch_map<RsqrtOp, false>(x, nullptr, out, n, 0.f, st, "sfu rsqrt"));
        case 4: return finish(launch_map<ExpOp, false>(x, nullptr, out, n, 0.f, st, "sfu exp"));
        default: return finish(launch_map<SqrtOp, false>(x, nullptr, out, n, 0.f, st, "sfu sqrt"));
    }
}

int32_t piton_mi355x_log(const float *x, float *out, int64_t n, void *stream) {
    const float *y = nullptr;
    PITON_MAP_ENTRY_CHECKS("log", false);
    return finish(launch_map<LogOp, false>(x, nullptr, out, n, 0.f, (hipStream_t)stream, "log"));
}

int32_t piton_mi355x_idiv(const int32_t *x, const int32_t *y, int32_t *q, int32_t *r, int64_t n, void *stream) {
    PITON_REQUIRE(n >= 0, PITON_EINVAL, "idiv: negative n=%lld", (long long)n);
    PITON_REQUIRE(n == 0 || (x && y && q && r), PITON_EINVAL, "idiv: null pointer");
    PITON_REQUIRE((n + 255) / 256 <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "idiv: n=%lld too large", (long long)n);
    int rc = require_device();
    if (rc) return rc;
    if (n == 0) return PITON_OK;
    hipStream_t st = (hipStream_t)stream;
    const bool vec = aligned16(x) && aligned16(y) && aligned16(q) && aligned16(r);
    const int64_t n4 = vec ? n / 4 : 0;
    if (n4 > 0)
        PITON_LAUNCH(idiv_kernel<true>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, x, y, q, r,
                           (int64_t)0, n4);
    if (4 * n4 < n)
        PITON_LAUNCH(idiv_kernel<false>, dim3((unsigned)((n - 4 * n4 + 255) / 256)), dim3(256), 0, st, x, y,
                           q, r, 4 * n4, n);
    return finish(check_launch("idiv"));
}

static int32_t row_reduce_entry(bool is_max, const float *x, float *out, int64_t rows, int64_t n_cols, int64_t stride,
                                void *stream) {
    const char *what = is_max ? "row_max" : "row_sum";
    PITON_REQUIRE(rows >= 0 && n_cols >= 0 && (rows <= 1 || stride >= n_cols), PITON_EINVAL,
                  "%s: rows=%lld n_cols=%lld stride=%lld", what, (long long)rows, (long long)n_cols, (long long)stride);
    PITON_REQUIRE(rows == 0 || (x && out), PITON_EINVAL, "%s: null pointer", what);
    PITON_REQUIRE((rows + 3) / 4 <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "%s: too many rows", what);
    int rc = require_device();
    if (rc) return rc;
    if (rows == 0) return PITON_OK;
    const int vec = aligned16(x) && (stride % 4 == 0 || rows == 1);
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    if (is_max) PITON_LAUNCH(row_reduce_kernel<true>, grid, block, 0, (hipStream_t)stream, x, out, rows, n_cols, stride, vec);
    else PITON_LAUNCH(row_reduce_kernel<false>, grid, block, 0, (hipStream_t)stream, x, out, rows, n_cols, stride, vec);
    return finish(check_launch(what));
}

int32_t piton_mi355x_row_sum(const float *x, float *out, int64_t rows, int64_t n_cols, int64_t stride, void *stream) {
    return row_reduce_entry(false, x, out, rows, n_cols, stride, stream);
}

int32_t piton_mi355x_row_max(const float *x, float *out, int64_t rows, int64_t n_cols, int64_t stride, void *stream) {
    return row_reduce_entry(true, x, out, rows, n_cols, stride, stream);
}

int32_t piton_mi355x_transpose(const float *x, float *out, int64_t n_rows, int64_t n_cols, int64_t stride_x,
                               int64_t stride_out, void *stream) {
    PITON_REQUIRE(n_rows >= 0 && n_cols >= 0, PITON_EINVAL, "transpose: negative size");
    PITON_REQUIRE(n_rows <= 1 || stride_x >= n_cols, PITON_EINVAL, "transpose: stride_x %lld < n_cols %lld",
                  (long long)stride_x, (long long)n_cols);
    PITON_REQUIRE(n_cols <= 1 || stride_out >= n_rows, PITON_EINVAL, "transpose: stride_out %lld < n_rows %lld",
                  (long long)stride_out, (long long)n_rows);
    PITON_REQUIRE(n_rows == 0 || n_cols == 0 || (x && out), PITON_EINVAL, "transpose: null pointer");
    const int64_t tiles_m = (n_rows + 63) / 64, tiles_n = (n_cols + 63) / 64;
    PITON_REQUIRE(sat_mul(tiles_m, tiles_n) <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "transpose: too large");
    int rc = require_device();
    if (rc) return rc;
    if (n_rows == 0 || n_cols == 0) return PITON_OK;
    const bool vec = aligned16(x) && aligned16(out) && n_cols % 4 == 0 && n_rows % 4 == 0 &&
                     (stride_x % 4 == 0 || n_rows == 1) && (stride_out % 4 == 0 || n_cols == 1);
    if (vec) {
        const int64_t tr = (n_rows + kTrR - 1) / kTrR, tc = (n_cols + kTrC - 1) / kTrC;
        PITON_LAUNCH(transpose_vec_kernel, dim3((unsigned)(tr * tc)), dim3(kTrT), 0, (hipStream_t)stream, x, out,
                           n_rows, n_cols, stride_x, stride_out, tr);
    } else {
        PITON_LAUNCH(transpose_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), 0, (hipStream_t)stream,
                           x, out, n_rows, n_cols, stride_x, stride_out, tiles_n);
    }
    return finish(check_launch("transpose"));
}

}  // extern "C"
