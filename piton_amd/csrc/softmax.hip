// Row softmax: softmax_kernel (examples/kernels.py:60-76), HBM-bound.
//
// Design (gfx950):
//   * one 64-lane wavefront per row, four rows per 256-thread workgroup, no LDS and no
//     barriers: the row is loaded once into registers (CH float4 chunks per lane), reduced
//     twice with DPP lane moves (max, then sum), and written once: 8 bytes of HBM traffic per
//     element, the minimum;
//   * rows need not be 16-byte aligned (n = 1823): each row is read through the aligned
//     float4 window that covers it, and elements outside [0, n) of the row are masked to
//     -inf. An aligned 16-byte block lies inside one page, so the window never touches an
//     unmapped address. Stores use float4 where the output row has the same alignment as the
//     input row and the chunk is whole, scalar stores at the row's two ends;
//   * exp is v_exp_f32 on x*log2(e) with the product's rounding error added back (one FMA),
//     so each e^x is within about 1 ulp; the row sum's reciprocal is correctly rounded;
//   * special values follow IEEE/numpy: a +inf or NaN entry, or an all -inf row, makes the
//     whole row NaN; a -inf entry in a finite row gives exactly 0;
//   * rows longer than 8189 columns take a workgroup-per-row kernel that reads the row three
//     times (max, sum, write).
#include "common.h"

namespace piton {

__device__ __forceinline__ float exp_acc(float d) {
    const float kL2E = 1.44269502162933349609375f;  // float(log2 e)
    const float kL2ELo = 1.925963033500011e-08f;     // log2 e - kL2E
    d = d < -160.f ? -160.f : d;                     // e^-160 is 0 in float32; NaN passes
    const float t = d * kL2E;
    const float lo = fmaf(d, kL2E, -t) + d * kL2ELo;
    const float e = __builtin_amdgcn_exp2f(t);
    return fmaf(e, lo * 0.69314718055994531f, e);
}

template <int CH>
__global__ __launch_bounds__(256) void softmax_rows_kernel(float *out, const float *in, int64_t in_rs, int64_t out_rs,
                                                           int64_t n, int64_t rows) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= rows) return;  // whole wavefront leaves together
    const float *rp = in + row * in_rs;
    const int off = (int)((reinterpret_cast<uintptr_t>(rp) >> 2) & 3);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(rp - off);
    const int64_t nch = (off + n + 3) >> 2;

    float v[CH][4];
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int64_t ci = lane + 64 * c;
        f32x4 f = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (ci < nch) f = __builtin_nontemporal_load(src + ci);
        const int64_t e0 = 4 * ci - off;
        v[c][0] = (e0 >= 0 && e0 < n) ? f.x : -INFINITY;
        v[c][1] = (e0 + 1 >= 0 && e0 + 1 < n) ? f.y : -INFINITY;
        v[c][2] = (e0 + 2 >= 0 && e0 + 2 < n) ? f.z : -INFINITY;
        v[c][3] = (e0 + 3 < n) ? f.w : -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; j++) mx = fmaxf(mx, v[c][j]);
    }
    const float m = wave_reduce(mx, MaxOp());

    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int64_t e0 = 4 * (int64_t)(lane + 64 * c) - off;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool ok = e0 + j >= 0 && e0 + j < n;
            const float e = ok ? exp_acc(v[c][j] - m) : 0.f;
            v[c][j] = e;
            s += e;
        }
    }
    s = wave_reduce(s, SumOp());
    const float inv = 1.0f / s;

    float *op = out + row * out_rs;
    const int ooff = (int)((reinterpret_cast<uintptr_t>(op) >> 2) & 3);
    if (ooff == off) {
        f32x4 *dst = reinterpret_cast<f32x4 *>(op - off);
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int64_t ci = lane + 64 * c;
            if (ci >= nch) continue;
            const int64_t e0 = 4 * ci - off;
            if (e0 >= 0 && e0 + 3 < n) {
                const f32x4 w = {v[c][0] * inv, v[c][1] * inv, v[c][2] * inv, v[c][3] * inv};
                __builtin_nontemporal_store(w, dst + ci);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (e0 + j >= 0 && e0 + j < n) op[e0 + j] = v[c][j] * inv;
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int64_t e0 = 4 * (int64_t)(lane + 64 * c) - off;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (e0 + j >= 0 && e0 + j < n) op[e0 + j] = v[c][j] * inv;
        }
    }
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
    for (int64_t i = threadIdx.x; i < n; i += 256) s += exp_acc(rp[i] - m);
    s = block_reduce(s, red, false);
    const float inv = 1.0f / s;
    for (int64_t i = threadIdx.x; i < n; i += 256) op[i] = exp_acc(rp[i] - m) * inv;
}

}  // namespace piton

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
    const dim3 grid((unsigned)((n_rows + 3) / 4)), block(256);
    PITON_REQUIRE(n_rows <= 0x7FFFFFFFLL * 4, PITON_EUNSUPPORTED, "softmax: too many rows");
    if (per_lane <= 1) hipLaunchKernelGGL(softmax_rows_kernel<1>, grid, block, 0, st, out, in, in_row_stride, out_row_stride, n, n_rows);
    else if (per_lane <= 2) hipLaunchKernelGGL(softmax_rows_kernel<2>, grid, block, 0, st, out, in, in_row_stride, out_row_stride, n, n_rows);
    else if (per_lane <= 4) hipLaunchKernelGGL(softmax_rows_kernel<4>, grid, block, 0, st, out, in, in_row_stride, out_row_stride, n, n_rows);
    else if (per_lane <= 8) hipLaunchKernelGGL(softmax_rows_kernel<8>, grid, block, 0, st, out, in, in_row_stride, out_row_stride, n, n_rows);
    else if (per_lane <= 16) hipLaunchKernelGGL(softmax_rows_kernel<16>, grid, block, 0, st, out, in, in_row_stride, out_row_stride, n, n_rows);
    else if (per_lane <= 32) hipLaunchKernelGGL(softmax_rows_kernel<32>, grid, block, 0, st, out, in, in_row_stride, out_row_stride, n, n_rows);
    else {
        PITON_REQUIRE(n_rows <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "softmax: too many rows");
        hipLaunchKernelGGL(softmax_long_kernel, dim3((unsigned)n_rows), block, 0, st, out, in, in_row_stride,
                           out_row_stride, n);
    }
    rc = check_launch("softmax");
    if (rc == PITON_OK) clear_error();
    return rc;
}
