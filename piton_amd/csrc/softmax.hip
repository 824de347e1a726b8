// Row softmax: softmax_kernel (examples/kernels.py:60-76), HBM-bound.
//
// Design (gfx950):
//   * one 64-lane wavefront per row at a time, four wavefronts per 256-thread workgroup, no
//     LDS and no barriers: the row is loaded once into registers (CH float4 chunks per lane),
//     reduced twice with DPP lane moves (max, then sum), and written once: 8 bytes of HBM
//     traffic per element, the minimum. Rows of 8+ chunks per lane go two to a wavefront,
//     the second row's loads issued before the first row is reduced and written;
//   * loads and stores are nontemporal: the row is touched once;
//   * rows need not be 16-byte aligned (n = 1823): each row is read through the aligned
//     float4 window that covers it, and elements outside [0, n) of the row are masked to
//     -inf. An aligned 16-byte block lies inside one page, so the window never touches an
//     unmapped address. Stores use float4 where the output row has the same alignment as the
//     input row and the chunk is whole, scalar stores at the row's two ends;
//   * exp is v_exp_f32 on x*log2(e) with the product's rounding error added back (one FMA),
//     so each e^x is within about 1 ulp; the row sum's reciprocal is correctly rounded;
//   * special values follow IEEE/numpy: a +inf or NaN entry, or an all -inf row, makes the
//     whole row NaN; a -inf entry in a finite row gives exactly 0;
//   * rows longer than 4093 columns take a workgroup-per-row kernel that reads the row three
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

// Loads row r's aligned float4 window (CH chunks per lane) into b; elements of the window
// outside the row are masked when the row is processed.
template <int CH, bool ALIGNED>
__device__ __forceinline__ void load_row(const float *in, int64_t in_rs, int64_t r, int n, int lane,
                                         f32x4 (&b)[CH], int &off) {
    const float *rp = in + r * in_rs;
    off = ALIGNED ? 0 : (int)((reinterpret_cast<uintptr_t>(rp) >> 2) & 3);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(rp - off);
    const int nch = (off + n + 3) >> 2;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ci = lane + 64 * c;
        f32x4 f = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (ci < nch) f = __builtin_nontemporal_load(src + ci);
        b[c] = f;
    }
}

// RPW consecutive rows per wavefront: the next row's loads are issued before the current row
// is reduced and stored, so every wave keeps reads in flight while it writes.
// ALIGNED: every row of in and out starts 16-byte aligned and n % 4 == 0, so windows are the
// rows themselves and only whole chunks need a bound. Rows here are < 8190 columns: element
// indices inside a row fit 32 bits.
template <int CH, int RPW, bool ALIGNED>
__global__ __launch_bounds__(256) void softmax_rows_kernel(float *out, const float *in, int64_t in_rs, int64_t out_rs,
                                                           int n, int64_t rows) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t r0 = ((int64_t)blockIdx.x * 4 + wave) * RPW;
    if (r0 >= rows) return;  // whole wavefront leaves together
    const int64_t r1 = r0 + RPW < rows ? r0 + RPW : rows;

    f32x4 cur[CH], nxt[CH];
    int off, off_next = 0;
    load_row<CH, ALIGNED>(in, in_rs, r0, n, lane, cur, off);
    for (int64_t row = r0; row < r1; row++) {
        if (RPW > 1 && row + 1 < r1) load_row<CH, ALIGNED>(in, in_rs, row + 1, n, lane, nxt, off_next);
        const int nch = (off + n + 3) >> 2;
        // mask the window to the row in place (-inf outside [0, n))
        float mx = -INFINITY;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int e0 = 4 * (lane + 64 * c) - off;
            if (ALIGNED) {
                if (e0 >= n) cur[c] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (!(e0 + j >= 0 && e0 + j < n)) cur[c][j] = -INFINITY;
            }
            mx = fmaxf(mx, fmaxf(fmaxf(cur[c].x, cur[c].y), fmaxf(cur[c].z, cur[c].w)));
        }
        const float m = wave_reduce(mx, MaxOp());

        float s = 0.f;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int e0 = 4 * (lane + 64 * c) - off;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool ok = ALIGNED ? e0 < n : (e0 + j >= 0 && e0 + j < n);
                const float e = ok ? exp_acc(cur[c][j] - m) : 0.f;
                cur[c][j] = e;
                s += e;
            }
        }
        s = wave_reduce(s, SumOp());
        const float inv = 1.0f / s;

        float *op = out + row * out_rs;
        const int ooff = ALIGNED ? 0 : (int)((reinterpret_cast<uintptr_t>(op) >> 2) & 3);
        if (ooff == off) {
            f32x4 *dst = reinterpret_cast<f32x4 *>(op - off);
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const int ci = lane + 64 * c;
                if (ci >= nch) continue;
                const int e0 = 4 * ci - off;
                if (ALIGNED || (e0 >= 0 && e0 + 3 < n)) {
                    __builtin_nontemporal_store(cur[c] * inv, dst + ci);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (e0 + j >= 0 && e0 + j < n) op[e0 + j] = cur[c][j] * inv;
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const int e0 = 4 * (lane + 64 * c) - off;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (e0 + j >= 0 && e0 + j < n) op[e0 + j] = cur[c][j] * inv;
            }
        }
        if (RPW > 1) {
#pragma unroll
            for (int c = 0; c < CH; c++) cur[c] = nxt[c];
            off = off_next;
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
    const dim3 block(256);
    // two rows per wave once a row is 8+ chunks per lane (measured: the next row's reads
    // overlap the current row's writes); one row per wave for short rows
    const dim3 grid1((unsigned)((n_rows + 3) / 4)), grid2((unsigned)((n_rows + 7) / 8));
    PITON_REQUIRE(n_rows <= 0x7FFFFFFFLL * 4, PITON_EUNSUPPORTED, "softmax: too many rows");
    const bool aligned = aligned16(in) && aligned16(out) && n % 4 == 0 &&
                         ((in_row_stride % 4 == 0 && out_row_stride % 4 == 0) || n_rows == 1);
#define PITON_SM(CH, RPW, G)                                                                                        \
    do {                                                                                                            \
        if (aligned)                                                                                                \
            hipLaunchKernelGGL((softmax_rows_kernel<CH, RPW, true>), G, block, 0, st, out, in, in_row_stride,       \
                               out_row_stride, (int)n, n_rows);                                                     \
        else                                                                                                        \
            hipLaunchKernelGGL((softmax_rows_kernel<CH, RPW, false>), G, block, 0, st, out, in, in_row_stride,      \
                               out_row_stride, (int)n, n_rows);                                                     \
    } while (0)
    if (per_lane <= 1) PITON_SM(1, 1, grid1);
    else if (per_lane <= 2) PITON_SM(2, 1, grid1);
    else if (per_lane <= 4) PITON_SM(4, 1, grid1);
    else if (per_lane <= 8) PITON_SM(8, 2, grid2);
    else if (per_lane <= 16) PITON_SM(16, 2, grid2);
    else {
        PITON_REQUIRE(n_rows <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "softmax: too many rows");
        hipLaunchKernelGGL(softmax_long_kernel, dim3((unsigned)n_rows), block, 0, st, out, in, in_row_stride,
                           out_row_stride, n);
    }
#undef PITON_SM
    rc = check_launch("softmax");
    if (rc == PITON_OK) clear_error();
    return rc;
}
