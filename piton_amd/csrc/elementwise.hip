// HBM-bound kernels of the decoder chain: add_kernel (examples/kernels.py:6-15), the
// test-local layernorm_kernel (tests/test_reroll_reduce.py:199-208) and the token/position
// embedding gather the decoder needs (no reference counterpart).
#include "common.h"

namespace piton {

// out = x + y: float4 when all three pointers are 16-byte aligned, grid-stride loop.
__global__ __launch_bounds__(256) void add_vec4_kernel(const f32x4 *x, const f32x4 *y, f32x4 *out, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const f32x4 a = __builtin_nontemporal_load(x + i), b = __builtin_nontemporal_load(y + i);
        __builtin_nontemporal_store(a + b, out + i);
    }
}

__global__ __launch_bounds__(256) void add_scalar_kernel(const float *x, const float *y, float *out, int64_t begin,
                                                         int64_t n) {
    for (int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = x[i] + y[i];
}

// Layernorm, one wavefront per row (CH float4 chunks per lane, rows read as in the softmax
// kernel through their aligned float4 window): mean and biased variance by DPP reductions,
// then (x - mean) * (1 / sqrt(var + eps)) with a correctly rounded square root and reciprocal.
template <int CH>
__global__ __launch_bounds__(256) void layernorm_rows_kernel(const float *x, float *out, int64_t n, float eps,
                                                             int64_t rows, int64_t rs) {
    eps = sgpr_keep(eps);  // read with the other arguments, not reloaded after the mean
    out = sgpr_keep(out);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= rows) return;
    const float *rp = x + row * rs;
    const int off = (int)((reinterpret_cast<uintptr_t>(rp) >> 2) & 3);
    const float4 *src = reinterpret_cast<const float4 *>(rp - off);
    const int64_t nch = (off + n + 3) >> 2;
    float v[CH][4];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int64_t ci = lane + 64 * c;
        float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ci < nch) f = src[ci];
        const int64_t e0 = 4 * ci - off;
        v[c][0] = (e0 >= 0 && e0 < n) ? f.x : 0.f;
        v[c][1] = (e0 + 1 >= 0 && e0 + 1 < n) ? f.y : 0.f;
        v[c][2] = (e0 + 2 >= 0 && e0 + 2 < n) ? f.z : 0.f;
        v[c][3] = (e0 + 3 < n) ? f.w : 0.f;
        s += (v[c][0] + v[c][1]) + (v[c][2] + v[c][3]);
    }
    const float mean = wave_reduce(s, SumOp()) / (float)n;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int64_t e0 = 4 * (int64_t)(lane + 64 * c) - off;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool ok = e0 + j >= 0 && e0 + j < n;
            v[c][j] = ok ? v[c][j] - mean : 0.f;
            q = fmaf(v[c][j], v[c][j], q);
        }
    }
    const float var = wave_reduce(q, SumOp()) / (float)n;
    const float inv = 1.0f / sqrtf(var + eps);
    float *op = out + row * rs;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int64_t e0 = 4 * (int64_t)(lane + 64 * c) - off;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (e0 + j >= 0 && e0 + j < n) op[e0 + j] = v[c][j] * inv;
    }
}

// out[b, t, :] = tok[ids[b, t], :] + pos[pos_offset + t, :] through element strides
__global__ __launch_bounds__(256) void embedding_kernel(const int32_t *ids, int64_t ids_sb, int64_t ids_st,
                                                        const float *tok, const float *pos, float *out, int64_t out_sb,
                                                        int64_t out_st, int64_t T, int64_t d, int64_t vocab,
                                                        int64_t pos_offset, int64_t total, int32_t *err) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t bt = i / d, c = i % d;
        const int64_t b = bt / T, t = bt % T;
        const int32_t id = ids[b * ids_sb + t * ids_st];
        float *o = out + b * out_sb + t * out_st + c;
        if (id < 0 || id >= vocab) {
            *o = __int_as_float(0x7FC00000);
            if (err) *err = 1;
        } else {
            *o = tok[(int64_t)id * d + c] + pos[(pos_offset + t) * d + c];
        }
    }
}

static unsigned grid_for(int64_t work) {
    int64_t g = (work + 255) / 256;
    if (g > 256 * 64) g = 256 * 64;  // 64 workgroups per CU, then grid-stride
    return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace piton

extern "C" {

int32_t piton_mi355x_add(const float *x, const float *y, float *out, int64_t n, void *stream) {
    using namespace piton;
    PITON_REQUIRE(n >= 0, PITON_EINVAL, "add: negative n");
    PITON_REQUIRE(n == 0 || (x && y && out), PITON_EINVAL, "add: null pointer");
    PITON_REQUIRE(aligned4(x) && aligned4(y) && aligned4(out), PITON_EINVAL, "add: pointers must be 4-byte aligned");
    int rc = require_device();
    if (rc) return rc;
    if (n == 0) return PITON_OK;
    hipStream_t st = (hipStream_t)stream;
    int64_t done = 0;
    if (aligned16(x) && aligned16(y) && aligned16(out) && n >= 4) {
        const int64_t n4 = n / 4;
        PITON_LAUNCH(add_vec4_kernel, dim3(grid_for(n4)), dim3(256), 0, st, reinterpret_cast<const f32x4 *>(x),
                           reinterpret_cast<const f32x4 *>(y), reinterpret_cast<f32x4 *>(out), n4);
        done = n4 * 4;
    }
    if (done < n) PITON_LAUNCH(add_scalar_kernel, dim3(grid_for(n - done)), dim3(256), 0, st, x, y, out, done, n);
    rc = check_launch("add");
    if (rc == PITON_OK) clear_error();
    return rc;
}

int32_t piton_mi355x_layernorm(const float *x, float *out, int64_t n, float eps, int64_t rows, int64_t row_stride,
                               void *stream) {
    using namespace piton;
    PITON_REQUIRE(n >= 1 && rows >= 0, PITON_EINVAL, "layernorm: n=%lld rows=%lld", (long long)n, (long long)rows);
    PITON_REQUIRE(rows <= 1 || row_stride >= n, PITON_EINVAL, "layernorm: row stride %lld < n %lld",
                  (long long)row_stride, (long long)n);
    PITON_REQUIRE(rows == 0 || (x && out), PITON_EINVAL, "layernorm: null pointer");
    PITON_REQUIRE(aligned4(x) && aligned4(out), PITON_EINVAL, "layernorm: pointers must be 4-byte aligned");
    const bool all_aligned = aligned16(x) && (row_stride % 4 == 0 || rows == 1);
    const int64_t per_lane = ((n + 3 + (all_aligned ? 0 : 3)) / 4 + 63) / 64;
    PITON_REQUIRE(per_lane <= 32, PITON_EUNSUPPORTED, "layernorm: rows of %lld elements exceed 8189", (long long)n);
    int rc = require_device();
    if (rc) return rc;
    if (rows == 0) return PITON_OK;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    if (per_lane <= 1) PITON_LAUNCH(layernorm_rows_kernel<1>, grid, block, 0, st, x, out, n, eps, rows, row_stride);
    else if (per_lane <= 2) PITON_LAUNCH(layernorm_rows_kernel<2>, grid, block, 0, st, x, out, n, eps, rows, row_stride);
    else if (per_lane <= 4) PITON_LAUNCH(layernorm_rows_kernel<4>, grid, block, 0, st, x, out, n, eps, rows, row_stride);
    else if (per_lane <= 8) PITON_LAUNCH(layernorm_rows_kernel<8>, grid, block, 0, st, x, out, n, eps, rows, row_stride);
    else if (per_lane <= 16) PITON_LAUNCH(layernorm_rows_kernel<16>, grid, block, 0, st, x, out, n, eps, rows, row_stride);
    else PITON_LAUNCH(layernorm_rows_kernel<32>, grid, block, 0, st, x, out, n, eps, rows, row_stride);
    rc = check_launch("layernorm");
    if (rc == PITON_OK) clear_error();
    return rc;
}

int32_t piton_mi355x_embedding(const int32_t *ids, int64_t ids_sb, int64_t ids_st, const float *tok, const float *pos,
                               float *out, int64_t out_sb, int64_t out_st, int64_t batch, int64_t T, int64_t d_model,
                               int64_t vocab, int64_t pos_offset, int32_t *err_flag, void *stream) {
    using namespace piton;
    PITON_REQUIRE(batch >= 0 && T >= 0 && d_model >= 1 && vocab >= 1 && pos_offset >= 0, PITON_EINVAL,
                  "embedding: batch=%lld T=%lld d_model=%lld vocab=%lld pos_offset=%lld", (long long)batch,
                  (long long)T, (long long)d_model, (long long)vocab, (long long)pos_offset);
    PITON_REQUIRE(batch * T == 0 || (ids && tok && pos && out), PITON_EINVAL, "embedding: null pointer");
    int rc = require_device();
    if (rc) return rc;
    const int64_t total = batch * T * d_model;
    if (total == 0) return PITON_OK;
    PITON_LAUNCH(embedding_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream, ids, ids_sb, ids_st,
                       tok, pos, out, out_sb, out_st, T, d_model, vocab, pos_offset, total, err_flag);
    rc = check_launch("embedding");
    if (rc == PITON_OK) clear_error();
    return rc;
}

}  // extern "C"
