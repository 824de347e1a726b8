/*
 * libpiton_mi355x.so: hand-written gfx950 (MI355X, CDNA4) kernels for PIton's data-parallel
 * kernel set, behind a plain C ABI.
 *
 * Conventions (every entry point):
 *   - pointers are device pointers owned by the caller; sizes and strides are int64 element
 *     counts; `stream` is a hipStream_t (NULL = the default stream);
 *   - launches are asynchronous on `stream`; nothing is allocated by the library;
 *   - arguments are validated before any HIP call; the return value is a status code below,
 *     and piton_mi355x_last_error() gives this thread's message for the last failure.
 *
 * Each kernel entry replaces one `kernel[grid](...)` launch of the reference
 * (piton/runtime/launcher.py:217-245, the `device == "emu"` / `"pi"` dispatch at :238-244),
 * with the reference kernel's runtime arguments in the same order and meaning.
 */
#ifndef PITON_MI355X_H
#define PITON_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PITON_MI355X_ABI_VERSION 1

#if defined(__GNUC__)
#define PITON_API __attribute__((visibility("default")))
#else
#define PITON_API
#endif

enum {
    PITON_OK = 0,
    PITON_EINVAL = -1,      /* invalid argument (null pointer, negative size, bad flag) */
    PITON_EUNSUPPORTED = -2, /* valid but unsupported shape or layout */
    PITON_EHIP = -3,        /* a HIP call failed; the message names it */
    PITON_ENODEV = -4       /* no usable gfx950 device */
};

typedef struct {
    int32_t cu_count;          /* compute units */
    int32_t max_clock_khz;     /* peak engine clock */
    int32_t mem_clock_khz;     /* memory clock */
    int32_t mem_bus_width;     /* bits */
    int64_t hbm_bytes;         /* device memory */
    int32_t lds_per_cu;        /* bytes of LDS per compute unit (max per workgroup) */
    int32_t l2_bytes;          /* L2 of one XCD as the runtime reports it */
    int32_t wavefront_size;
    int32_t xcd_count;         /* 0 when the runtime does not say */
    char arch[64];             /* gcnArchName */
} piton_device_info_t;

/* One kernel launch made by the last entry call of this thread (piton_mi355x_last_launches). */
typedef struct {
    char kernel[96];           /* the device kernel as the library's source names it */
    uint32_t grid[3];          /* workgroups */
    uint32_t block[3];         /* work-items per workgroup */
    uint32_t lds_bytes;        /* static + dynamic LDS per workgroup */
    int32_t vgprs;             /* vector registers per lane (hipFuncGetAttributes numRegs) */
    uint32_t scratch_bytes;    /* private memory per lane (register spills) */
} piton_launch_info_t;

/* Version of this ABI (PITON_MI355X_ABI_VERSION). No reference counterpart. */
PITON_API int32_t piton_mi355x_abi_version(void);

/* Message of this thread's last failed call ("" if none). No reference counterpart. */
PITON_API const char *piton_mi355x_last_error(void);

/* Properties of the current device, used for roofline figures. No reference counterpart;
 * it plays the role of piton_qpu_count (pi/runtime/piton_rt.h:70). */
PITON_API int32_t piton_mi355x_device_info(piton_device_info_t *out);

/* The kernel launches (up to 8) of this thread's last entry call that reached the device:
 * *count receives their number, and the first min(max, *count) are written to out (out may be
 * NULL when max is 0). The counterpart of the emulator statistics the reference stores in
 * CompiledKernel.last_stats after a launch (piton/runtime/launcher.py:238-245,
 * piton/qpu/emulator.py:1111-1174): what ran, on how many workgroups, with what resources. */
PITON_API int32_t piton_mi355x_last_launches(piton_launch_info_t *out, int32_t max, int32_t *count);

/* matmul_kernel (examples/kernels.py:18-57): C[M,N] = A[M,K] B[K,N] in float32 through six
 * runtime element strides; rows/cols past M/N are never stored and the K tail adds nothing.
 * group_size_m is GROUP_SIZE_M's tile order (>= 1); it changes the order, not the bits. */
PITON_API int32_t piton_mi355x_matmul(const float *a, const float *b, float *c, int64_t M, int64_t N,
                            int64_t K, int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
                            int64_t stride_bn, int64_t stride_cm, int64_t stride_cn,
                            int32_t group_size_m, void *stream);

/* softmax_kernel (examples/kernels.py:60-76): one row per program; the first
 * min(block_size, n_cols) columns of each of n_rows rows are normalised and stored, other
 * columns are untouched. block_size is the kernel's BLOCK_SIZE constexpr (>= 1). */
PITON_API int32_t piton_mi355x_softmax(float *out, const float *in, int64_t in_row_stride,
                             int64_t out_row_stride, int64_t n_cols, int64_t n_rows,
                             int64_t block_size, void *stream);

/* attn_fwd_kernel (examples/attention.py:67-113): Out = softmax(Q K^T sm_scale) V per head,
 * causal or not. Q, V, Out rows are contiguous (last stride 1) with row strides stride_qm,
 * stride_vn, stride_om; K is read through (stride_kn, stride_kk), so [N,D] and pre-transposed
 * [D,N] storage both work; heads advance by the stride_*h arguments. head_dim in
 * {16, 32, 64, 128}. */
PITON_API int32_t piton_mi355x_attn_fwd(const float *q, const float *k, const float *v, float *out,
                              float sm_scale, int64_t stride_qh, int64_t stride_qm,
                              int64_t stride_kh, int64_t stride_kn, int64_t stride_kk,
                              int64_t stride_vh, int64_t stride_vn, int64_t stride_oh,
                              int64_t stride_om, int64_t n_ctx, int64_t n_heads,
                              int32_t head_dim, int32_t causal, void *stream);

/* dense_layer_kernel (examples/nn_kernels.py:23-74): Y[M,N] = [ReLU](X[M,K] W[K,N] [+ bias]),
 * contiguous row-major. When argmax_out is not NULL, it also receives, per row, the first
 * index of the largest of the first n_classes outputs (examples/digits_model.py:137-139),
 * computed from the stored values. */
PITON_API int32_t piton_mi355x_dense(const float *x, const float *w, const float *bias, float *y,
                           int64_t M, int64_t N, int64_t K, int32_t add_bias, int32_t relu,
                           int32_t *argmax_out, int32_t n_classes, void *stream);

/* add_kernel (examples/kernels.py:6-15): out[i] = x[i] + y[i] for i < n. */
PITON_API int32_t piton_mi355x_add(const float *x, const float *y, float *out, int64_t n, void *stream);

/* layernorm_kernel (tests/test_reroll_reduce.py:199-208): over the first n elements of each
 * of `rows` rows (row stride row_stride), (x - mean) / sqrt(var + eps) with the biased
 * variance and no affine; elements past n are untouched. */
PITON_API int32_t piton_mi355x_layernorm(const float *x, float *out, int64_t n, float eps, int64_t rows,
                               int64_t row_stride, void *stream);

/* Host argmax of the digits driver (examples/digits_model.py:137-139; the firmware's scan,
 * pi/examples/digits/main.c:140-145): out[r] = first index of the largest of x[r, 0:n]
 * (a NaN wins at its first position, as numpy's argmax). */
PITON_API int32_t piton_mi355x_argmax_rows(const float *x, int64_t rows, int64_t ld, int64_t n,
                                 int32_t *out, void *stream);

/* Token + position embedding gather. No reference counterpart (the reference has no decoder
 * model): out[b, t, :] = tok[ids[b, t], :] + pos[pos_offset + t, :] for b < batch, t < T, with
 * ids[b, t] at ids[b*ids_sb + t*ids_st] and out[b, t, c] at out[b*out_sb + t*out_st + c]; tok is
 * [vocab, d_model] and pos [>= pos_offset + T, d_model], contiguous. An id outside [0, vocab)
 * writes NaN and sets *err_flag = 1 (err_flag may be NULL). */
PITON_API int32_t piton_mi355x_embedding(const int32_t *ids, int64_t ids_sb, int64_t ids_st, const float *tok,
                               const float *pos, float *out, int64_t out_sb, int64_t out_st, int64_t batch,
                               int64_t T, int64_t d_model, int64_t vocab, int64_t pos_offset,
                               int32_t *err_flag, void *stream);

/* Y[M,N] = [ReLU](X[M,K] W[K,N] [+ bias]) [+ residual], X, Y and residual rows at strides ldx,
 * ldy, ldr (W contiguous). The decoder's projections: the residual add of a transformer block is
 * fused into the epilogue (residual may equal Y). Generalises dense_layer_kernel
 * (examples/nn_kernels.py:23-74) to strided rows and the residual; bias and residual may be
 * NULL. */
PITON_API int32_t piton_mi355x_linear(const float *x, int64_t ldx, const float *w, const float *bias,
                            const float *residual, int64_t ldr, float *y, int64_t ldy, int64_t M,
                            int64_t N, int64_t K, int32_t relu, void *stream);

/* The digits MLP chain (examples/digits_model.py:120-139: three dense_layer_kernel launches of
 * examples/nn_kernels.py:23-74 with ReLU on the hidden layers, then numpy's argmax of the
 * first n_classes logits) in one launch: x [M, k0] row-major, w_l [K_l, N_l] row-major, biases
 * nullable; logits [M, n3] and pred (the predictions) nullable. The digits network (64 -> 128
 * -> 64 -> 10 or 16, x 16-byte aligned) runs on 16-row tiles in another k order than the dense
 * GEMM's: its logits are within the float32 error bound of the chain, not the dense launches'
 * bits. Other sizes: logits bit-identical to the three piton_mi355x_dense launches. Layer sizes
 * even and <= 256 (n3 <= 256, any parity), else PITON_EUNSUPPORTED. No reference counterpart:
 * one launch for the chain the reference runs as three. */
PITON_API int32_t piton_mi355x_mlp3(const float *x, int64_t M, const float *w1, const float *b1,
                          const float *w2, const float *b2, const float *w3, const float *b3,
                          int64_t k0, int64_t n1, int64_t n2, int64_t n3, float *logits,
                          int32_t *pred, int32_t n_classes, void *stream);

/* piton_mi355x_linear of layer-normalised rows: Y = LN(X) W (+ bias) (ReLU) (+ R), where
 * LN(x) = (x - mean) / sqrt(var + eps) over each row's K columns with the statistics of
 * piton_mi355x_layernorm (the layernorm_kernel of tests/test_reroll_reduce.py:199-208), so the
 * result equals layernorm followed by linear bit for bit. No reference counterpart: it serves
 * the decoder's per-token steps (one launch instead of two). Needs M <= 64, K % 256 == 0 and
 * 16-byte-aligned X rows; anything else returns PITON_EUNSUPPORTED. */
PITON_API int32_t piton_mi355x_linear_ln(const float *x, int64_t ldx, float eps, const float *w,
                               const float *bias, const float *residual, int64_t ldr, float *y,
                               int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t relu,
                               void *stream);

/* attn_fwd_kernel (examples/attention.py:67-113) over batch x n_heads heads: grid row y is
 * head y % n_heads of batch y / n_heads, whose Q / K / V / Out start at b*stride_?b + h*stride_?h.
 * piton_mi355x_attn_fwd is the batch = 1 case. */
PITON_API int32_t piton_mi355x_attn_fwd_batched(const float *q, const float *k, const float *v, float *out,
                                      float sm_scale, int64_t stride_qb, int64_t stride_qh,
                                      int64_t stride_qm, int64_t stride_kb, int64_t stride_kh,
                                      int64_t stride_kn, int64_t stride_kk, int64_t stride_vb,
                                      int64_t stride_vh, int64_t stride_vn, int64_t stride_ob,
                                      int64_t stride_oh, int64_t stride_om, int64_t n_ctx, int64_t batch,
                                      int64_t n_heads, int32_t head_dim, int32_t causal, void *stream);

/* One new query per (batch, head) attending to keys 0 .. n_keys-1 of a K/V cache: the decode
 * step of a KV-cached decoder, equal to the last query row of attn_fwd with causal masking over
 * n_keys keys. Rows of q, k, v, out are contiguous along head_dim; n_keys <= 8192. No reference
 * counterpart (the reference has no decoder). */
PITON_API int32_t piton_mi355x_attn_decode(const float *q, const float *k, const float *v, float *out,
                                 float sm_scale, int64_t stride_qb, int64_t stride_qh, int64_t stride_kb,
                                 int64_t stride_kh, int64_t stride_kn, int64_t stride_vb,
                                 int64_t stride_vh, int64_t stride_vn, int64_t stride_ob,
                                 int64_t stride_oh, int64_t n_keys, int64_t batch, int64_t n_heads,
                                 int32_t head_dim, void *stream);

/* A decode step of one decoder layer in one launch: for each sequence b < batch, the new row
 * LN(x[b]) W + bias (LN as in piton_mi355x_linear_ln, W [d_model, 3 d_model] row-major, bias
 * nullable) is written to cache row (n_keys - 1) * batch + b (q | k | v, each d_model wide, row
 * stride ldc), and out[b, h*64 .. h*64+63] gets head h's attention of that q over the keys
 * 0 .. n_keys-1 of the position-major cache (row t * batch + b: k at column d_model + h*64, v at
 * 2 d_model + h*64). Equal to piton_mi355x_linear_ln followed by piton_mi355x_attn_decode to
 * rounding. With ids (nullable; the first layer of a step) x[b] is first set to
 * tok[ids[b]] + pos (tok [vocab, d_model], pos one row of d_model), as piton_mi355x_embedding
 * does: an id outside [0, vocab) gives a NaN row and *err = 1 (err nullable). Needs head_dim 64,
 * d_model = n_heads * 64 a multiple of 256 up to 1024, n_keys <= 256, x, W, the cache, tok and
 * pos 16-byte aligned with ldx % 4 == 0 and ldc % 4 == 0; otherwise PITON_EUNSUPPORTED. No
 * reference counterpart (the reference has no decoder): it serves the decoder's per-token steps. */
PITON_API int32_t piton_mi355x_decode_layer(float *x, int64_t ldx, float eps, const float *w, const float *bias,
                                            float *cache, int64_t ldc, float *out, int64_t ldo, float sm_scale,
                                            int64_t n_keys, int64_t batch, int64_t n_heads, int32_t head_dim,
                                            int64_t d_model, const int32_t *ids, const float *tok,
                                            const float *pos, int64_t vocab, int32_t *err, void *stream);

/* The decoder's last step in one launch, one workgroup per row m < M: logits[m] = LN(x[m]) W
 * (+ bias), LN as in piton_mi355x_linear_ln, W [K, N] row-major, bias and logits nullable, and
 * next[m] = the first index of the largest of the first n_classes logits (numpy's argmax: a NaN
 * wins). Equal to piton_mi355x_linear_ln followed by piton_mi355x_argmax_rows to rounding. Needs
 * K a multiple of 256 and N a multiple of 4, both up to 1024, x rows and W 16-byte aligned;
 * otherwise PITON_EUNSUPPORTED. No reference counterpart: it serves the decoder's greedy step
 * (the reference has no decoder; its argmax rule is the digits driver's,
 * examples/digits_model.py:139). */
PITON_API int32_t piton_mi355x_lm_head_argmax(const float *x, int64_t ldx, float eps, const float *w,
                                              const float *bias, float *logits, int64_t ldl, int32_t *next,
                                              int64_t M, int64_t N, int64_t K, int32_t n_classes, void *stream);

/* ---- the perf suite's primitives (perf/suite.py:323-351): elementwise over n elements ---- */

/* out = x. Replaces copy_kernel (examples/primitive_kernels.py:12-17). */
PITON_API int32_t piton_mi355x_copy(const float *x, float *out, int64_t n, void *stream);

/* out = x * y. Replaces mul_kernel (examples/elementwise.py:5-9). */
PITON_API int32_t piton_mi355x_mul(const float *x, const float *y, float *out, int64_t n, void *stream);

/* out = x * alpha + y. Replaces fma_kernel (examples/primitive_kernels.py:20-27). */
PITON_API int32_t piton_mi355x_fma(const float *x, const float *y, float *out, int64_t n, float alpha,
                                   void *stream);

/* out = x > 0 ? x * alpha : 0. Replaces scaled_relu_kernel (examples/kernels.py:79-85). */
PITON_API int32_t piton_mi355x_scaled_relu(const float *x, float *out, int64_t n, float alpha, void *stream);

/* out = f(x) for OP 0 exp2, 1 log2, 2 1/x, 3 1/sqrt, 4 exp, 5 sqrt. Replaces sfu_kernel
 * (examples/sfu_tests.py:5-22). */
PITON_API int32_t piton_mi355x_sfu(const float *x, float *out, int64_t n, int32_t op, void *stream);

/* out = ln(x). Replaces log_kernel (examples/primitive_kernels.py:70-76). */
PITON_API int32_t piton_mi355x_log(const float *x, float *out, int64_t n, void *stream);

/* q = x / y and r = x % y on int32, truncating toward zero as C does (y = 0 gives an unspecified
 * value, no trap). Replaces idiv_kernel (examples/primitive_kernels.py:30-38). */
PITON_API int32_t piton_mi355x_idiv(const int32_t *x, const int32_t *y, int32_t *q, int32_t *r, int64_t n,
                                    void *stream);

/* out[r] = sum (or max, starting from -FLT_MAX) of x[r, 0:n_cols], rows of stride `stride`.
 * Replace row_sum_kernel (examples/kernels.py:88-96) and row_max_kernel
 * (examples/primitive_kernels.py:41-50). */
PITON_API int32_t piton_mi355x_row_sum(const float *x, float *out, int64_t rows, int64_t n_cols, int64_t stride,
                                       void *stream);
PITON_API int32_t piton_mi355x_row_max(const float *x, float *out, int64_t rows, int64_t n_cols, int64_t stride,
                                       void *stream);

/* out[c, r] = x[r, c] for r < n_rows, c < n_cols. Replaces transpose_kernel
 * (examples/primitive_kernels.py:53-67). */
PITON_API int32_t piton_mi355x_transpose(const float *x, float *out, int64_t n_rows, int64_t n_cols,
                                         int64_t stride_x, int64_t stride_out, void *stream);

/* ---- diagnostics ---- */

/* The sustained fp32 MFMA rate, measured: `workgroups` workgroups of four waves each issue
 * iters x 32 v_mfma_f32_32x32x2_f32 (4096 flops each) in two independent chains; the caller
 * times the launch on `stream`. out holds workgroups x 256 floats (written, meaningless). No
 * counterpart in the reference: it measures the MFMA roofline of the device at hand beside the
 * published peak, which assumes the 2.4 GHz peak engine clock. */
PITON_API int32_t piton_mi355x_mfma_probe(float *out, int64_t workgroups, int32_t iters, void *stream);

#ifdef __cplusplus
}
#endif

#endif
