/*
 * TEST INFRASTRUCTURE ONLY: the oracle. A CPU restatement, in the emulator's operation
 * order and with its round-toward-zero arithmetic (qpu_float.h), of the reference kernels on
 * the hot path. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load the
 * library built from this file; the product library never links or calls it.
 *
 * Each function cites the reference lines it follows. Arrays are float32 bit patterns
 * (uint32_t) in row-major storage with explicit element strides where the reference kernel
 * takes runtime strides.
 */
#include <fenv.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#if defined(__SSE__)
#include <xmmintrin.h>
#endif
#ifdef _OPENMP
#include <omp.h>
#endif

#include "qpu_float.h"

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------------------------
 * Math sequences (piton/backend/lower.py, issue mode, the compiler default: compiler.py:503)
 * ---------------------------------------------------------------------------------------- */

/* _exp_core, lower.py:2716-2790, issue variant: 2^x (base2) or e^x. */
static uint32_t q_exp_core(uint32_t x, int base2) {
    uint32_t xc = q_fmax(x, q_fk(base2 ? -150.0 : -104.0));
    uint32_t y = base2 ? xc : q_fmul(xc, q_fk(1.4426950408889634));
    uint32_t half = (y & Q_SIGN) | 0x3F000000u; /* +-0.5 with the sign of y */
    uint32_t t = q_fadd(y, half);
    uint32_t n = q_ftoi(t); /* round half away from zero */
    uint32_t nf = q_itof(n);
    uint32_t r;
    if (base2) {
        r = q_fsub(xc, nf);
        r = q_fmul(r, q_fk(0.6931471805599453));
    } else {
        uint32_t t1 = q_fmul(nf, q_fk(0.693145751953125)); /* ln2, high part */
        uint32_t t2 = q_fsub(xc, t1);
        t1 = q_fmul(nf, q_fk(1.428606765330187e-06)); /* ln2, low part */
        r = q_fsub(t2, t1);
    }
    static const double coef[5] = {1.0 / 120, 1.0 / 24, 1.0 / 6, 0.5, 1.0};
    uint32_t p = q_fmul(r, q_fk(1.0 / 720));
    for (int i = 0; i < 5; i++) {
        uint32_t q = q_fadd(p, q_fk(coef[i]));
        p = q_fmul(q, r);
    }
    uint32_t q = q_fadd(p, q_fk(1.0));
    /* q * 2^n with n clamped to [-127, 127], built in the exponent field */
    int32_t ni = (int32_t)n;
    int32_t nc = ni < -127 ? -127 : ni;
    nc = nc > 127 ? 127 : nc;
    uint32_t c = (uint32_t)(ni - nc) << 23;
    uint32_t q2 = q + c;
    uint32_t scale = (uint32_t)(nc + 127) << 23;
    uint32_t d = q_fmul(q2, scale);
    if (base2) {
        if (!q_negative(q_fsub(x, q_fk(128.0)))) d = Q_INF;
    } else {
        if (q_negative(q_fsub(0x42B17217u, x))) d = Q_INF;
    }
    return q_keep_nan(d, x);
}

/* recip_core, lower.py:657-669: integer seed, three Newton steps. */
static uint32_t q_recip_core(uint32_t b) {
    uint32_t r = 0x7EF311C3u - b;
    for (int k = 0; k < 3; k++) {
        uint32_t t = q_fmul(b, r);
        uint32_t e = q_fsub(q_fk(2.0), t);
        r = q_fmul(r, e);
    }
    return r;
}

/* recip, lower.py:633-655 (non-constant b). */
static uint32_t q_recip(uint32_t b) {
    uint32_t r = q_recip_core(b);
    uint32_t eb = b & 0x7F800000u, sg = b & Q_SIGN;
    if (!q_negative(eb - 0x7E800000u)) r = sg;  /* |b| >= 2^126, inf: +-0 */
    if (eb == 0u) r = sg | 0x7F800000u;        /* +-0 and denormals: +-inf */
    return q_keep_nan(r, b);
}

/* fdiv, lower.py:671-699: a * recip(b), then NaN for NaN operands, 0/0 and inf/inf. */
static uint32_t q_fdiv(uint32_t a, uint32_t b) {
    uint32_t d = q_fmul(a, q_recip(b));
    uint32_t ma = a & 0x7FFFFFFFu, mb = b & 0x7FFFFFFFu;
    uint32_t t = (int32_t)ma > (int32_t)mb ? ma : mb;
    if (!q_negative(t - 0x7F800001u)) d = Q_NAN;
    if (q_negative((ma | mb) - 0x00800000u)) d = Q_NAN;
    if (!q_negative((ma & mb) - 0x7F800000u)) d = Q_NAN;
    return d;
}

/* fdiv_uniform, lower.py:736-764: the same bits as fdiv for a divisor shared by all lanes. */
static uint32_t q_fdiv_uniform(uint32_t a, uint32_t b) {
    uint32_t d = q_fmul(a, q_recip(b));
    uint32_t mb = b & 0x7FFFFFFFu;
    uint32_t hi = 0x7F800001u, lo = 0u;
    if (mb == 0x7F800000u) hi = 0x7F800000u;
    if (!q_negative(mb - 0x7F800001u)) hi = 0u;
    if (q_negative(mb - 0x00800000u)) lo = 0x00800000u;
    uint32_t ma = a & 0x7FFFFFFFu;
    if (!q_negative(ma - hi)) d = Q_NAN;
    if (q_negative(ma - lo)) d = Q_NAN;
    return d;
}

/* rsqrt_core, lower.py:766-795, issue variant: scaled Newton steps, c = 1, 2, 16, 8192. */
static uint32_t q_rsqrt_core(uint32_t x) {
    uint32_t r = 0x5F375A86u - (x >> 1);
    double c = 1.0;
    for (int i = 0; i < 3; i++) {
        uint32_t t1 = q_fmul(x, r);
        uint32_t t2 = q_fmul(t1, r);
        uint32_t u = q_fsub(q_fk(3.0 * c * c), t2);
        r = q_fmul(r, u);
        c = 2.0 * c * c * c;
    }
    return q_fmul(r, q_fk(1.0 / c));
}

/* op_math_sqrt, lower.py:2921-2939. */
static uint32_t q_sqrt(uint32_t x) {
    uint32_t d = q_fmul(x, q_rsqrt_core(x));
    uint32_t eb = x & 0x7F800000u;
    if (eb == 0x7F800000u) d = x;   /* inf, NaN */
    if (x >> 31) d = Q_NAN;         /* x < 0 */
    if (eb == 0u) d = x & Q_SIGN;   /* +-0 and denormals */
    return d;
}

/* op_math_rsqrt, lower.py:2899-2919. */
static uint32_t q_rsqrt(uint32_t x) {
    uint32_t d = q_rsqrt_core(x);
    uint32_t eb = x & 0x7F800000u;
    if (eb == 0x7F800000u) d = 0u;
    if (x >> 31) d = Q_NAN;
    if (eb == 0u) d = (x & Q_SIGN) | 0x7F800000u;
    return q_keep_nan(d, x);
}

/* ------------------------------------------------------------------------------------------
 * Reductions (lower.py:3911-3988, 4043-4063; reroll.py:45-55)
 * ---------------------------------------------------------------------------------------- */

typedef uint32_t (*q_binop)(uint32_t, uint32_t);

/* 16-lane butterfly: v[i] = op(v[i], v[i - s]) for s = 8, 4, 2, 1; lane 0 is the result. */
static uint32_t q_lane_reduce(uint32_t *lane, q_binop op) {
    uint32_t nxt[16];
    for (int s = 8; s >= 1; s >>= 1) {
        for (int i = 0; i < 16; i++) nxt[i] = op(lane[i], lane[(i - s + 16) & 15]);
        memcpy(lane, nxt, sizeof nxt);
    }
    return lane[0];
}

/* A row of L elements (element f in lane f % 16 of register f / 16). L >= 16 and a multiple
 * of 16: lanes fold their registers first to last, then the butterfly. L < 16 (a single
 * register): lanes >= L take `pad`, then the butterfly. */
static uint32_t q_row_reduce(const uint32_t *x, int L, q_binop op, uint32_t pad) {
    uint32_t lane[16];
    if (L < 16) {
        for (int l = 0; l < 16; l++) lane[l] = l < L ? x[l] : pad;
    } else {
        int nb = L / 16;
        for (int l = 0; l < 16; l++) {
            uint32_t cur = x[l];
            for (int j = 1; j < nb; j++) cur = op(cur, x[16 * j + l]);
            lane[l] = cur;
        }
    }
    return q_lane_reduce(lane, op);
}

/* ------------------------------------------------------------------------------------------
 * Elementwise entry points (vectorised over n values), for the tests' known answers
 * ---------------------------------------------------------------------------------------- */

EXPORT void oracle_fadd(const uint32_t *a, const uint32_t *b, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fadd(a[i], b[i]);
}
EXPORT void oracle_fsub(const uint32_t *a, const uint32_t *b, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fsub(a[i], b[i]);
}
EXPORT void oracle_fmul(const uint32_t *a, const uint32_t *b, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fmul(a[i], b[i]);
}
EXPORT void oracle_fmax(const uint32_t *a, const uint32_t *b, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fmax(a[i], b[i]);
}
EXPORT void oracle_fmin(const uint32_t *a, const uint32_t *b, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fmin(a[i], b[i]);
}
EXPORT void oracle_ftoi(const uint32_t *a, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_ftoi(a[i]);
}
EXPORT void oracle_itof(const uint32_t *a, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_itof(a[i]);
}
EXPORT void oracle_exp(const uint32_t *a, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_exp_core(a[i], 0);
}
EXPORT void oracle_exp2(const uint32_t *a, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_exp_core(a[i], 1);
}
EXPORT void oracle_recip(const uint32_t *a, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_recip(a[i]);
}
EXPORT void oracle_fdiv(const uint32_t *a, const uint32_t *b, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fdiv(a[i], b[i]);
}
EXPORT void oracle_fdiv_uniform(const uint32_t *a, const uint32_t *b, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fdiv_uniform(a[i], b[i]);
}
EXPORT void oracle_rsqrt(const uint32_t *a, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_rsqrt(a[i]);
}
EXPORT void oracle_sqrt(const uint32_t *a, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_sqrt(a[i]);
}

/* Row reductions of `rows` rows of L elements (row stride ld): kind 0 = sum, 1 = max. */
EXPORT void oracle_row_reduce(const uint32_t *x, int64_t rows, int64_t ld, int32_t L, int32_t kind,
                              uint32_t *out) {
    for (int64_t r = 0; r < rows; r++)
        out[r] = kind ? q_row_reduce(x + r * ld, L, q_fmax, 0xFFFFFFFFu)
                      : q_row_reduce(x + r * ld, L, q_fadd, 0u);
}

/* ------------------------------------------------------------------------------------------
 * Kernels
 * ---------------------------------------------------------------------------------------- */

/* matmul_kernel (examples/kernels.py:18-57) with tl.dot's order (lower.py:3761-3877): for
 * every stored C[m, n], acc = +0 and, for k ascending, acc = fadd(acc, fmul(a[m,k], b[k,n])).
 * K-masked lanes load 0 and add +0, which changes nothing, and the tile shape does not change
 * any element's order, so the result is this closed form. Rows [row0, row1) only. */
EXPORT void oracle_matmul(const uint32_t *a, const uint32_t *b, uint32_t *c, int64_t M, int64_t N,
                          int64_t K, int64_t s_am, int64_t s_ak, int64_t s_bk, int64_t s_bn,
                          int64_t s_cm, int64_t s_cn, int64_t row0, int64_t row1) {
    (void)M;
    for (int64_t m = row0; m < row1; m++)
        for (int64_t n = 0; n < N; n++) {
            uint32_t acc = 0u;
            for (int64_t k = 0; k < K; k++)
                acc = q_fadd(acc, q_fmul(a[m * s_am + k * s_ak], b[k * s_bk + n * s_bn]));
            c[m * s_cm + n * s_cn] = acc;
        }
}

/* The same closed form computed with the host FPU in round-toward-zero mode with flush-to-zero
 * and denormals-are-zero, vectorised over n. It equals oracle_matmul bit for bit when every
 * input is finite and no partial sum reaches 2^127 (the only differences of the FPU's mode
 * from the QPU's rules are the sign of zero results, fixed at the end, and overflow to
 * FLT_MAX instead of inf). Contiguous row-major A [M,K] and B [K,N]; rows [row0, row1). */
EXPORT void oracle_matmul_fast(const float *a, const float *b, float *c, int64_t N, int64_t K,
                               int64_t row0, int64_t row1, int32_t threads) {
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
    {
        int old_round = fegetround();
        fesetround(FE_TOWARDZERO);
#if defined(__SSE__)
        unsigned int old_csr = _mm_getcsr();
        _mm_setcsr(old_csr | 0x8040u); /* FTZ | DAZ */
#endif
        float *acc = (float *)aligned_alloc(64, (size_t)((N + 15) / 16 * 16) * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t m = row0; m < row1; m++) {
            for (int64_t n = 0; n < N; n++) acc[n] = 0.0f;
            const float *arow = a + m * K;
            for (int64_t k = 0; k < K; k++) {
                const float av = arow[k];
                const float *brow = b + k * N;
                for (int64_t n = 0; n < N; n++) {
                    float p = av * brow[n];
                    acc[n] = acc[n] + p;
                }
            }
            float *crow = c + m * N;
            for (int64_t n = 0; n < N; n++) crow[n] = acc[n] + 0.0f; /* -0 -> +0 in RTZ */
        }
        free(acc);
#if defined(__SSE__)
        _mm_setcsr(old_csr);
#endif
        fesetround(old_round);
    }
}

/* dense_layer_kernel (examples/nn_kernels.py:23-74): the dot chain as above, then
 * acc = fadd(acc, bias[n]) after the whole K chain (:64-66), then ReLU = fmax(acc, +0)
 * (:67-68; lower.py:529-535). X [M,K], W [K,N], Y [M,N] contiguous. */
EXPORT void oracle_dense(const uint32_t *x, const uint32_t *w, const uint32_t *bias, uint32_t *y,
                         int64_t M, int64_t N, int64_t K, int32_t add_bias, int32_t relu) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            uint32_t acc = 0u;
            for (int64_t k = 0; k < K; k++) acc = q_fadd(acc, q_fmul(x[m * K + k], w[k * N + n]));
            if (add_bias) acc = q_fadd(acc, bias[n]);
            if (relu) acc = q_fmax(acc, 0u);
            y[m * N + n] = acc;
        }
}

/* softmax_kernel (examples/kernels.py:60-76): BLOCK_SIZE columns loaded with -inf past
 * n_cols (:66-69); m = tl.max (row reduction); e = exp(fsub(x, m)); s = tl.sum(e);
 * out = fdiv_uniform(e, s) (lower.py:701-709, 736-764); columns < min(n_cols, BLOCK_SIZE)
 * stored (:74-76). */
EXPORT void oracle_softmax(uint32_t *out, const uint32_t *in, int64_t in_row_stride,
                           int64_t out_row_stride, int64_t n_cols, int64_t n_rows, int32_t block) {
    uint32_t *x = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)block);
    uint32_t *e = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)block);
    for (int64_t r = 0; r < n_rows; r++) {
        const uint32_t *row = in + r * in_row_stride;
        for (int32_t i = 0; i < block; i++) x[i] = i < n_cols ? row[i] : 0xFF800000u;
        uint32_t m = q_row_reduce(x, block, q_fmax, 0xFFFFFFFFu);
        for (int32_t i = 0; i < block; i++) e[i] = q_exp_core(q_fsub(x[i], m), 0);
        uint32_t s = q_row_reduce(e, block, q_fadd, 0u);
        uint32_t *orow = out + r * out_row_stride;
        for (int32_t i = 0; i < block && i < n_cols; i++) orow[i] = q_fdiv_uniform(e[i], s);
    }
    free(x);
    free(e);
}

/* attn_fwd_kernel + _attn_fwd_inner (examples/attention.py:33-113), one query row at a time
 * (every operation of the kernel is row-wise). Keys are visited in aligned blocks of BLOCK_N
 * up to the program's bound; a block whose keys are all masked for this row leaves the row's
 * state bit-identical (alpha = exp2(+0) = 1, p = +0), so BLOCK_M does not change results.
 * Q, V, Out [H, N, D] through (stride_h, row stride, 1); K through (stride_kh, stride_kn,
 * stride_kk). Rows [q0, q1) of every head. */
EXPORT void oracle_attention(const uint32_t *Q, const uint32_t *Kp, const uint32_t *V, uint32_t *Out,
                             uint32_t sm_scale, int64_t s_qh, int64_t s_qm, int64_t s_kh,
                             int64_t s_kn, int64_t s_kk, int64_t s_vh, int64_t s_vn, int64_t s_oh,
                             int64_t s_om, int64_t n_ctx, int64_t heads, int32_t head_dim,
                             int32_t block_n, int32_t causal, int64_t q0, int64_t q1) {
    const uint32_t NEG_INF = 0xFF800000u;
    uint32_t qk_scale = q_fmul(sm_scale, q_fk(1.44269504)); /* runtime multiply (:87) */
    uint32_t *qk = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)block_n);
    uint32_t *p = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)block_n);
    uint32_t *acc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)head_dim);
    int64_t n_full = n_ctx / block_n * block_n;
    for (int64_t h = 0; h < heads; h++)
        for (int64_t m = q0; m < q1 && m < n_ctx; m++) {
            const uint32_t *q = Q + h * s_qh + m * s_qm;
            /* keys this row's program visits: causal -> up to hi = min((start_m+1)*BM, N) rounded
             * up to a block; every block past row m is a no-op for the row, so stopping at the
             * block holding key m gives the same bits. Non-causal -> all of N_CTX. */
            int64_t last = causal ? m + 1 : n_ctx;
            uint32_t m_i = NEG_INF, l_i = 0u;
            for (int d = 0; d < head_dim; d++) acc[d] = 0u;
            for (int64_t start = 0; start < last; start += block_n) {
                int mask_keys = causal ? 1 : (start >= n_full);
                for (int j = 0; j < block_n; j++) {
                    int64_t n = start + j;
                    uint32_t s = 0u;
                    int valid_load = n < n_ctx;
                    for (int d = 0; d < head_dim; d++) {
                        uint32_t kv = valid_load ? Kp[h * s_kh + n * s_kn + d * s_kk] : 0u;
                        s = q_fadd(s, q_fmul(q[d], kv));
                    }
                    s = q_fmul(s, qk_scale);
                    if (mask_keys && n >= n_ctx) s = NEG_INF;
                    if (causal && m < n) s = NEG_INF;
                    qk[j] = s;
                }
                uint32_t m_ij = q_fmax(m_i, q_row_reduce(qk, block_n, q_fmax, 0xFFFFFFFFu));
                for (int j = 0; j < block_n; j++) p[j] = q_exp_core(q_fsub(qk[j], m_ij), 1);
                uint32_t alpha = q_exp_core(q_fsub(m_i, m_ij), 1);
                l_i = q_fadd(q_fmul(l_i, alpha), q_row_reduce(p, block_n, q_fadd, 0u));
                for (int d = 0; d < head_dim; d++) {
                    uint32_t a = q_fmul(acc[d], alpha);
                    for (int j = 0; j < block_n; j++) {
                        int64_t n = start + j;
                        uint32_t vv = n < n_ctx ? V[h * s_vh + n * s_vn + d] : 0u;
                        a = q_fadd(a, q_fmul(p[j], vv));
                    }
                    acc[d] = a;
                }
                m_i = m_ij;
            }
            uint32_t *o = Out + h * s_oh + m * s_om;
            for (int d = 0; d < head_dim; d++) o[d] = q_fdiv(acc[d], l_i);
        }
    free(qk);
    free(p);
    free(acc);
}

/* layernorm_kernel (tests/test_reroll_reduce.py:199-208): x masked with 0 past n;
 * mean = fdiv(sum(x), itof(n)); d = where(mask, fsub(x, mean), 0); var = fdiv(sum(d*d), itof(n));
 * out = fdiv_uniform(d, sqrt(fadd(var, eps))). Rows of `block` elements at row stride ld. */
EXPORT void oracle_layernorm(const uint32_t *xin, uint32_t *out, int64_t n, uint32_t eps,
                             int64_t rows, int64_t ld, int32_t block) {
    uint32_t *x = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)block);
    uint32_t *d = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)block);
    uint32_t *dd = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)block);
    uint32_t nf = q_itof((uint32_t)(int32_t)n);
    for (int64_t r = 0; r < rows; r++) {
        for (int32_t i = 0; i < block; i++) x[i] = i < n ? xin[r * ld + i] : 0u;
        uint32_t mean = q_fdiv(q_row_reduce(x, block, q_fadd, 0u), nf);
        for (int32_t i = 0; i < block; i++) {
            d[i] = i < n ? q_fsub(x[i], mean) : 0u;
            dd[i] = q_fmul(d[i], d[i]);
        }
        uint32_t var = q_fdiv(q_row_reduce(dd, block, q_fadd, 0u), nf);
        uint32_t sd = q_sqrt(q_fadd(var, eps));
        for (int32_t i = 0; i < block && i < n; i++) out[r * ld + i] = q_fdiv_uniform(d[i], sd);
    }
    free(x);
    free(d);
    free(dd);
}

/* add_kernel (examples/kernels.py:6-15): out = fadd(x, y) for i < n. */
EXPORT void oracle_add(const uint32_t *x, const uint32_t *y, uint32_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = q_fadd(x[i], y[i]);
}

/* First index of the largest value over the first n of each row, the rule of numpy's argmax
 * (examples/digits_model.py:137-139) and the firmware's strict '>' scan
 * (pi/examples/digits/main.c:140-145); a NaN wins at its first position, as in numpy. */
EXPORT void oracle_argmax_rows(const float *x, int64_t rows, int64_t ld, int32_t n, int32_t *out) {
    for (int64_t r = 0; r < rows; r++) {
        const float *row = x + r * ld;
        int32_t best = 0;
        float bv = row[0];
        if (bv == bv) {
            for (int32_t i = 1; i < n; i++) {
                float v = row[i];
                if (v != v) { best = i; break; }
                if (v > bv) { bv = v; best = i; }
            }
        }
        out[r] = best;
    }
}

EXPORT int32_t oracle_abi_version(void) { return 1; }
