/*
 * TEST INFRASTRUCTURE ONLY. This header belongs to the oracle: a CPU restatement of the
 * reference's own arithmetic, used by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker. Nothing in the product library includes it.
 *
 * Scalar float semantics of the VideoCore IV QPU as the reference emulator models them
 * (piton/qpu/emulator.py:139-235):
 *   - an operand is read as float64 after two rules: a denormal reads as +0 and an
 *     exponent-255 value (inf or NaN) reads as the infinity of its sign (_qpu_in, :173-178);
 *   - fadd / fsub / fmul / itof keep the exact result truncated toward zero; an exact
 *     |result| >= 2^128 is +-inf, |truncated| < 2^-126 is +0, so every zero result is +0
 *     (_rtz, :155-170);
 *   - 0 * inf = +0 (:193-198) and inf + (-inf) = the second operand (:181-190);
 *   - fmin / fmax order operands by their sign-magnitude bits and return an operand
 *     unchanged (_fkey :201-205, alu_add :222-225);
 *   - ftoi truncates and keeps the low 32 bits; exponents 0 or >= 127+55 give 0 (:208-212).
 * Float constants that the compiler folds are rounded to nearest (piton/passes.py:152-157,
 * piton/backend/lower.py:4884-4891): q_fk below.
 *
 * Values travel as uint32_t bit patterns so that NaN payloads and signed zeros survive.
 */
#ifndef PITON_ORACLE_QPU_FLOAT_H
#define PITON_ORACLE_QPU_FLOAT_H

#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float q_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t q_u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

#define Q_NAN 0x7FC00000u
#define Q_INF 0x7F800000u
#define Q_SIGN 0x80000000u

/* An integer ALU result's N flag: bit 31 (emulator.py:903-907). */
static inline int q_negative(uint32_t v) { return (v >> 31) != 0; }

/* Operand as the float ALUs read it (_qpu_in). */
static inline double q_in(uint32_t x) {
    uint32_t e = (x >> 23) & 0xFFu;
    if (e == 255u) return (x >> 31) ? -INFINITY : INFINITY;
    if (e == 0u && (x & 0x7FFFFFu)) return 0.0;
    return (double)q_f(x);
}

/* exact (+ err, the part TwoSum lost) truncated toward zero, with the overflow and flush
 * rules (_rtz). */
static inline uint32_t q_rtz(double exact, double err) {
    float rn = (float)exact;
    float out = rn;
    if (isfinite(exact) && fabs((double)rn) > fabs(exact)) out = nextafterf(rn, 0.0f);
    if (err != 0.0 && (double)out == exact) {
        int se = (exact > 0) - (exact < 0);
        int sr = (err > 0) - (err < 0);
        if (se != sr) out = nextafterf(out, 0.0f);
    }
    if (fabs(exact) >= 0x1p128) out = (exact < 0) ? -INFINITY : INFINITY;
    if (fabsf(out) < 0x1p-126f) out = 0.0f;
    return q_u(out);
}

static inline uint32_t q_fadd(uint32_t a, uint32_t b) {
    double fa = q_in(a), fb = q_in(b);
    if (isinf(fb)) return q_u((float)fb);
    if (isinf(fa)) return q_u((float)fa);
    double s = fa + fb;
    double bb = s - fa;
    double err = (fa - (s - bb)) + (fb - bb);
    return q_rtz(s, err);
}

static inline uint32_t q_fsub(uint32_t a, uint32_t b) { return q_fadd(a, b ^ Q_SIGN); }

static inline uint32_t q_fmul(uint32_t a, uint32_t b) {
    double fa = q_in(a), fb = q_in(b);
    if ((fa == 0.0 && isinf(fb)) || (isinf(fa) && fb == 0.0)) return 0u;
    return q_rtz(fa * fb, 0.0); /* a product of two floats is exact in float64 */
}

static inline int64_t q_fkey(uint32_t x) {
    int64_t m = (int64_t)(x & 0x7FFFFFFFu);
    return ((x >> 31) && ((x >> 23) & 0xFFu)) ? -m : m;
}
static inline uint32_t q_fmax(uint32_t a, uint32_t b) { return q_fkey(a) > q_fkey(b) ? a : b; }
static inline uint32_t q_fmin(uint32_t a, uint32_t b) { return q_fkey(a) <= q_fkey(b) ? a : b; }

static inline uint32_t q_ftoi(uint32_t a) {
    uint32_t e = (a >> 23) & 0xFFu;
    double f = (e == 0u || e >= 127u + 55u) ? 0.0 : (double)q_f(a);
    int64_t t = (int64_t)trunc(f);
    return (uint32_t)((uint64_t)t & 0xFFFFFFFFu);
}

static inline uint32_t q_itof(uint32_t a) { return q_rtz((double)(int32_t)a, 0.0); }

/* A float constant as the compiler materialises it: float32 round-to-nearest. */
static inline uint32_t q_fk(double v) { return q_u((float)v); }

/* d = x where x is NaN (lower.py:2792-2797). */
static inline uint32_t q_keep_nan(uint32_t d, uint32_t x) {
    return q_negative((x & 0x7FFFFFFFu) - 0x7F800001u) ? d : x;
}

#endif
