// The KV-cached decoder's fused steps (piton_mi355x_decode_layer, piton_mi355x_lm_head_argmax).
// No reference counterpart: the reference has no decoder. The pieces it composes are the
// layernorm of tests/test_reroll_reduce.py:199-208, the dense layer of
// examples/nn_kernels.py:23-74, the attention of examples/attention.py:33-113 and the argmax of
// examples/digits_model.py:139.
//
// decode_layer: one decode step of a layer in one launch -- the layernorm of the new token's
// row, its QKV projection (written into the cache row of its position) and the single-query
// attention of every head over the cache. It equals piton_mi355x_linear_ln (QKV) followed by
// piton_mi355x_attn_decode on the decoder's position-major cache, to rounding: the projection
// here is a dot product per output instead of the matrix-core product.
// Design (gfx950): one 512-thread workgroup (8 waves) per (sequence b, head h), 1 per CU at the
// decoder's 64 x 4 heads:
//   * waves 6 and 7 copy the head's cached keys and values of the earlier positions memory ->
//     LDS by 16-byte LDS-DMA (no registers; rows past the last one read as zeros), so the cache
//     streams in while the projection runs;
//   * wave 0 normalises the row (float4 loads, mean and variance by wave reductions) into LDS;
//     the 384 threads of waves 0-5 compute the head's 3 x 64 projection outputs: thread
//     (slice s, column group c) owns 4 consecutive columns of q, k or v and the k range
//     [s K/8, (s+1) K/8), reading 16-byte weight vectors (64 consecutive columns of a weight row
//     per 16 threads) in chunks of 16 rows, the first two requested before the layernorm; the
//     eight slices add in slice order, then the bias;
//   * the vector-memory counter is in order per wave (a wave's wait for one load covers every
//     load it issued before), so the waves that copy the cache issue nothing else and the
//     projection waves no copies; loads are unconditional (a load under a condition compiles to
//     a branch whose join waits for it); and the barriers wait for LDS work only (__syncthreads
//     would also wait for the copies and for the cache-row store);
//   * the new q, k, v go to the cache row (t = n_keys - 1) and to LDS, and the attention runs
//     as attn_decode_short does: TPK = 4 lanes per key score 16 dims each (read from LDS in a
//     bank-conflict-free chunk order), the maximum and the sum of 2^(s - m) reduce over the
//     workgroup, thread (d, g) sums p_j V[j][d] over the keys j = g (mod 8) in key order, and
//     the eight partial sums add in order.
//
// lm_head_argmax: the decoder's last step, one 512-thread workgroup per row: the layernorm, the
// N logits of the head (wave w the k range [w K/8, (w+1) K/8), lane l the column groups l + 64 j,
// the slices added in order, then the bias) and numpy's argmax of the first n_classes, whose
// (value, index) combine is order-free.
#include "common.h"

namespace piton {

namespace {

constexpr int kDlD = 64;           // head_dim
constexpr int kDlKeys = 256;       // cache rows a launch attends to (the decoder's context)
constexpr int kDlMaxModel = 1024;  // d_model
constexpr int kDlThreads = 512, kDlWaves = kDlThreads / 64;

struct DecodeLayerArgs {
    float *x;  // the new rows, row b at x + b * ldx (written with ids)
    int64_t ldx;
    float eps;
    const float *w;     // [d_model, 3 d_model] row-major
    const float *bias;  // [3 d_model] or null
    float *cache;       // row t * batch + b: q | k | v, each d_model wide, stride ldc
    int64_t ldc;
    float *o;  // row b at o + b * ldo, head h at column h * 64
    int64_t ldo;
    float scale;  // sm_scale * log2(e)
    int n_keys, batch, n_heads, d_model;
    // with ids (the first layer of a step): x[b] = tok[ids[b]] + pos, written to x by the
    // workgroups of head 0; an id outside [0, vocab) gives a NaN row and *err = 1
    const int32_t *ids;
    const float *tok, *pos;
    int64_t vocab;
    int32_t *err;
    PhaseRecord *phase;  // the launch's phase-trace records (diagnostics builds; null otherwise)
};

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// A workgroup barrier for LDS data: this wave's LDS stores are done, then s_barrier. Unlike
// __syncthreads, whose release fence waits for every memory operation in flight, it lets the
// cache copies and the global stores (the cache row, which nothing here reads back) stay in
// flight. The empty asm with a memory clobber keeps the compiler from moving an LDS store below
// the barrier (the waitcnt and s_barrier builtins do not order memory); a release fence limited
// to LDS would do the same but also waits for the LDS-DMA cache copies in flight (vmcnt(0)).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitcntLgkm0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
}

// sum or max over the workgroup: DPP within each wave, then the eight wave results through
// `red` (eight floats of its own per call), combined in a fixed pairwise order
template <class Op>
__device__ __forceinline__ float wg_reduce(float v, Op op, float *red) {
    static_assert(kDlWaves == 8, "eight wave results");
    v = wave_reduce(v, op);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    return op(op(op(red[0], red[1]), op(red[2], red[3])), op(op(red[4], red[5]), op(red[6], red[7])));
}

// A row's layernorm (K % 256 == 0, K <= kDlMaxModel) by one wave: ln_row_load requests the
// row, lane l's chunks being columns 4 l + 256 i .. + 3 (unconditional loads; chunks past the row
// re-read its last one and are dropped when summed), and ln_row_store, once the caller has issued
// whatever it wants in flight meanwhile, computes the mean and variance by wave reductions and
// writes (x - mean) / sqrt(var + eps) to lnx, as 1 / sqrt once and a product per element.
constexpr int kLnChunks = kDlMaxModel / 256;
__device__ __forceinline__ void ln_row_load(const float *x, int K, int lane, f32x4 (&xv)[kLnChunks]) {
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(x);
    const int nx = K / 256;
#pragma unroll
    for (int i = 0; i < kLnChunks; i++) xv[i] = xr[min(lane + 64 * i, 64 * nx - 1)];
}
__device__ __forceinline__ void ln_row_store(const f32x4 (&xv)[kLnChunks], int K, float eps, int lane, float *lnx) {
    const int nx = K / 256;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kLnChunks; i++)
        if (i < nx) s += (xv[i][0] + xv[i][1]) + (xv[i][2] + xv[i][3]);
    const float mean = wave_reduce(s, SumOp()) / (float)K;
    float q2 = 0.f;
#pragma unroll
    for (int i = 0; i < kLnChunks; i++)
        if (i < nx)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float d = xv[i][e] - mean;
                q2 = fmaf(d, d, q2);
            }
    const float inv_sd = 1.0f / sqrtf(wave_reduce(q2, SumOp()) / (float)K + eps);
#pragma unroll
    for (int i = 0; i < kLnChunks; i++)
        if (i < nx) {
            f32x4 y;
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = (xv[i][e] - mean) * inv_sd;
            *reinterpret_cast<f32x4 *>(&lnx[4 * lane + 256 * i]) = y;
        }
}

// The embedding of token `id` at a position instead of a stored row (same chunks as ln_row_load):
// tok[id] + pos, a NaN row for an id outside [0, vocab). The loads are unconditional (an id
// outside the vocabulary reads row 0 and is replaced afterwards).
__device__ __forceinline__ void emb_row_load(const float *tok, const float *pos, int id, int64_t vocab, int K,
                                             int lane, f32x4 (&xv)[kLnChunks]) {
    const bool bad = id < 0 || id >= vocab;
    const f32x4 *tr = reinterpret_cast<const f32x4 *>(tok + (int64_t)(bad ? 0 : id) * K);
    const f32x4 *pr = reinterpret_cast<const f32x4 *>(pos);
    const int nx = K / 256;
#pragma unroll
    for (int i = 0; i < kLnChunks; i++) {
        const int c = min(lane + 64 * i, 64 * nx - 1);
        const f32x4 a = tr[c], p = pr[c];
#pragma unroll
        for (int e = 0; e < 4; e++) xv[i][e] = bad ? __int_as_float(0x7FC00000) : a[e] + p[e];
    }
}

// A thread's 4 columns of a row-vector x matrix product over a k range of kq rows (kq % 32 == 0):
// 16-byte weight vectors in chunks of kRpCh = 16 rows, two chunks in flight. The loads go
// through a buffer descriptor over the weights with the thread's column offset per lane and the
// row offset in the scalar operand (uniform), so 32 loads in flight hold no address registers.
// rp_first requests the first two chunks (the caller issues it early); rp_rest multiplies them
// and the remaining chunks by the activations a[0 .. kq) into acc.
constexpr int kRpCh = 16;
struct RowOperand {
    __amdgpu_buffer_rsrc_t r;  // the weights
    uint32_t col;              // byte offset of the thread's 4 columns in the range's first row
    uint32_t row;              // bytes per weight row
};
__device__ __forceinline__ void rp_load(f32x4 (&w)[kRpCh], const RowOperand &o, int k) {
#pragma unroll
    for (int i = 0; i < kRpCh; i++)
        w[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(o.r, (int)o.col, (int)((k + i) * o.row), 0));
}
__device__ __forceinline__ void rp_first(f32x4 (&wa)[kRpCh], f32x4 (&wb)[kRpCh], const RowOperand &o) {
    rp_load(wa, o, 0);
    rp_load(wb, o, kRpCh);
}
__device__ __forceinline__ void rp_mul(const f32x4 (&w)[kRpCh], const float *a, f32x4 &acc) {
#pragma unroll
    for (int i = 0; i < kRpCh; i++) {
        const float x = a[i];
#pragma unroll
        for (int e = 0; e < 4; e++) acc[e] = fmaf(x, w[i][e], acc[e]);
    }
}
__device__ __forceinline__ void rp_rest(f32x4 (&wa)[kRpCh], f32x4 (&wb)[kRpCh], const RowOperand &o, int kq,
                                        const float *a, f32x4 &acc) {
    // Every refill in the loop is unconditional and the last two chunks multiply after it: a
    // refill under a condition would keep the chunk it replaces live on the other path (three
    // sets of registers). The scheduling barriers keep each refill after the products that free
    // its registers.
    int k = 0;
    for (; k + 2 * kRpCh < kq; k += 2 * kRpCh) {
        rp_mul(wa, a + k, acc);
        __builtin_amdgcn_sched_barrier(0);
        rp_load(wa, o, k + 2 * kRpCh);
        rp_mul(wb, a + k + kRpCh, acc);
        __builtin_amdgcn_sched_barrier(0);
        rp_load(wb, o, k + 3 * kRpCh);
    }
    rp_mul(wa, a + k, acc);
    rp_mul(wb, a + k + kRpCh, acc);
}

__global__ __launch_bounds__(kDlThreads) void decode_layer_kernel(DecodeLayerArgs g) {
    constexpr int D = kDlD, TPK = D / 16, KPP = kDlThreads / TPK, KG = kDlThreads / D, NIT = kDlKeys / KPP;
    constexpr int NCG = 3 * D / 4;                       // projection column groups (48)
    constexpr int PT = NCG * kDlWaves;                    // projection threads (384: waves 0-5)
    static_assert(PT % 64 == 0 && PT / 64 <= kDlWaves - 2, "two waves left for the cache copies");
    __shared__ __attribute__((aligned(16))) float ks[kDlKeys][D];  // keys of the head (64 KB)
    __shared__ __attribute__((aligned(16))) float vs[kDlKeys][D];  // values (64 KB)
    __shared__ __attribute__((aligned(16))) float lnx[kDlMaxModel];
    __shared__ __attribute__((aligned(16))) float gp[kDlWaves][3 * D];  // projection partials per k slice
    __shared__ float qn[D];
    __shared__ float p[kDlKeys];
    __shared__ float red[4 * kDlWaves];
    __shared__ float part[kDlThreads];

    // the wave index is uniform (readfirstlane): its branches are scalar, and the copies' LDS
    // addresses need no per-lane loop
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int b = __builtin_amdgcn_readfirstlane(blockIdx.x / g.n_heads);
    const int h = __builtin_amdgcn_readfirstlane(blockIdx.x % g.n_heads);
    const int n_keys = g.n_keys, jn = n_keys - 1, Dm = g.d_model, K = Dm;
    const int64_t ldw = 3 * (int64_t)Dm;
    PITON_PHASE_VARS;
    PITON_PHASE(0);
    // output t < 192 of the projection (part t / 64: q, k, v; dim t % 64): its bias, requested
    // now and from a valid address for every thread (the weights stand in without a bias)
    const float *bias_p = g.bias ? g.bias : g.w;
    const int tb = min(t, 3 * D - 1);
    const float bias_raw = bias_p[(tb / D) * Dm + h * D + tb % D];

    // 1. waves 6 (keys) and 7 (values): the earlier positions' rows -> LDS. Lane l of a copy
    // carries 16 bytes of row 4 i + l / 16 (dims 4 (l % 16) ..); the descriptor ends at the last
    // earlier row, so the rows from jn on arrive as zeros. A wave holds at most 63 memory
    // operations in flight and stalls issuing the next, so the copies of groups past kPreGroups
    // are issued after the layernorm's barrier, which the stall would otherwise hold up.
    constexpr int kPreGroups = 56;
    const int groups = (jn + 3) / 4;
    const bool copier = wave >= kDlWaves - 2;
    auto copy_rows = [&](int i0, int i1) {
        const int64_t row_stride = (int64_t)g.batch * g.ldc;  // floats between positions
        const int which = wave - (kDlWaves - 2);              // 0: keys, 1: values
        float *base = g.cache + (int64_t)b * g.ldc + (1 + which) * Dm + h * D;
        float(*dst)[D] = which ? vs : ks;
        const uint32_t bytes = jn > 0 ? (uint32_t)(((int64_t)(jn - 1) * row_stride + D) * 4) : 0u;
        const auto r = __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
        for (int i = i0; i < i1; i++) {
            const uint32_t off = (uint32_t)(((int64_t)(4 * i + (lane >> 4)) * row_stride + 4 * (lane & 15)) * 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)&dst[4 * i][0], 16, off, 0, 0, 0);
        }
    };
    if (copier) copy_rows(0, min(groups, kPreGroups));

    // 2. wave 0: the layernorm of row b into LDS. 3. waves 0-5: the head's projection, thread
    // t < 384 = (slice t / 48, column group c = t % 48: the 4 columns 4 (c % 16) .. of part c / 16
    // of head h), its first chunks requested before the layernorm.
    const int cgi = t % NCG, slice = min(t / NCG, kDlWaves - 1);
    const int part_i = cgi / (D / 4), c4 = cgi % (D / 4);
    const int kq = K / kDlWaves;
    const RowOperand wo{__builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(g.w), (short)0, (int)(K * ldw * 4),
                                                          0x00020000),
                        (uint32_t)(((int64_t)slice * kq * ldw + (int64_t)part_i * Dm + h * D + 4 * c4) * 4),
                        (uint32_t)(ldw * 4)};
    f32x4 wa[kRpCh], wb[kRpCh];
    if (!copier) {
        f32x4 xv[kLnChunks];
        const int id = g.ids ? g.ids[b] : 0;  // uniform: one scalar load
        if (wave == 0) {
            if (g.ids) emb_row_load(g.tok, g.pos, id, g.vocab, K, lane, xv);
            else ln_row_load(g.x + (int64_t)b * g.ldx, K, lane, xv);
        }
        rp_first(wa, wb, wo);
        if (wave == 0) {
            if (g.ids && h == 0) {
                // head 0 stores the embedded row for the layer's residual path
                f32x4 *xr = reinterpret_cast<f32x4 *>(g.x + (int64_t)b * g.ldx);
#pragma unroll
                for (int i = 0; i < kLnChunks; i++)
                    if (i < K / 256) xr[lane + 64 * i] = xv[i];
                if (lane == 0 && (id < 0 || id >= g.vocab) && g.err) *g.err = 1;
            }
            ln_row_store(xv, K, g.eps, lane, lnx);
        }
    }
    lds_barrier();  // the normalised row is in LDS (the cache copies may still be in flight)
    PITON_PHASE(1);
    if (copier) copy_rows(kPreGroups, groups);
    if (!copier) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        rp_rest(wa, wb, wo, kq, lnx + slice * kq, acc);
        *reinterpret_cast<f32x4 *>(&gp[slice][4 * cgi]) = acc;
    }
    PITON_PHASE_WAIT_LOADS();  // traced builds: the copiers' stamps mark their copies landed
    PITON_PHASE(2);
    // the copies have landed (each wave waits for its own), then every wave's partials and
    // copies are visible after the barrier
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    lds_barrier();
    if (t < 3 * D) {
        const int pt = t / D, d = t % D;
        float v = gp[0][t];
#pragma unroll
        for (int sl = 1; sl < kDlWaves; sl++) v += gp[sl][t];
        if (g.bias) v += bias_raw;
        g.cache[((int64_t)jn * g.batch + b) * g.ldc + (int64_t)pt * Dm + h * D + d] = v;
        if (pt == 0) qn[d] = v;
        else if (pt == 1) ks[jn][d] = v;
        else vs[jn][d] = v;
    }
    lds_barrier();

    // 4. attention of q over keys 0 .. jn. Lane (kslot, sub) scores keys kslot + KPP it over
    // dims [16 sub, 16 sub + 16), its four 16-byte chunks in the order c + kslot (mod 4): the
    // 16 lanes of a read then fetch 16 distinct chunks of their keys' rows (rows 256 bytes apart
    // fall on the same banks).
    const int sub = t % TPK, kslot = t / TPK, d0 = 16 * sub;
    auto chunk = [&](int c) { return d0 + 4 * ((c + kslot) & 3); };
    float q16[16];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int e = 0; e < 4; e++) q16[4 * c + e] = qn[chunk(c) + e] * g.scale;
    float mloc = -INFINITY;
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int j = it * KPP + kslot;
        float sc = 0.f;
        if (j < n_keys) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const f32x4 kk = *reinterpret_cast<const f32x4 *>(&ks[j][chunk(c)]);
                sc = fmaf(q16[4 * c], kk[0], sc);
                sc = fmaf(q16[4 * c + 1], kk[1], sc);
                sc = fmaf(q16[4 * c + 2], kk[2], sc);
                sc = fmaf(q16[4 * c + 3], kk[3], sc);
            }
        }
#pragma unroll
        for (int o = 1; o < TPK; o <<= 1) sc += __shfl_xor(sc, o);
        if (j < n_keys) {
            if (sub == 0) p[j] = sc;
            mloc = fmaxf(mloc, sc);
        }
    }
    const float m = wg_reduce(mloc, MaxOp(), red);
    float lsum = 0.f;
    for (int j = t; j < n_keys; j += kDlThreads) {
        const float e = __builtin_amdgcn_exp2f(p[j] - m);
        p[j] = e;
        lsum += e;
    }
    const float inv = 1.0f / wg_reduce(lsum, SumOp(), red + kDlWaves);
    // thread (d, kg) sums keys kg, kg + KG, ... below n_keys in order
    const int d = t % D, kg = t / D;
    float acc = 0.f;
    int j = kg;
    for (; j + 7 * KG < n_keys; j += 8 * KG) {  // eight keys' reads ahead of their products
        float pj[8], vj[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            pj[u] = p[j + u * KG];
            vj[u] = vs[j + u * KG][d];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) acc = fmaf(pj[u], vj[u], acc);
    }
    for (; j < n_keys; j += KG) acc = fmaf(p[j], vs[j][d], acc);
    part[t] = acc;
    lds_barrier();
    if (t < D) {
        float v = part[t];
#pragma unroll
        for (int w = 1; w < KG; w++) v += part[w * D + t];
        g.o[(int64_t)b * g.ldo + h * D + t] = v * inv;
    }
    PITON_PHASE(3);
    PITON_PHASE_END(kPhaseDecodeLayer, g.phase);
}

struct LmHeadArgs {
    const float *x;  // row m at x + m * ldx
    int64_t ldx;
    float eps;
    const float *w;     // [K, N] row-major
    const float *bias;  // [N] or null
    float *logits;      // row m at logits + m * ldl, or null
    int64_t ldl;
    int32_t *next;  // [M]
    int N, K, n_classes;
};

__global__ __launch_bounds__(kDlThreads) void lm_head_kernel(LmHeadArgs g) {
    // read with the other arguments, not reloaded where they are first used
    g.eps = sgpr_keep(g.eps);
    g.logits = sgpr_keep(g.logits);
    g.next = sgpr_keep(g.next);
    g.n_classes = sgpr_keep(g.n_classes);
    constexpr int kMaxN = kDlMaxModel, NJ = kMaxN / kDlThreads;
    __shared__ __attribute__((aligned(16))) float lnx[kDlMaxModel];
    __shared__ __attribute__((aligned(16))) float gp[kDlWaves][kMaxN];
    __shared__ float rv[kDlWaves];
    __shared__ int ri[kDlWaves];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int m = blockIdx.x, N = g.N, K = g.K, ng = N / 4;
    // the bias of logits t + 512 j (from a valid address for every thread: the weights stand in
    // without a bias, K N >= N floats)
    const float *bias_p = g.bias ? g.bias : g.w;
    float bias_raw[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) bias_raw[j] = bias_p[min(t + kDlThreads * j, N - 1)];
    // wave w: k range [w K/8, (w+1) K/8); lane l: column groups l + 64 j (groups past N/4 re-read
    // the last one and are not stored)
    const int kq = K / kDlWaves;
    const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(g.w), (short)0, K * N * 4, 0x00020000);
    auto cols = [&](int j) {
        return RowOperand{rw, (uint32_t)(((int64_t)wave * kq * N + 4 * min(lane + 64 * j, ng - 1)) * 4),
                          (uint32_t)(N * 4)};
    };
    f32x4 wa[kRpCh], wb[kRpCh];
    f32x4 xv[kLnChunks];
    if (wave == 0) ln_row_load(g.x + (int64_t)m * g.ldx, K, lane, xv);
    rp_first(wa, wb, cols(0));
    if (wave == 0) ln_row_store(xv, K, g.eps, lane, lnx);
    lds_barrier();
    for (int j = 0; j < (ng + 63) / 64; j++) {
        if (j > 0) rp_first(wa, wb, cols(j));
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        rp_rest(wa, wb, cols(j), kq, lnx + wave * kq, acc);
        if (lane + 64 * j < ng) *reinterpret_cast<f32x4 *>(&gp[wave][4 * (lane + 64 * j)]) = acc;
    }
    lds_barrier();
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int n = t + kDlThreads * j;
        if (n < N) {
            float v = gp[0][n];
#pragma unroll
            for (int w = 1; w < kDlWaves; w++) v += gp[w][n];
            if (g.bias) v += bias_raw[j];
            if (g.logits) g.logits[(int64_t)m * g.ldl + n] = v;
            if (n < g.n_classes) argmax_combine(bv, bi, v, n);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v2 = __shfl_xor(bv, o);
        const int i2 = __shfl_xor(bi, o);
        argmax_combine(bv, bi, v2, i2);
    }
    if (lane == 0) {
        rv[wave] = bv;
        ri[wave] = bi;
    }
    lds_barrier();
    if (t == 0) {
        float v = rv[0];
        int i = ri[0];
#pragma unroll
        for (int w = 1; w < kDlWaves; w++) argmax_combine(v, i, rv[w], ri[w]);
        g.next[m] = i;
    }
}

}  // namespace

}  // namespace piton

PITON_PHASE_TU(decode_layer)

extern "C" int32_t piton_mi355x_decode_layer(float *x, int64_t ldx, float eps, const float *w, const float *bias,
                                             float *cache, int64_t ldc, float *out, int64_t ldo, float sm_scale,
                                             int64_t n_keys, int64_t batch, int64_t n_heads, int32_t head_dim,
                                             int64_t d_model, const int32_t *ids, const float *tok,
                                             const float *pos, int64_t vocab, int32_t *err, void *stream) {
    using namespace piton;
    PITON_REQUIRE(n_keys >= 1 && batch >= 0 && n_heads >= 1 && d_model >= 1, PITON_EINVAL,
                  "decode_layer: n_keys=%lld batch=%lld n_heads=%lld d_model=%lld", (long long)n_keys,
                  (long long)batch, (long long)n_heads, (long long)d_model);
    PITON_REQUIRE(head_dim == kDlD && d_model == n_heads * kDlD, PITON_EUNSUPPORTED,
                  "decode_layer: needs head_dim 64 and d_model = n_heads * 64 (head_dim %d, d_model %lld, %lld heads)",
                  head_dim, (long long)d_model, (long long)n_heads);
    PITON_REQUIRE(d_model % 256 == 0 && d_model <= kDlMaxModel, PITON_EUNSUPPORTED,
                  "decode_layer: d_model %lld not a multiple of 256 up to %d", (long long)d_model, kDlMaxModel);
    PITON_REQUIRE(n_keys <= kDlKeys, PITON_EUNSUPPORTED, "decode_layer: %lld keys exceed %d", (long long)n_keys,
                  kDlKeys);
    PITON_REQUIRE(batch == 0 || (x && w && cache && out), PITON_EINVAL, "decode_layer: null pointer");
    PITON_REQUIRE(ldx >= d_model && ldo >= d_model && ldc >= 3 * d_model, PITON_EINVAL,
                  "decode_layer: row strides ldx=%lld ldc=%lld ldo=%lld below the row widths", (long long)ldx,
                  (long long)ldc, (long long)ldo);
    PITON_REQUIRE(aligned16(w) && aligned16(cache) && ldc % 4 == 0 && aligned16(x) && ldx % 4 == 0 &&
                      aligned4(out) && (!bias || aligned4(bias)),
                  PITON_EUNSUPPORTED,
                  "decode_layer: W, the cache and x need 16-byte alignment (ldc %% 4 == 0, ldx %% 4 == 0)");
    // every cache offset the kernel forms (copies of up to three rows past the last one included)
    // fits 31 bits
    PITON_REQUIRE(sat_mul(sat_mul(n_keys + 3, batch), ldc) < 0x7FFFFFFF / 4 - 3 * d_model, PITON_EUNSUPPORTED,
                  "decode_layer: the cache exceeds 2 GiB");
    PITON_REQUIRE(sat_mul(batch, n_heads) <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "decode_layer: too many heads");
    PITON_REQUIRE(!ids || (tok && pos && vocab >= 1 && aligned16(tok) && aligned16(pos) && aligned4(ids)),
                  ids && (!tok || !pos || vocab < 1) ? PITON_EINVAL : PITON_EUNSUPPORTED,
                  "decode_layer: with ids, tok and pos are required (16-byte aligned) and vocab >= 1");
    int rc = require_device();
    if (rc) return rc;
    if (batch == 0) return PITON_OK;
    DecodeLayerArgs g{x, ldx, eps, w, bias, cache, ldc, out, ldo, sm_scale * 1.44269504088896341f,
                      (int)n_keys, (int)batch, (int)n_heads, (int)d_model, ids, tok, pos, vocab, err, phase_slot()};
    PITON_LAUNCH(decode_layer_kernel, dim3((unsigned)(batch * n_heads)), dim3(kDlThreads), 0, (hipStream_t)stream, g);
    rc = check_launch("decode_layer");
    if (rc == PITON_OK) clear_error();
    return rc;
}

extern "C" int32_t piton_mi355x_lm_head_argmax(const float *x, int64_t ldx, float eps, const float *w,
                                               const float *bias, float *logits, int64_t ldl, int32_t *next,
                                               int64_t M, int64_t N, int64_t K, int32_t n_classes, void *stream) {
    using namespace piton;
    PITON_REQUIRE(M >= 0 && N >= 1 && K >= 1 && n_classes >= 1 && n_classes <= N, PITON_EINVAL,
                  "lm_head_argmax: M=%lld N=%lld K=%lld n_classes=%d", (long long)M, (long long)N, (long long)K,
                  n_classes);
    PITON_REQUIRE(K % 256 == 0 && K <= kDlMaxModel && N % 4 == 0 && N <= kDlMaxModel, PITON_EUNSUPPORTED,
                  "lm_head_argmax: needs K a multiple of 256 and N a multiple of 4, both up to %d (K=%lld N=%lld)",
                  kDlMaxModel, (long long)K, (long long)N);
    PITON_REQUIRE(M == 0 || (x && w && next), PITON_EINVAL, "lm_head_argmax: null pointer");
    PITON_REQUIRE(ldx >= K && (!logits || ldl >= N), PITON_EINVAL, "lm_head_argmax: row strides below the rows");
    PITON_REQUIRE(aligned16(x) && ldx % 4 == 0 && aligned16(w) && (!logits || aligned4(logits)) && aligned4(next) &&
                      (!bias || aligned4(bias)),
                  PITON_EUNSUPPORTED, "lm_head_argmax: x rows and W need 16-byte alignment");
    PITON_REQUIRE(M <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "lm_head_argmax: too many rows");
    int rc = require_device();
    if (rc) return rc;
    if (M == 0) return PITON_OK;
    LmHeadArgs g{x, ldx, eps, w, bias, logits, ldl, next, (int)N, (int)K, n_classes};
    PITON_LAUNCH(lm_head_kernel, dim3((unsigned)M), dim3(kDlThreads), 0, (hipStream_t)stream, g);
    rc = check_launch("lm_head_argmax");
    if (rc == PITON_OK) clear_error();
    return rc;
}
