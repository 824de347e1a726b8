// One decode step of a layer of the KV-cached decoder in one launch: the layernorm of the new
// token's row, its QKV projection (written into the cache row of its position), and the
// single-query attention of every head over the cache. It equals piton_mi355x_linear_ln (QKV)
// followed by piton_mi355x_attn_decode on the decoder's position-major cache, to rounding: the
// projection here is a dot product per output instead of the matrix-core product.
//
// No reference counterpart: the reference has no decoder. The pieces it composes are the
// layernorm of tests/test_reroll_reduce.py:199-208, the dense layer of
// examples/nn_kernels.py:23-74 and the attention of examples/attention.py:33-113.
//
// Design (gfx950): one 256-thread workgroup per (sequence b, head h), 1 per CU at the decoder's
// 64 x 4 heads:
//   * first, wave 3 copies the head's cached keys and values of the earlier positions
//     memory -> LDS by 16-byte LDS-DMA (no registers; rows past the last one read as zeros), so
//     the cache streams in while the projection runs instead of after it;
//   * wave 0 normalises the row (float4 loads, mean and variance by wave reductions) into LDS;
//     192 threads of waves 0-2 then compute the head's 3 x 64 projection outputs: thread
//     (slice s, column group c) owns 4 consecutive columns of q, k or v and the k range
//     [s K/4, (s+1) K/4), reading 16-byte weight vectors (64 consecutive columns of a weight row
//     per 16 threads), two chunks of 16 rows in flight; the four slices add in slice order,
//     then the bias;
//   * the new q, k, v go to the cache row (t = n_keys - 1) and to LDS, and the attention runs
//     as attn_decode_short does: TPK = 4 lanes per key score 16 dims each (read from LDS in a
//     bank-conflict-free chunk order), the maximum and the sum of 2^(s - m) reduce over the
//     workgroup, thread (d, g) sums p_j V[j][d] over the keys j = g (mod 4) in key order, and
//     the four partial sums add in order.
#include "common.h"

namespace piton {

namespace {

constexpr int kDlD = 64;          // head_dim
constexpr int kDlKeys = 256;      // cache rows a launch attends to (the decoder's context)
constexpr int kDlMaxModel = 1024;  // d_model

struct DecodeLayerArgs {
    const float *x;  // the new rows, row b at x + b * ldx
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
    PhaseRecord *phase;  // the launch's phase-trace records (diagnostics builds; null otherwise)
};

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// A workgroup barrier for LDS data: this wave's LDS stores are done, then s_barrier. Unlike
// __syncthreads, whose release fence waits for every memory operation in flight, it lets the
// cache copies and the global stores (the cache row, which nothing here reads back) stay in
// flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitcntLgkm0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
}

// sum or max over the workgroup's 256 threads: DPP within the wave, then the four wave results
// through `red` (four floats of its own per call), combined in wave order
template <class Op>
__device__ __forceinline__ float wg_reduce(float v, Op op, float *red) {
    v = wave_reduce(v, op);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    return op(op(red[0], red[1]), op(red[2], red[3]));
}

__global__ __launch_bounds__(256) void decode_layer_kernel(DecodeLayerArgs g) {
    constexpr int D = kDlD, TPK = D / 16, KPP = 256 / TPK, KG = 256 / D, NIT = kDlKeys / KPP;
    __shared__ __attribute__((aligned(16))) float ks[kDlKeys][D];  // keys of the head (64 KB)
    __shared__ __attribute__((aligned(16))) float vs[kDlKeys][D];  // values (64 KB)
    __shared__ __attribute__((aligned(16))) float lnx[kDlMaxModel];
    __shared__ __attribute__((aligned(16))) float gp[4][3 * D];  // projection partials per k slice
    __shared__ float qn[D];
    __shared__ float p[kDlKeys];
    __shared__ float red[16];
    __shared__ float part[256];

    // the wave index is uniform (readfirstlane): its branches are scalar, and the copies' LDS
    // addresses need no per-lane loop
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int b = __builtin_amdgcn_readfirstlane(blockIdx.x / g.n_heads);
    const int h = __builtin_amdgcn_readfirstlane(blockIdx.x % g.n_heads);
    const int n_keys = g.n_keys, jn = n_keys - 1, Dm = g.d_model, K = Dm;
    const int64_t ldw = 3 * (int64_t)Dm;
    PITON_PHASE_VARS;
    PITON_PHASE(0);
    // output t < 192 of the projection: part t / 64 (q, k, v), dim t % 64. Its bias is requested
    // now, not after the product, and unconditionally (every thread, from a valid address; the
    // value is selected where it is used): a load under a condition compiles to a branch whose
    // join waits for it, which would hold the wave for a memory round trip here.
    // (threads past 192 re-read output 191's; without a bias the weights stand in, 3 d_model
    // floats long at least, and the value is not used)
    const float *bias_p = g.bias ? g.bias : g.w;
    const int tb = min(t, 3 * D - 1);
    const float bias_raw = bias_p[(tb / D) * Dm + h * D + tb % D];

    // The vector-memory counter is in order per wave: a wave that waits for one load waits for
    // every load it issued before it. So the cache copies come from wave 3 alone, which takes no
    // part in the projection, and waves 0-2 issue only the projection's loads (wave 0 the row's
    // first): none of their waits covers a cache copy.
    // 1. wave 3: the earlier positions' keys and values -> LDS. Lane l of a copy carries 16 bytes
    // of key 4 i + l / 16 (dims 4 (l % 16) ..); the descriptors end at the last earlier row, so
    // the rows from jn on arrive as zeros.
    // A wave holds at most 63 memory operations in flight and stalls issuing the next, so wave 3
    // issues the copies of the first kPreGroups groups of four keys before the layernorm's
    // barrier (which it would otherwise hold up) and the rest after it.
    constexpr int kPreGroups = 28;
    const int groups = (jn + 3) / 4;
    auto copy_kv = [&](int i0, int i1) {
        const int64_t row_stride = (int64_t)g.batch * g.ldc;  // floats between positions
        float *kb = g.cache + (int64_t)b * g.ldc + Dm + h * D;
        const uint32_t bytes = jn > 0 ? (uint32_t)(((int64_t)(jn - 1) * row_stride + D) * 4) : 0u;
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(kb, (short)0, (int)bytes, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(kb + Dm, (short)0, (int)bytes, 0x00020000);
        for (int i = i0; i < i1; i++) {
            const uint32_t off = (uint32_t)(((int64_t)(4 * i + (lane >> 4)) * row_stride + 4 * (lane & 15)) * 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)&ks[4 * i][0], 16, off, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)&vs[4 * i][0], 16, off, 0, 0, 0);
        }
    };
    if (wave == 3) copy_kv(0, min(groups, kPreGroups));

    // 2. wave 0: layernorm of row b into LDS, lane l holding columns 4 l + 256 i .. + 3
    // (K % 256 == 0). 3. waves 0-2: the head's projection, thread t < 192 = (slice, column group):
    // group c covers the 4 columns 4 (c % 16) .. of part c / 16 (q, k, v) of head h and the k
    // range [slice K/4, (slice+1) K/4); its first chunk of weights is requested before the
    // layernorm.
    const int cgi = t % (3 * D / 4), slice = t / (3 * D / 4);
    const int part_i = cgi / (D / 4), c4 = cgi % (D / 4);
    const int kq = K / 4, k0 = slice * kq;
    const float *wp = g.w + (int64_t)k0 * ldw + (int64_t)part_i * Dm + h * D + 4 * c4;
    constexpr int CH = 16;
    f32x4 wa[CH], wb[CH];
    auto load = [&](f32x4 (&w)[CH], int k) {
#pragma unroll
        for (int i = 0; i < CH; i++) w[i] = *reinterpret_cast<const f32x4 *>(wp + (int64_t)(k + i) * ldw);
    };
    if (wave < 3) {
        constexpr int NX = kDlMaxModel / 256;
        const int nx = K / 256;
        f32x4 xv[NX];
        if (wave == 0) {
            // unconditional loads (chunks past the row re-read its last one and are dropped
            // when summed): a conditional load's join would wait for it
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(g.x + (int64_t)b * g.ldx);
#pragma unroll
            for (int i = 0; i < NX; i++) xv[i] = xr[min(lane + 64 * i, 64 * nx - 1)];
        }
        load(wa, 0);
        if (wave == 0) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < NX; i++)
                if (i < nx) s += (xv[i][0] + xv[i][1]) + (xv[i][2] + xv[i][3]);
            const float mean = wave_reduce(s, SumOp()) / (float)K;
            float q2 = 0.f;
#pragma unroll
            for (int i = 0; i < NX; i++)
                if (i < nx)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float d = xv[i][e] - mean;
                        q2 = fmaf(d, d, q2);
                    }
            const float inv_sd = 1.0f / sqrtf(wave_reduce(q2, SumOp()) / (float)K + g.eps);
#pragma unroll
            for (int i = 0; i < NX; i++)
                if (i < nx) {
                    f32x4 y;
#pragma unroll
                    for (int e = 0; e < 4; e++) y[e] = (xv[i][e] - mean) * inv_sd;
                    *reinterpret_cast<f32x4 *>(&lnx[4 * lane + 256 * i]) = y;
                }
        }
    }
    lds_barrier();  // the normalised row is in LDS (the cache copies may still be in flight)
    PITON_PHASE(1);
    if (wave == 3) copy_kv(kPreGroups, groups);
    if (wave < 3) {
        const float *ap = lnx + k0;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        auto mul = [&](const f32x4 (&w)[CH], int k) {
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const float a = ap[k + i];
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = fmaf(a, w[i][e], acc[e]);
            }
        };
        // kq % (2 CH) == 0 (K % 128 == 0)
        for (int k = 0; k < kq; k += 2 * CH) {
            load(wb, k + CH);
            mul(wa, k);
            if (k + 2 * CH < kq) load(wa, k + 2 * CH);
            mul(wb, k + CH);
        }
        *reinterpret_cast<f32x4 *>(&gp[slice][4 * cgi]) = acc;
    }
    PITON_PHASE_WAIT_LOADS();  // traced builds: wave 3's stamp marks its cache copies landed
    PITON_PHASE(2);
    // the cache copies have landed (this wave's), and every wave's partials and copies are
    // visible after the barrier
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    lds_barrier();
    if (wave < 3) {
        const int part_i = t / D, d = t % D;
        float v = gp[0][t];
#pragma unroll
        for (int sl = 1; sl < 4; sl++) v += gp[sl][t];
        if (g.bias) v += bias_raw;
        g.cache[((int64_t)jn * g.batch + b) * g.ldc + (int64_t)part_i * Dm + h * D + d] = v;
        if (part_i == 0) qn[d] = v;
        else if (part_i == 1) ks[jn][d] = v;
        else vs[jn][d] = v;
    }
    lds_barrier();

    // 4. attention of q over keys 0 .. jn (attn_decode_short's arithmetic)
    // Lane (kslot, sub) scores keys kslot + 64 it over dims [16 sub, 16 sub + 16), its four
    // 16-byte chunks in the order c + kslot (mod 4): the 16 lanes of a read then fetch 16
    // distinct chunks of their keys' rows (rows 256 bytes apart fall on the same banks).
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
    const float m = wg_reduce(mloc, MaxOp(), red + 8);
    float lsum = 0.f;
    for (int j = t; j < n_keys; j += 256) {
        const float e = __builtin_amdgcn_exp2f(p[j] - m);
        p[j] = e;
        lsum += e;
    }
    const float inv = 1.0f / wg_reduce(lsum, SumOp(), red + 12);
    // thread (d, kg) sums keys kg, kg + KG, ... below n_keys in order (the absent keys of the
    // short kernel add exact zeros, so stopping at n_keys gives the same sum)
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

}  // namespace

}  // namespace piton

PITON_PHASE_TU(decode_layer)

extern "C" int32_t piton_mi355x_decode_layer(const float *x, int64_t ldx, float eps, const float *w,
                                             const float *bias, float *cache, int64_t ldc, float *out, int64_t ldo,
                                             float sm_scale, int64_t n_keys, int64_t batch, int64_t n_heads,
                                             int32_t head_dim, int64_t d_model, void *stream) {
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
    PITON_REQUIRE(((n_keys + 3) * batch * ldc + 3 * d_model) * 4 < 0x7FFFFFFF, PITON_EUNSUPPORTED,
                  "decode_layer: the cache exceeds 2 GiB");
    PITON_REQUIRE(batch * n_heads <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "decode_layer: too many heads");
    int rc = require_device();
    if (rc) return rc;
    if (batch == 0) return PITON_OK;
    DecodeLayerArgs g{x, ldx, eps, w, bias, cache, ldc, out, ldo, sm_scale * 1.44269504088896341f,
                      (int)n_keys, (int)batch, (int)n_heads, (int)d_model, phase_slot()};
    PITON_LAUNCH(decode_layer_kernel, dim3((unsigned)(batch * n_heads)), dim3(256), 0, (hipStream_t)stream, g);
    rc = check_launch("decode_layer");
    if (rc == PITON_OK) clear_error();
    return rc;
}
