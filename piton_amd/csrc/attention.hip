// Flash attention forward: attn_fwd_kernel + _attn_fwd_inner (examples/attention.py:33-113).
//
// Design (gfx950, fp32 MFMA v_mfma_f32_32x32x2_f32):
//   * workgroup = 4 wavefronts = 64 query rows of one head: two query groups of 32, each split
//     over two waves by key parity; the workgroup walks the keys in tiles of 64 (two 32-key
//     MFMA blocks) staged through LDS (two buffers, the next tile prefetched into registers
//     while the current one is multiplied); the two waves of a query group merge their
//     partial softmax states through LDS at the end;
//   * the score block is computed transposed, S^T = K Q^T (keys x queries), so a lane holds
//     16 scores of ONE query (lane % 32): the row max and row sum are 15 in-lane operations
//     plus one exchange with lane ^ 32, and the running max / sum / rescale factor of a query
//     live in its own lanes;
//   * the output is accumulated transposed too, O^T += V^T P^T: the B operand of step s is
//     exactly the lane's own score register s (key order permuted to match the MFMA's output
//     layout), so P never moves between lanes, and alpha rescales the lane's own accumulators;
//   * sm_scale * log2(e) is folded into Q once, and the online softmax uses v_exp_f32 (exp2)
//     as the reference does with tl.exp2;
//   * causal: a workgroup loads key blocks up to its last query; a wave skips the blocks
//     entirely past its own queries; the diagonal block is masked per element; workgroups
//     are issued longest-first;
//   * K is read through (stride_kn, stride_kk): float4 along d for [N, D] storage, float4 along
//     keys for pre-transposed [D, N] storage, scalar otherwise.
#include "common.h"

namespace piton {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// widest head dimension that uses the register prefetch of the next tile
#ifndef PITON_ATTN_PREFETCH_MAX_D
#define PITON_ATTN_PREFETCH_MAX_D 64
#endif

constexpr int ABN = 32;  // keys per MFMA block
constexpr int ABM = 64;  // queries per workgroup
constexpr int AKT = 64;  // keys per LDS tile (two blocks: one per key parity)

enum : int { K_VEC_D = 0, K_VEC_N = 1, K_SCALAR = 2 };

struct AttnArgs {
    const float *q, *k, *v;
    float *o;
    float scale;  // sm_scale * log2(e)
    int64_t s_qh, s_qm, s_kh, s_kn, s_kk, s_vh, s_vn, s_oh, s_om;
    int64_t n_ctx;
    int64_t s_qb, s_kb, s_vb, s_ob;  // batch strides: grid row y is (batch y / n_heads, head y % n_heads)
    int64_t n_heads;
    int head_dim;
    int causal;
    int v_vec;  // V rows loadable as float4
};

// values per thread of one K (or V) tile of AKT keys x D
template <int D>
struct Tile {
    static constexpr int kVals = AKT * D / 256;
    static constexpr int kVec = kVals / 4;
};

template <int D, int KL>
__device__ __forceinline__ void attn_load(const AttnArgs &g, int t, const float *kb, const float *vb, int64_t key0,
                                          float (&rk)[Tile<D>::kVals], float (&rv)[Tile<D>::kVals]) {
    constexpr int NV = Tile<D>::kVec, NS = Tile<D>::kVals;
    if constexpr (KL == K_VEC_D) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = t + 256 * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            const int64_t n = key0 + key;
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (n < g.n_ctx && 4 * dq < g.head_dim) f = *reinterpret_cast<const float4 *>(kb + n * g.s_kn + 4 * dq);
            rk[4 * i] = f.x; rk[4 * i + 1] = f.y; rk[4 * i + 2] = f.z; rk[4 * i + 3] = f.w;
        }
    } else if constexpr (KL == K_VEC_N) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = t + 256 * i;
            const int d = idx / (AKT / 4), kq = idx % (AKT / 4);
            const int64_t n = key0 + 4 * kq;
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (n < g.n_ctx && d < g.head_dim) f = *reinterpret_cast<const float4 *>(kb + d * g.s_kk + n);
            rk[4 * i] = f.x; rk[4 * i + 1] = f.y; rk[4 * i + 2] = f.z; rk[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int idx = t + 256 * i;
            const int key = idx / D, d = idx % D;
            const int64_t n = key0 + key;
            rk[i] = (n < g.n_ctx && d < g.head_dim) ? kb[n * g.s_kn + d * g.s_kk] : 0.f;
        }
    }
    if (g.v_vec) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = t + 256 * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            const int64_t n = key0 + key;
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (n < g.n_ctx && 4 * dq < g.head_dim) f = *reinterpret_cast<const float4 *>(vb + n * g.s_vn + 4 * dq);
            rv[4 * i] = f.x; rv[4 * i + 1] = f.y; rv[4 * i + 2] = f.z; rv[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int idx = t + 256 * i;
            const int key = idx / D, d = idx % D;
            const int64_t n = key0 + key;
            rv[i] = (n < g.n_ctx && d < g.head_dim) ? vb[n * g.s_vn + d] : 0.f;
        }
    }
}

template <int D, int KL>
__device__ __forceinline__ void attn_store(const AttnArgs &g, int t, float (*Ks)[D + 1], float (*Vs)[D],
                                           const float (&rk)[Tile<D>::kVals], const float (&rv)[Tile<D>::kVals]) {
    constexpr int NV = Tile<D>::kVec, NS = Tile<D>::kVals;
    if constexpr (KL == K_VEC_D) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = t + 256 * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
#pragma unroll
            for (int j = 0; j < 4; j++) Ks[key][4 * dq + j] = rk[4 * i + j];
        }
    } else if constexpr (KL == K_VEC_N) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = t + 256 * i;
            const int d = idx / (AKT / 4), kq = idx % (AKT / 4);
#pragma unroll
            for (int j = 0; j < 4; j++) Ks[4 * kq + j][d] = rk[4 * i + j];
        }
    } else {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int idx = t + 256 * i;
            Ks[idx / D][idx % D] = rk[i];
        }
    }
    if (g.v_vec) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int idx = t + 256 * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            *reinterpret_cast<float4 *>(&Vs[key][4 * dq]) = make_float4(rv[4 * i], rv[4 * i + 1], rv[4 * i + 2], rv[4 * i + 3]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int idx = t + 256 * i;
            Vs[idx / D][idx % D] = rv[i];
        }
    }
}

// Workgroup: 64 queries of one head; wave w = (query group w / 2, key parity w % 2). Each
// iteration stages 64 keys (two 32-key blocks) in LDS; wave (g, p) multiplies block p of the
// tile for its 32 queries, so the two waves of a query group split the keys and each walks
// half as many blocks. Their running (max, sum, O) merge through LDS at the end.
template <int D, int KL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1)))
void attn_fwd_kernel_f32(AttnArgs g) {
    // D <= 64: two LDS buffers and the next tile prefetched into registers during the
    // current tile's products; D = 128: one buffer, loaded between two barriers (the
    // registers the prefetch would hold are the accumulators' at this width)
    constexpr bool kPrefetch = D <= PITON_ATTN_PREFETCH_MAX_D;
    constexpr int KS = AKT * (D + 1), VS = AKT * D, NBUF = kPrefetch ? 2 : 1;
    __shared__ float smem[NBUF * (KS + VS)];
    auto kt = [&](int buf) { return reinterpret_cast<float(*)[D + 1]>(smem + buf * (KS + VS)); };
    auto vt = [&](int buf) { return reinterpret_cast<float(*)[D]>(smem + buf * (KS + VS) + KS); };

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, half = lane >> 5, l31 = lane & 31;
    const int grp = wave >> 1, par = wave & 1;
    const int qb = g.causal ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;  // longest first
    const int64_t bh = blockIdx.y, bi = bh / g.n_heads, h = bh % g.n_heads;
    const int64_t q0 = (int64_t)qb * ABM + grp * 32;  // this wave's first query
    const int64_t qi = q0 + l31;                       // this lane's query

    const float *qp = g.q + bi * g.s_qb + h * g.s_qh;
    const float *kbase = g.k + bi * g.s_kb + h * g.s_kh;
    const float *vbase = g.v + bi * g.s_vb + h * g.s_vh;

    // Q'^T fragments: B[k = d][n = query] for d = 2s + half, scaled by sm_scale * log2 e
    float qf[D / 2];
#pragma unroll
    for (int s = 0; s < D / 2; s++) {
        const int d = 2 * s + half;
        qf[s] = (qi < g.n_ctx && d < g.head_dim) ? qp[qi * g.s_qm + d] * g.scale : 0.f;
    }

    f32x16 o[D / 32];
#pragma unroll
    for (int b = 0; b < D / 32; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[b][r] = 0.f;
    float m_i = -INFINITY, l_i = 0.f;

    const int64_t nkb_all = (g.n_ctx + ABN - 1) / ABN;
    const int64_t nkb = g.causal ? min(nkb_all, (int64_t)(qb + 1) * (ABM / ABN)) : nkb_all;
    const int64_t nit = (nkb + 1) / 2;
    const int64_t wave_last = g.causal ? (q0 + 31) / ABN : nkb_all - 1;  // last block this wave needs

    float rk[Tile<D>::kVals], rv[Tile<D>::kVals];
    if (kPrefetch) {
        attn_load<D, KL>(g, t, kbase, vbase, 0, rk, rv);
        attn_store<D, KL>(g, t, kt(0), vt(0), rk, rv);
        __syncthreads();
    }

    for (int64_t it = 0; it < nit; it++) {
        const int cur = kPrefetch ? (int)(it & 1) : 0;
        const bool more = kPrefetch && it + 1 < nit;
        if (more) attn_load<D, KL>(g, t, kbase, vbase, (it + 1) * AKT, rk, rv);
        if (!kPrefetch) {
            attn_load<D, KL>(g, t, kbase, vbase, it * AKT, rk, rv);
            attn_store<D, KL>(g, t, kt(0), vt(0), rk, rv);
            __syncthreads();
        }

        const int64_t kb = 2 * it + par;
        if (kb < nkb && kb <= wave_last) {
            float(*Kt)[D + 1] = kt(cur) + par * ABN;
            float(*Vt)[D] = vt(cur) + par * ABN;
            // S^T block: A = K [key][d], B = Q'^T
            f32x16 st;
#pragma unroll
            for (int r = 0; r < 16; r++) st[r] = 0.f;
#pragma unroll
            for (int s = 0; s < D / 2; s++)
                st = __builtin_amdgcn_mfma_f32_32x32x2f32(Kt[l31][2 * s + half], qf[s], st, 0, 0, 0);

            // masks: register r holds key kb*32 + 8*(r/4) + 4*half + r%4 of query qi
            // key indices fit 32 bits (N_CTX < 2^31 is checked on the host)
            const int key0 = (int)kb * ABN + 4 * half, n_ctx = (int)g.n_ctx, qi32 = (int)qi;
            float mloc = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = key0 + 8 * (r >> 2) + (r & 3);
                if (key >= n_ctx || (g.causal && key > qi32)) st[r] = -INFINITY;
                mloc = fmaxf(mloc, st[r]);
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
            const float m_new = fmaxf(m_i, mloc);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;  // rows with nothing visible yet
            const float alpha = __builtin_amdgcn_exp2f(m_i - m_use);
            float lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                st[r] = __builtin_amdgcn_exp2f(st[r] - m_use);
                lsum += st[r];
            }
            lsum += __shfl_xor(lsum, 32);
            l_i = l_i * alpha + lsum;
            m_i = m_new;

            // O^T = O^T * alpha + V^T P^T; step s pairs key (s/4)*8 + 4*half + s%4 with P^T
            // register s of this lane
#pragma unroll
            for (int b = 0; b < D / 32; b++) {
#pragma unroll
                for (int r = 0; r < 16; r++) o[b][r] *= alpha;
#pragma unroll
                for (int s = 0; s < 16; s++) {
                    const int key = (s >> 2) * 8 + 4 * half + (s & 3);
                    o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vt[key][b * 32 + l31], st[s], o[b], 0, 0, 0);
                }
            }
        }

        if (more) attn_store<D, KL>(g, t, kt(cur ^ 1), vt(cur ^ 1), rk, rv);
        __syncthreads();
    }

    // merge the key-parity halves of each query group: parity-1 waves hand (m, l, O) over LDS
    // (same lane = same query and output element), parity-0 waves combine and store
    float *xo = smem;                              // [grp][D/2 values][64 lanes]
    float *xm = smem + 2 * (D / 2) * 64;           // [grp][2][64]
    if (par == 1) {
#pragma unroll
        for (int b = 0; b < D / 32; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) xo[(grp * (D / 2) + b * 16 + r) * 64 + lane] = o[b][r];
        xm[(grp * 2 + 0) * 64 + lane] = m_i;
        xm[(grp * 2 + 1) * 64 + lane] = l_i;
    }
    __syncthreads();
    if (par == 0 && qi < g.n_ctx) {
        const float m_b = xm[(grp * 2 + 0) * 64 + lane], l_b = xm[(grp * 2 + 1) * 64 + lane];
        const float m = fmaxf(m_i, m_b);
        const float mu = m == -INFINITY ? 0.f : m;
        const float ca = __builtin_amdgcn_exp2f(m_i - mu), cb = __builtin_amdgcn_exp2f(m_b - mu);
        const float inv = 1.0f / (l_i * ca + l_b * cb);
        float *op = g.o + bi * g.s_ob + h * g.s_oh + qi * g.s_om;
#pragma unroll
        for (int b = 0; b < D / 32; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int d = b * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                const float ob = xo[(grp * (D / 2) + b * 16 + r) * 64 + lane];
                if (d < g.head_dim) op[d] = (o[b][r] * ca + ob * cb) * inv;
            }
    }
}

template <int D>
static void launch_d(int kl, const AttnArgs &g, dim3 grid, hipStream_t st) {
    if (kl == K_VEC_D) hipLaunchKernelGGL((attn_fwd_kernel_f32<D, K_VEC_D>), grid, dim3(256), 0, st, g);
    else if (kl == K_VEC_N) hipLaunchKernelGGL((attn_fwd_kernel_f32<D, K_VEC_N>), grid, dim3(256), 0, st, g);
    else hipLaunchKernelGGL((attn_fwd_kernel_f32<D, K_SCALAR>), grid, dim3(256), 0, st, g);
}

// One new query per (batch, head) against keys 0 .. n_keys-1 of a cache (the decode step of a
// KV-cached decoder): one wavefront per (batch, head); lanes score keys j = lane, lane + 64, ...
// into LDS, two DPP reductions give the max and the sum, then lane d accumulates
// sum_j p_j V[j][d] with coalesced V rows.
constexpr int kMaxDecodeKeys = 8192;

struct DecodeArgs {
    const float *q, *k, *v;
    float *o;
    float scale;  // sm_scale * log2(e)
    int64_t s_qb, s_qh, s_kb, s_kh, s_kn, s_vb, s_vh, s_vn, s_ob, s_oh;
    int n_keys, n_heads, head_dim;
};

template <int D>
__global__ __launch_bounds__(64) void attn_decode_kernel(DecodeArgs g) {
    __shared__ float p[kMaxDecodeKeys];
    const int lane = threadIdx.x;
    const int64_t bh = blockIdx.x, b = bh / g.n_heads, h = bh % g.n_heads;
    const float *qp = g.q + b * g.s_qb + h * g.s_qh;
    const float *kp = g.k + b * g.s_kb + h * g.s_kh;
    const float *vp = g.v + b * g.s_vb + h * g.s_vh;
    float q[D];
#pragma unroll
    for (int d = 0; d < D; d++) q[d] = d < g.head_dim ? qp[d] * g.scale : 0.f;
    float mloc = -INFINITY;
    for (int j = lane; j < g.n_keys; j += 64) {
        const float *kr = kp + (int64_t)j * g.s_kn;
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < g.head_dim) s = fmaf(q[d], kr[d], s);
        p[j] = s;
        mloc = fmaxf(mloc, s);
    }
    const float m = wave_reduce(mloc, MaxOp());
    float lsum = 0.f;
    for (int j = lane; j < g.n_keys; j += 64) {
        const float e = __builtin_amdgcn_exp2f(p[j] - m);
        p[j] = e;
        lsum += e;
    }
    const float inv = 1.0f / wave_reduce(lsum, SumOp());
    __syncthreads();
    float *op = g.o + b * g.s_ob + h * g.s_oh;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += 64) {
        const int d = d0 + lane;
        if (d < g.head_dim) {
            float acc = 0.f;
            for (int j = 0; j < g.n_keys; j++) acc = fmaf(p[j], vp[(int64_t)j * g.s_vn + d], acc);
            op[d] = acc * inv;
        }
    }
}

static int attn_launch(AttnArgs g, int64_t batch, int64_t n_heads, int32_t head_dim, hipStream_t st) {
    g.v_vec = aligned16(g.v) && g.s_vn % 4 == 0 && g.s_vh % 4 == 0 && g.s_vb % 4 == 0 && head_dim % 4 == 0;
    int kl = K_SCALAR;
    if (g.s_kk == 1 && g.s_kn % 4 == 0 && g.s_kh % 4 == 0 && g.s_kb % 4 == 0 && aligned16(g.k) && head_dim % 4 == 0)
        kl = K_VEC_D;
    else if (g.s_kn == 1 && g.s_kk % 4 == 0 && g.s_kh % 4 == 0 && g.s_kb % 4 == 0 && aligned16(g.k) && g.n_ctx % 4 == 0)
        kl = K_VEC_N;
    const dim3 grid((unsigned)((g.n_ctx + ABM - 1) / ABM), (unsigned)(batch * n_heads));
    if (head_dim <= 32) launch_d<32>(kl, g, grid, st);
    else if (head_dim == 64) launch_d<64>(kl, g, grid, st);
    else launch_d<128>(kl, g, grid, st);
    return check_launch("attn_fwd");
}

static int attn_check(const float *q, const float *k, const float *v, const float *out, int64_t n_ctx, int64_t batch,
                      int64_t n_heads, int32_t head_dim) {
    PITON_REQUIRE(n_ctx >= 0 && n_heads >= 0 && batch >= 0, PITON_EINVAL, "attn_fwd: negative N_CTX, batch or heads");
    PITON_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128, PITON_EUNSUPPORTED,
                  "attn_fwd: HEAD_DIM %d not in {16, 32, 64, 128}", head_dim);
    PITON_REQUIRE(n_ctx == 0 || n_heads == 0 || batch == 0 || (q && k && v && out), PITON_EINVAL,
                  "attn_fwd: null pointer");
    PITON_REQUIRE(aligned4(q) && aligned4(k) && aligned4(v) && aligned4(out), PITON_EINVAL,
                  "attn_fwd: pointers must be 4-byte aligned");
    PITON_REQUIRE(batch * n_heads <= 65535, PITON_EUNSUPPORTED, "attn_fwd: %lld heads exceed grid axis 1",
                  (long long)(batch * n_heads));
    PITON_REQUIRE(n_ctx < (1LL << 31) - 64, PITON_EUNSUPPORTED, "attn_fwd: N_CTX %lld too large", (long long)n_ctx);
    return PITON_OK;
}

}  // namespace piton

extern "C" {

int32_t piton_mi355x_attn_fwd(const float *q, const float *k, const float *v, float *out, float sm_scale,
                              int64_t stride_qh, int64_t stride_qm, int64_t stride_kh, int64_t stride_kn,
                              int64_t stride_kk, int64_t stride_vh, int64_t stride_vn, int64_t stride_oh,
                              int64_t stride_om, int64_t n_ctx, int64_t n_heads, int32_t head_dim, int32_t causal,
                              void *stream) {
    using namespace piton;
    int rc = attn_check(q, k, v, out, n_ctx, 1, n_heads, head_dim);
    if (rc) return rc;
    rc = require_device();
    if (rc) return rc;
    if (n_ctx == 0 || n_heads == 0) return PITON_OK;
    AttnArgs g{q, k, v, out, sm_scale * 1.44269504088896341f, stride_qh, stride_qm, stride_kh, stride_kn, stride_kk,
               stride_vh, stride_vn, stride_oh, stride_om, n_ctx, 0, 0, 0, 0, n_heads, head_dim, causal ? 1 : 0, 0};
    rc = attn_launch(g, 1, n_heads, head_dim, (hipStream_t)stream);
    if (rc == PITON_OK) clear_error();
    return rc;
}

int32_t piton_mi355x_attn_fwd_batched(const float *q, const float *k, const float *v, float *out, float sm_scale,
                                      int64_t stride_qb, int64_t stride_qh, int64_t stride_qm, int64_t stride_kb,
                                      int64_t stride_kh, int64_t stride_kn, int64_t stride_kk, int64_t stride_vb,
                                      int64_t stride_vh, int64_t stride_vn, int64_t stride_ob, int64_t stride_oh,
                                      int64_t stride_om, int64_t n_ctx, int64_t batch, int64_t n_heads,
                                      int32_t head_dim, int32_t causal, void *stream) {
    using namespace piton;
    int rc = attn_check(q, k, v, out, n_ctx, batch, n_heads, head_dim);
    if (rc) return rc;
    rc = require_device();
    if (rc) return rc;
    if (n_ctx == 0 || n_heads == 0 || batch == 0) return PITON_OK;
    AttnArgs g{q, k, v, out, sm_scale * 1.44269504088896341f, stride_qh, stride_qm, stride_kh, stride_kn, stride_kk,
               stride_vh, stride_vn, stride_oh, stride_om, n_ctx, stride_qb, stride_kb, stride_vb, stride_ob, n_heads,
               head_dim, causal ? 1 : 0, 0};
    rc = attn_launch(g, batch, n_heads, head_dim, (hipStream_t)stream);
    if (rc == PITON_OK) clear_error();
    return rc;
}

int32_t piton_mi355x_attn_decode(const float *q, const float *k, const float *v, float *out, float sm_scale,
                                 int64_t stride_qb, int64_t stride_qh, int64_t stride_kb, int64_t stride_kh,
                                 int64_t stride_kn, int64_t stride_vb, int64_t stride_vh, int64_t stride_vn,
                                 int64_t stride_ob, int64_t stride_oh, int64_t n_keys, int64_t batch, int64_t n_heads,
                                 int32_t head_dim, void *stream) {
    using namespace piton;
    PITON_REQUIRE(n_keys >= 1 && batch >= 0 && n_heads >= 0, PITON_EINVAL, "attn_decode: n_keys=%lld batch=%lld",
                  (long long)n_keys, (long long)batch);
    PITON_REQUIRE(n_keys <= kMaxDecodeKeys, PITON_EUNSUPPORTED, "attn_decode: %lld keys exceed %d",
                  (long long)n_keys, kMaxDecodeKeys);
    PITON_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128, PITON_EUNSUPPORTED,
                  "attn_decode: HEAD_DIM %d not in {16, 32, 64, 128}", head_dim);
    PITON_REQUIRE(batch * n_heads == 0 || (q && k && v && out), PITON_EINVAL, "attn_decode: null pointer");
    PITON_REQUIRE(batch * n_heads <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "attn_decode: too many heads");
    int rc = require_device();
    if (rc) return rc;
    if (batch * n_heads == 0) return PITON_OK;
    DecodeArgs g{q, k, v, out, sm_scale * 1.44269504088896341f, stride_qb, stride_qh, stride_kb, stride_kh, stride_kn,
                 stride_vb, stride_vh, stride_vn, stride_ob, stride_oh, (int)n_keys, (int)n_heads, head_dim};
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(batch * n_heads)), block(64);
    if (head_dim <= 32) hipLaunchKernelGGL(attn_decode_kernel<32>, grid, block, 0, st, g);
    else if (head_dim == 64) hipLaunchKernelGGL(attn_decode_kernel<64>, grid, block, 0, st, g);
    else hipLaunchKernelGGL(attn_decode_kernel<128>, grid, block, 0, st, g);
    rc = check_launch("attn_decode");
    if (rc == PITON_OK) clear_error();
    return rc;
}

}  // extern "C"
