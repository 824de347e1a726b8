// Flash attention forward: attn_fwd_kernel + _attn_fwd_inner (examples/attention.py:33-113).
//
// Design (gfx950, fp32 MFMA v_mfma_f32_32x32x2_f32), no LDS staging and no barrier in the key
// loop:
//   * workgroup = 4 wavefronts on one group of 32 queries of one head; wave w walks key blocks
//     w, w + 4, ... (32 keys each), so a long causal row is split four ways; the four partial
//     softmax states (max, sum, O) merge through LDS once at the end;
//   * the score block is computed transposed, S^T = K Q^T (keys x queries), so a lane holds
//     16 scores of ONE query (lane % 32): the row max and row sum are 15 in-lane operations
//     plus one exchange with lane ^ 32, and the running max / sum / rescale factor of a query
//     live in its own lanes;
//   * the MFMA k-index is permuted so that lane half h carries head dims [h*D/2, (h+1)*D/2):
//     a lane's K operand is then a contiguous half row of one key and its Q operand a half row
//     of its query, loaded as float4 straight from global memory (L2) into operand registers;
//   * the output is accumulated transposed, O^T += V^T P^T: the A operand is V rows, 32
//     consecutive dims per half wave (128-byte coalesced loads), and the B operand of step s is
//     the lane's own score register s (key order permuted to the MFMA output layout), so P
//     never moves between lanes and alpha rescales the lane's own accumulators;
//   * sm_scale * log2(e) is folded into Q once; the online softmax uses v_exp_f32 (exp2) as the
//     reference does with tl.exp2;
//   * workgroups map to XCDs by whole heads (the dispatcher deals them round-robin over the 8
//     XCDs), so a head's K and V stay in one XCD's L2 while its query groups stream them;
//   * causal: a query group visits only the key blocks up to its last query, only blocks that
//     can hold a masked key are masked, and each XCD issues its longest groups first;
//   * K is read through (stride_kn, stride_kk): float4 along d for [N, D] storage, scalar
//     loads (consecutive keys across lanes) for pre-transposed [D, N] storage.
#include "common.h"

#include <algorithm>
#include <type_traits>

namespace piton {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// waves per SIMD the D <= 64 kernels are register-budgeted for
#ifndef PITON_ATTN_WAVES_PER_EU
#define PITON_ATTN_WAVES_PER_EU 2
#endif

constexpr int ABN = 32;  // keys per MFMA block
constexpr int AQG = 32;  // queries per workgroup (one query group)
constexpr int ANW = 4;   // waves per workgroup, each taking every ANW-th key block

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
    int q_vec;  // Q rows loadable as float4
    int v_vec;  // V rows loadable as float4
    int nqg, nbh;  // query groups per head, batch * heads (the 1-D grid is nqg * nbh)
    PhaseRecord *phase;  // the launch's phase-trace records (diagnostics builds; null otherwise)
};

// MFMA k-index of the score product: lane half h carries head dims [h*D/2, (h+1)*D/2), step s
// the dim h*D/2 + s, so each lane's operand is a contiguous half row of K (or Q).
template <int D, int KL>
__device__ __forceinline__ void load_k_operand(const AttnArgs &g, const float *kb, int64_t key, int half,
                                               float (&kf)[D / 2]) {
    const int d0 = half * (D / 2);
    const bool ok = key < g.n_ctx;
    if constexpr (KL == K_VEC_D) {
#pragma unroll
        for (int c = 0; c < D / 8; c++) {
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (ok && d0 + 4 * c < g.head_dim) f = *reinterpret_cast<const float4 *>(kb + key * g.s_kn + d0 + 4 * c);
            kf[4 * c] = f.x; kf[4 * c + 1] = f.y; kf[4 * c + 2] = f.z; kf[4 * c + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < D / 2; s++)
            kf[s] = (ok && d0 + s < g.head_dim) ? kb[key * g.s_kn + (int64_t)(d0 + s) * g.s_kk] : 0.f;
    }
}

// ---- the per-block steps both forward kernels share (identical arithmetic) ----------------

// workgroup -> (batch*head, query group): the dispatcher deals workgroups round-robin over the
// XCDs, so give each XCD whole heads (their K and V stay in that XCD's L2), and within an XCD
// issue the longest causal groups of all its heads first
__device__ __forceinline__ void map_group(const AttnArgs &g, int64_t &bh, int &qg) {
    const int nqg = g.nqg, nbh = g.nbh;
    int qrank;
    if (nbh % kXcdCount == 0) {
        const int xcd = blockIdx.x % kXcdCount, i = blockIdx.x / kXcdCount, per = nbh / kXcdCount;
        bh = (int64_t)xcd * per + i % per;
        qrank = i / per;
    } else {
        bh = blockIdx.x / nqg;
        qrank = blockIdx.x % nqg;
    }
    qg = g.causal ? nqg - 1 - qrank : qrank;
}

// The key blocks of a query group are dealt to the ANW waves round-robin, wave w taking blocks
// first_block(w, qg), + ANW, ... Groups qg = 2 (mod 4) start one wave later. A causal group has
// qg + 1 blocks, so its one to three blocks past a multiple of ANW land on waves {0} (qg = 0),
// {0, 1} (qg = 1) and {1, 2, 3} (qg = 2), qg taken mod 4: the two groups of a causal pair (qg + qg' =
// nqg - 1) then leave exactly one wave with a block more than the others, where dealing every
// group from wave 0 gives two waves one more and one wave one less whenever the pair's groups
// are 1 and 2 (mod 4). The rule depends on the group alone, so a query's keys are split among
// the waves the same way whatever n_ctx is (causal prefixes stay bit-identical).
static_assert((ANW & (ANW - 1)) == 0, "ANW a power of two");
__device__ __forceinline__ int first_block(int wave, int qg) {
    return (wave - (qg % 4 == 2 ? 1 : 0)) & (ANW - 1);
}

// S^T = K Q'^T for one block of 32 keys: lane (half, l31) gets 16 scores of query l31, register r
// holding key 8*(r/4) + 4*half + r%4 of the block
template <int D>
__device__ __forceinline__ f32x16 block_scores(const float (&kf)[D / 2], const float (&qf)[D / 2]) {
    f32x16 st;
#pragma unroll
    for (int r = 0; r < 16; r++) st[r] = 0.f;
#pragma unroll
    for (int s = 0; s < D / 2; s++) st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[s], qf[s], st, 0, 0, 0);
    return st;
}

// The two halves of a wave hold the two halves of a query's keys. v_permlane32_swap of a value
// with itself leaves the low half's values in every lane of one result and the high half's in
// every lane of the other: a VALU exchange, no LDS round trip. max and + are commutative, so
// every lane gets the value fmaxf(x, __shfl_xor(x, 32)) or x + __shfl_xor(x, 32) would give it.
__device__ __forceinline__ float halves_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// keys past n_ctx, and under causal masking keys after the query, score -inf; only blocks that
// can hold such a key pay for the test
__device__ __forceinline__ void mask_scores(f32x16 &st, int key0, int n_ctx, int causal, int q0, int qi, int half) {
    if (key0 + ABN > n_ctx || (causal && key0 + ABN - 1 > q0)) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = key0 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (key >= n_ctx || (causal && key > qi)) st[r] = -INFINITY;
        }
    }
}

// Online softmax with a lazily moved reference: each query keeps a reference maximum m_i (log2
// units) and moves it only when a block's scores exceed it by more than kSlack. Then
// p = 2^(s - m_i) <= 2^kSlack (no overflow: l stays below 2^kSlack times the key count), and O
// and l are rescaled only on the rare blocks that move some query's reference, instead of on
// every block. The quotient O / l is the same mathematically; rounding differs by a few ulp.
// Turns st into p in place.
constexpr float kSlack = 8.f;

template <int D>
__device__ __forceinline__ float online_rescale(const f32x16 &st, float &m_i, float &l_i, f32x16 (&o)[D / 32]) {
    float mloc = st[0];
#pragma unroll
    for (int r = 1; r < 16; r++) mloc = fmaxf(mloc, st[r]);
    mloc = halves_max(mloc);                // the other half of the wave holds the query's other keys
    const bool move = mloc > m_i + kSlack;  // m_i = -inf: moves on the first visible score
    if (__any(move)) {
        const float m_new = move ? mloc : m_i;
        const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);  // 0 from -inf, 1 if not moved
#pragma unroll
        for (int b = 0; b < D / 32; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[b][r] *= alpha;
        l_i *= alpha;
        m_i = m_new;
    }
    return m_i == -INFINITY ? 0.f : m_i;  // nothing visible yet: every p is 0
}

// p = 2^(s - mref) in place; their sum over the query's 32 keys joins l
__device__ __forceinline__ void online_exp(f32x16 &st, float mref, float &l_i) {
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        st[r] = __builtin_amdgcn_exp2f(st[r] - mref);
        lsum += st[r];
    }
    l_i += halves_sum(lsum);
}

template <int D>
__device__ __forceinline__ void online_update(f32x16 &st, float &m_i, float &l_i, f32x16 (&o)[D / 32]) {
    online_exp(st, online_rescale<D>(st, m_i, l_i, o), l_i);
}

// O^T += V^T P^T from the wave's V slab (vw[key][dim]): step s pairs key (s/4)*8 + 4*half + s%4
// with dim b*32 + l31, and its B operand is the lane's own p register s
template <int D>
__device__ __forceinline__ void block_pv(f32x16 (&o)[D / 32], const f32x16 &p, const float (*vw)[D], int half, int l31) {
#pragma unroll
    for (int b = 0; b < D / 32; b++)
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const float a = vw[(s >> 2) * 8 + 4 * half + (s & 3)][b * 32 + l31];
            o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, p[s], o[b], 0, 0, 0);
        }
}

// Merges the ANW partial states of the group: waves 1.. hand (m, l, O) over LDS (same lane =
// same query and output element), wave 0 combines and stores row qi of the output.
template <int D>
__device__ __forceinline__ void merge_store(float *lds, const f32x16 (&o)[D / 32], float m_i, float l_i, float *op,
                                            bool row_ok, int head_dim) {
    float(*xo)[D / 2][64] = reinterpret_cast<float(*)[D / 2][64]>(lds);
    float(*xm)[2][64] = reinterpret_cast<float(*)[2][64]>(lds + (ANW - 1) * (D / 2) * 64);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5;
    __syncthreads();  // every wave is done with its V slab
    if (wave > 0) {
#pragma unroll
        for (int b = 0; b < D / 32; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) xo[wave - 1][b * 16 + r][lane] = o[b][r];
        xm[wave - 1][0][lane] = m_i;
        xm[wave - 1][1][lane] = l_i;
    }
    __syncthreads();
    if (wave == 0 && row_ok) {
        float m = m_i;
#pragma unroll
        for (int w = 0; w < ANW - 1; w++) m = fmaxf(m, xm[w][0][lane]);
        const float mu = m == -INFINITY ? 0.f : m;
        const float c0 = __builtin_amdgcn_exp2f(m_i - mu);
        float cw[ANW - 1];
        float l = l_i * c0;
#pragma unroll
        for (int w = 0; w < ANW - 1; w++) {
            cw[w] = __builtin_amdgcn_exp2f(xm[w][0][lane] - mu);
            l = __builtin_fmaf(xm[w][1][lane], cw[w], l);
        }
        const float inv = 1.0f / l;
#pragma unroll
        for (int b = 0; b < D / 32; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int d = b * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                float acc = o[b][r] * c0;
#pragma unroll
                for (int w = 0; w < ANW - 1; w++) acc = __builtin_fmaf(xo[w][b * 16 + r][lane], cw[w], acc);
                if (d < head_dim) op[d] = acc * inv;
            }
    }
}

// The general kernel: any head_dim <= D, any strides (K also pre-transposed), guarded loads.
// A wave computes a 32-query group against key blocks first_block(w, qg), + ANW, ...:
//   S^T = K Q'^T   A: K half rows, B: Q' half rows held for the whole kernel;
//   online softmax in the lane (lane % 32 is the query) plus one exchange with lane ^ 32;
//   O^T += V^T P^T A: V from the wave's LDS slab, B: the lane's own p registers.
template <int D, int KL>
__global__ __launch_bounds__(64 * ANW) __attribute__((amdgpu_waves_per_eu(D <= 64 ? PITON_ATTN_WAVES_PER_EU : 1)))
void attn_fwd_kernel_f32(AttnArgs g) {
    __shared__ float vslab[ANW][ABN][D];  // per-wave V staging; reused for the merge
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, half = lane >> 5, l31 = lane & 31;
    int64_t bh;
    int qg;
    map_group(g, bh, qg);
    const int64_t bi = bh / g.n_heads, h = bh % g.n_heads;
    const int64_t q0 = (int64_t)qg * AQG;
    const int64_t qi = q0 + l31;  // this lane's query

    const float *qp = g.q + bi * g.s_qb + h * g.s_qh;
    const float *kbase = g.k + bi * g.s_kb + h * g.s_kh;
    const float *vbase = g.v + bi * g.s_vb + h * g.s_vh;

    // Q'^T operand: the lane's half row of its query, scaled by sm_scale * log2 e
    float qf[D / 2];
    {
        const int d0 = half * (D / 2);
        const bool ok = qi < g.n_ctx;
        if (g.q_vec) {
#pragma unroll
            for (int c = 0; c < D / 8; c++) {
                float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
                if (ok && d0 + 4 * c < g.head_dim) f = *reinterpret_cast<const float4 *>(qp + qi * g.s_qm + d0 + 4 * c);
                qf[4 * c] = f.x * g.scale; qf[4 * c + 1] = f.y * g.scale;
                qf[4 * c + 2] = f.z * g.scale; qf[4 * c + 3] = f.w * g.scale;
            }
        } else {
#pragma unroll
            for (int s = 0; s < D / 2; s++)
                qf[s] = (ok && d0 + s < g.head_dim) ? qp[qi * g.s_qm + d0 + s] * g.scale : 0.f;
        }
    }

    f32x16 o[D / 32];
#pragma unroll
    for (int b = 0; b < D / 32; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[b][r] = 0.f;
    float m_i = -INFINITY, l_i = 0.f;

    const int n_ctx = (int)g.n_ctx, qi32 = (int)qi;  // fit 32 bits (checked on the host)
    const int nkb_all = (n_ctx + ABN - 1) / ABN;
    const int nkb = g.causal ? min(nkb_all, qg + 1) : nkb_all;

    float(*vw)[D] = reinterpret_cast<float(*)[D]>(&vslab[wave][0][0]);
    constexpr int NVQ = ABN * D / 4 / 64;  // float4 chunks of a V block per lane
    auto load_v = [&](int key0, float4 (&vr)[NVQ]) {
        const bool full = key0 + ABN <= n_ctx && D == g.head_dim && g.v_vec;
#pragma unroll
        for (int c = 0; c < NVQ; c++) {
            const int idx = lane + 64 * c, key = idx / (D / 4), dq = idx % (D / 4);
            if (full) {
                vr[c] = *reinterpret_cast<const float4 *>(vbase + (int64_t)(key0 + key) * g.s_vn + 4 * dq);
            } else {
                float e[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int d = 4 * dq + j;
                    e[j] = (key0 + key < n_ctx && d < g.head_dim) ? vbase[(int64_t)(key0 + key) * g.s_vn + d] : 0.f;
                }
                vr[c] = make_float4(e[0], e[1], e[2], e[3]);
            }
        }
    };
    auto stage_v = [&](const float4 (&vr)[NVQ]) {
#pragma unroll
        for (int c = 0; c < NVQ; c++) {
            const int idx = lane + 64 * c;
            *reinterpret_cast<f32x4 *>(&vw[idx / (D / 4)][4 * (idx % (D / 4))]) =
                f32x4{vr[c].x, vr[c].y, vr[c].z, vr[c].w};
        }
    };
    auto process = [&](int kb, const float (&kf)[D / 2]) {
        const int key0 = kb * ABN;
        float4 vr[NVQ];
        if constexpr (D <= 64) load_v(key0, vr);  // in flight during the score product
        f32x16 st = block_scores<D>(kf, qf);
        if constexpr (D > 64) load_v(key0, vr);  // after it: Q, K, O and S already fill the registers
        mask_scores(st, key0, n_ctx, g.causal, (int)q0, qi32, half);
        online_update<D>(st, m_i, l_i, o);
        wave_lds_sync();  // the previous block's operand reads are done with the slab
        stage_v(vr);
        wave_lds_sync();  // rows staged by other lanes are visible to the operand reads
        block_pv<D>(o, st, vw, half, l31);
    };

    int kb = first_block(wave, qg);
    if constexpr (D <= 64) {
        // two K stages, unrolled by two so neither is copied: block kb + ANW's K loads while kb
        // is multiplied
        float kf0[D / 2], kf1[D / 2];
        if (kb < nkb) load_k_operand<D, KL>(g, kbase, kb * ABN + l31, half, kf0);
        while (kb < nkb) {
            if (kb + ANW < nkb) load_k_operand<D, KL>(g, kbase, (kb + ANW) * ABN + l31, half, kf1);
            process(kb, kf0);
            kb += ANW;
            if (kb >= nkb) break;
            if (kb + ANW < nkb) load_k_operand<D, KL>(g, kbase, (kb + ANW) * ABN + l31, half, kf0);
            process(kb, kf1);
            kb += ANW;
        }
    } else {
        // D = 128: one K stage, loaded at the top of its block, so that no phase holds more than
        // 256 values per lane
        for (; kb < nkb; kb += ANW) {
            float kf[D / 2];
            load_k_operand<D, KL>(g, kbase, kb * ABN + l31, half, kf);
            process(kb, kf);
        }
    }
    merge_store<D>(&vslab[0][0][0], o, m_i, l_i, g.o + bi * g.s_ob + h * g.s_oh + qi * g.s_om, qi < g.n_ctx,
                   g.head_dim);
}

// Raw buffer descriptor over [base, base + bytes): loads at byte offsets >= bytes return 0, so
// blocks past the end of the sequence need no guards.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f32x4 bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// The fast kernel: head_dim == D, Q / K / V / O rows contiguous and 16-byte aligned (K in
// [N, D] order), every row offset of a head within 2^31 bytes (checked on the host). Per query
// group it runs the general kernel's blocks and arithmetic (wave w takes key blocks
// first_block(w, qg), + ANW, ..., the same online softmax and the same merge formula), so the two
// agree bit for bit:
//   * Q, K and V come through buffer descriptors bounded at the head's last row. Loads past it
//     return zeros, LDS-DMA loads included, so nothing is guarded and every block, the partial
//     last one too, takes one code path (which also keeps the compiler's memory waits exact);
//   * Q' (pre-scaled) is staged once per workgroup in LDS. The paired kernel (two waves per
//     SIMD) loads a wave's B operand of the score product into 32 registers per group, so the
//     product is MFMAs alone; the single-group kernel (three waves per SIMD, no registers to
//     spare) keeps Q' transposed (qT[d][query]) and reads the operand per step, conflict-free;
//   * V blocks are copied from memory straight into the wave's LDS slab (16-byte LDS-DMA);
//   * software pipeline: block j+1's score product is issued beside block j's exps, K is loaded
//     two blocks ahead and V one block ahead; Q is requested first and the first block's K
//     right after it, so the Q staging overlaps its latency; the first V follows the barrier;
//   * PAIR (causal): the workgroup runs query group nqg-1-p, then group p, so each workgroup
//     visits nqg + 1 key blocks. A wave parks its first group's state in registers and the
//     pipeline runs on into the second group without a barrier; both merge at the end;
//   * the merge is spread over the four waves, each finishing a quarter of every output row.
#ifndef PITON_ATTN_FAST_WAVES
#define PITON_ATTN_FAST_WAVES 3
#endif
// causal query groups in pairs: 0 never, 1 always, 2 when the pairs fill at most two
// workgroups per CU (one generation)
#ifndef PITON_ATTN_PAIR_MODE
#define PITON_ATTN_PAIR_MODE 2
#endif

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// The Q' tile of a query group in LDS: q2[j][d] = Q'[query j][d], the 16-byte chunks of row j
// stored XOR-swizzled (chunk c at c ^ (j % (D/4))): the staging writes (a row's chunks from
// consecutive lanes) and the operand reads (chunk c of 32 rows) fall on distinct banks.
template <int D>
__device__ __forceinline__ int q2_col(int j, int c) {
    return (c ^ (j % (D / 4))) * 4;
}

// A lane's B operand of the score product, Q'[l31][half * D/2 + s] for s = 0 .. D/2-1 (the
// contraction order of block_scores), read from the swizzled tile
template <int D>
__device__ __forceinline__ void load_q_operand(float (&qf)[D / 2], const float (*q2)[D], int half, int l31) {
#pragma unroll
    for (int c = 0; c < D / 8; c++) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(&q2[l31][q2_col<D>(l31, half * (D / 8) + c)]);
#pragma unroll
        for (int e = 0; e < 4; e++) qf[4 * c + e] = v[e];
    }
}

// block_scores with the B operand read from a transposed tile qT[d][query] (for kernels without
// the registers to hold it): lane l31 of a step reads consecutive words, one immediate offset
// per step from a single address
template <int D>
__device__ __forceinline__ f32x16 block_scores_lds(const float (&kf)[D / 2], const float (*qT)[AQG], int half,
                                                   int l31) {
    f32x16 st;
#pragma unroll
    for (int r = 0; r < 16; r++) st[r] = 0.f;
#pragma unroll
    for (int s = 0; s < D / 2; s++)
        st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[s], qT[half * (D / 2) + s][l31], st, 0, 0, 0);
    return st;
}

// Causal pairs: workgroup -> (batch*head, pair rank p), whole heads per XCD as in map_group.
__device__ __forceinline__ void map_pair(const AttnArgs &g, int64_t &bh, int &prank) {
    const int npair = (g.nqg + 1) / 2, nbh = g.nbh;
    if (nbh % kXcdCount == 0) {
        const int xcd = blockIdx.x % kXcdCount, i = blockIdx.x / kXcdCount, per = nbh / kXcdCount;
        bh = (int64_t)xcd * per + i % per;
        prank = i / per;
    } else {
        bh = blockIdx.x / npair;
        prank = blockIdx.x % npair;
    }
}

// One query group's merge from the ANW wave states in LDS (xo[w][slot][lane] with slot
// b*16 + r for o[b][r], xm[w][0|1][lane] = m, l): merge_store's arithmetic (wave 0's state
// first, then waves 1.. in order, each added by a written-out fused multiply-add, so no kernel's
// result depends on which product of a*b + c*d the compiler would fuse), wave w finishing slots
// [w*D/8, (w+1)*D/8) of every lane, four consecutive dims per float4 store.
template <int D>
__device__ __forceinline__ void merge_quarter(const float (*xo)[D / 2][64], const float (*xm)[2][64], float *op,
                                              bool row_ok) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5;
    float m = xm[0][0][lane];
#pragma unroll
    for (int w = 1; w < ANW; w++) m = fmaxf(m, xm[w][0][lane]);
    const float mu = m == -INFINITY ? 0.f : m;
    const float c0 = __builtin_amdgcn_exp2f(xm[0][0][lane] - mu);
    float cw[ANW - 1];
    float l = xm[0][1][lane] * c0;
#pragma unroll
    for (int w = 1; w < ANW; w++) {
        cw[w - 1] = __builtin_amdgcn_exp2f(xm[w][0][lane] - mu);
        l = __builtin_fmaf(xm[w][1][lane], cw[w - 1], l);
    }
    const float inv = 1.0f / l;
    if (!row_ok) return;
    constexpr int SPW = D / 2 / ANW;
#pragma unroll
    for (int i = 0; i < SPW; i += 4) {
        const int s0 = wave * SPW + i, b = s0 >> 4, r = s0 & 15;
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float acc = xo[0][s0 + e][lane] * c0;
#pragma unroll
            for (int w = 1; w < ANW; w++) acc = __builtin_fmaf(xo[w][s0 + e][lane], cw[w - 1], acc);
            v[e] = acc * inv;
        }
        *reinterpret_cast<f32x4 *>(op + b * 32 + 8 * (r >> 2) + 4 * half) = v;
    }
}

template <int D, bool PAIR>
__global__ __launch_bounds__(64 * ANW) __attribute__((amdgpu_waves_per_eu(PAIR ? 2 : PITON_ATTN_FAST_WAVES)))
void attn_fwd_fast(AttnArgs g) {
    constexpr int NG = PAIR ? 2 : 1;
    // Two LDS objects. The V slabs (written by LDS-DMA) and the Q tiles are distinct variables,
    // so the compiler's wait-count pass can tell the Q reads of a score product from the V
    // copies in flight and does not make them wait for those copies. The merge reuses both: each
    // wave's O rows in the first, its (m, l) in the second.
    constexpr int SLAB_F = ANW * ABN * D, XO_F = NG * ANW * (D / 2) * 64;
    constexpr int QT_F = NG * D * AQG, XM_F = NG * ANW * 2 * 64;
    __shared__ __attribute__((aligned(16))) float lds_v[SLAB_F > XO_F ? SLAB_F : XO_F];
    __shared__ __attribute__((aligned(16))) float lds_q[QT_F > XM_F ? QT_F : XM_F];
    static_assert(!PAIR || sizeof(lds_v) + sizeof(lds_q) <= 80 * 1024, "two paired workgroups share a CU's 160 KB");
    float(*vslab)[ABN][D] = reinterpret_cast<float(*)[ABN][D]>(lds_v);
    // the Q' tiles: row-major and swizzled (q2) when the operand is loaded into registers once
    // per group, transposed (qT) when every score product reads it
    constexpr bool QREG = PAIR || PITON_ATTN_FAST_WAVES <= 2;
    float(*q2)[AQG][D] = reinterpret_cast<float(*)[AQG][D]>(lds_q);
    float(*qT)[D][AQG] = reinterpret_cast<float(*)[D][AQG]>(lds_q);

    const int t = threadIdx.x, lane = t & 63, half = lane >> 5, l31 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    PITON_PHASE_VARS;
    PITON_PHASE(0);
    int64_t bh;
    int qg0, qg1 = 0, ng = 1;
    if constexpr (PAIR) {
        int p;
        map_pair(g, bh, p);
        qg0 = g.nqg - 1 - p;
        qg1 = p;
        ng = p != qg0 ? 2 : 1;
    } else {
        map_group(g, bh, qg0);
    }
    const int64_t bi = bh / g.n_heads, h = bh % g.n_heads;
    const int n_ctx = (int)g.n_ctx;
    const uint32_t s_qm = (uint32_t)g.s_qm, s_kn = (uint32_t)g.s_kn, s_vn = (uint32_t)g.s_vn;
    const auto rq = make_rsrc(g.q + bi * g.s_qb + h * g.s_qh, ((uint32_t)(n_ctx - 1) * s_qm + D) * 4u);
    const auto rk = make_rsrc(g.k + bi * g.s_kb + h * g.s_kh, ((uint32_t)(n_ctx - 1) * s_kn + D) * 4u);
    const auto rv = make_rsrc(g.v + bi * g.s_vb + h * g.s_vh, ((uint32_t)(n_ctx - 1) * s_vn + D) * 4u);

    // this wave's blocks: list index j < n0 is block f0 + ANW*j of the first group, j >= n0
    // block f1 + ANW*(j - n0) of the second (the heavier group comes first)
    const int nkb_all = (n_ctx + ABN - 1) / ABN;
    const int nkb0 = g.causal ? min(nkb_all, qg0 + 1) : nkb_all, nkb1 = min(nkb_all, qg1 + 1);
    const int f0 = first_block(wave, qg0), f1 = first_block(wave, qg1);
    const int n0 = nkb0 > f0 ? (nkb0 - f0 + ANW - 1) / ANW : 0;
    const int n1 = (PAIR && ng > 1 && nkb1 > f1) ? (nkb1 - f1 + ANW - 1) / ANW : 0;
    const int n = n0 + n1;
    auto kb_of = [&](int j) { return j < n0 ? f0 + ANW * j : f1 + ANW * (j - n0); };

    // byte offsets: K half row of key kb*32 + l31; V chunk c of block kb at v_lane + kb*v_blk + c*v_c
    constexpr int KPC = 64 / (D / 4);  // V keys per float4 chunk step of the lane
    constexpr int NVQ = ABN * D / 4 / 64;
    constexpr int K_LOADS = D / 8;  // 16-byte loads of load_k: one lane-half row of the block
    static_assert(K_LOADS <= 63 && NVQ <= 63, "loads per block within the vmcnt range");
    const uint32_t k_lane = ((uint32_t)l31 * s_kn + half * (D / 2)) * 4u, k_blk = (uint32_t)ABN * s_kn * 4u;
    const uint32_t v_lane = ((uint32_t)(lane / (D / 4)) * s_vn + 4 * (lane % (D / 4))) * 4u;
    const uint32_t v_blk = (uint32_t)ABN * s_vn * 4u, v_c = (uint32_t)KPC * s_vn * 4u;
    float(*vw)[D] = vslab[wave];
    auto load_k = [&](float (&kf)[D / 2], int kb) {
        const uint32_t off = k_lane + (uint32_t)kb * k_blk;
#pragma unroll
        for (int c = 0; c < D / 8; c++) {
            const f32x4 f = bload4(rk, off + 16u * c);
#pragma unroll
            for (int j = 0; j < 4; j++) kf[4 * c + j] = f[j];
        }
    };
    // V of block kb into the slab by LDS-DMA: lane l's 16 bytes of chunk c land at row
    // KPC*c + l / (D/4), dims 4*(l % (D/4)) (the slab's row-major layout); rows past n_ctx
    // arrive as zeros
    auto fetch_v = [&](int kb) {
        const uint32_t off = v_lane + (uint32_t)kb * v_blk;
#pragma unroll
        for (int c = 0; c < NVQ; c++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)&vw[KPC * c][0], 16, off + v_c * c, 0, 0, 0);
    };

    // Q' of the groups: q2[gi][j][d] = qT[gi][d][j] = Q[qg_gi*AQG + j][d] * sm_scale * log2 e
    // (rows past n_ctx: 0). Every Q chunk is requested first, then the first block's K: the memory counter
    // is in order, so the Q writes wait for Q alone while K is still in flight. Every wave
    // requests a first K block (one without blocks requests block `wave`, never used).
    constexpr int QIT = NG * AQG * D / 4 / (64 * ANW);
    static_assert(NG * AQG * D / 4 % (64 * ANW) == 0, "whole Q chunks per thread");
    auto q_chunk = [&](int c, int &gi, int &j, int &dq) {
        const int i = t + 64 * ANW * c, r = i % (AQG * D / 4);
        gi = i / (AQG * D / 4);
        j = r / (D / 4);
        dq = r % (D / 4);
    };
    float kf[D / 2];
    f32x4 qv[QIT];
#pragma unroll
    for (int c = 0; c < QIT; c++) {
        int gi, j, dq;
        q_chunk(c, gi, j, dq);
        qv[c] = bload4(rq, ((uint32_t)((gi ? qg1 : qg0) * AQG + j) * s_qm + 4 * dq) * 4u);
    }
    load_k(kf, kb_of(0));
#pragma unroll
    for (int c = 0; c < QIT; c++) {
        int gi, j, dq;
        q_chunk(c, gi, j, dq);
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; e++) w[e] = qv[c][e] * g.scale;
        if constexpr (QREG) {
            *reinterpret_cast<f32x4 *>(&q2[gi][j][q2_col<D>(j, dq)]) = w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) qT[gi][4 * dq + e][j] = w[e];
        }
    }
    // the other waves need the Q tiles only: wait for this wave's LDS writes and meet at the
    // barrier, without the release fence of __syncthreads, whose wait covers every memory
    // operation in flight (the first block's K, which only this wave reads, included); the
    // empty asm with a memory clobber keeps the compiler from moving a Q store below the barrier
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitcntLgkm0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
    PITON_PHASE(1);

    f32x16 o[D / 32], po[D / 32];  // the running state and (PAIR) the parked first group's
#pragma unroll
    for (int b = 0; b < D / 32; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[b][r] = po[b][r] = 0.f;
    float m_i = -INFINITY, l_i = 0.f, pm = -INFINITY, pl = 0.f;

    if (n > 0) {
        // the current group's Q' operand, in registers where the occupancy leaves room for it
        float qf[D / 2];
        // (a wave can hold no block of the first group and some of the second)
        if constexpr (QREG) load_q_operand<D>(qf, q2[PAIR && n0 == 0 ? 1 : 0], half, l31);
        auto scores = [&]() { return QREG ? block_scores<D>(kf, qf) : block_scores_lds<D>(kf, qT[0], half, l31); };
        f32x16 st = scores();
        // Every pass of the loop starts with block j+1's K in flight ahead of block j's V, so
        // the wait for that K lets the newer V copies stay in flight. Block 0's V is therefore
        // requested after block 1's K: issued before it (as soon as Q is staged), the compiler
        // merges the two orders at the loop head, assumes the V copies are the older loads in
        // every pass and waits for them at the next block's score product.
        load_k(kf, kb_of(1));  // past the list it reads a block nobody uses (or zeros)
        __builtin_amdgcn_sched_barrier(0);
        fetch_v(kb_of(0));
        __builtin_amdgcn_sched_barrier(0);
        auto step = [&](int j, auto has_next) {
            constexpr bool NEXT = decltype(has_next)::value;
            const int q0 = (PAIR && j >= n0 ? qg1 : qg0) * AQG;
            mask_scores(st, kb_of(j) * ABN, n_ctx, g.causal, q0, q0 + l31, half);
            const float mref = online_rescale<D>(st, m_i, l_i, o);
            f32x16 st_next;
            if constexpr (NEXT) {
                if (PAIR && j + 1 == n0) load_q_operand<D>(qf, q2[1], half, l31);  // j+1 opens group 2
                st_next = scores();
            }
            online_exp(st, mref, l_i);
            if constexpr (NEXT) load_k(kf, kb_of(j + 2));
            // block j's V is in the slab once at most the K loads just issued (D / 8 of them) are
            // in flight (vmcnt counts in issue order; the scheduling barriers keep that order)
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(NEXT ? waitcnt_vm(K_LOADS) : waitcnt_vm(0));
            __builtin_amdgcn_sched_barrier(0);
            wave_lds_sync();  // rows written for other lanes are visible to the operand reads
            block_pv<D>(o, st, vw, half, l31);
            if constexpr (NEXT) {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_waitcnt(kWaitcntLgkm0);  // the operand reads have their data
                __builtin_amdgcn_sched_barrier(0);
                wave_lds_sync();
                fetch_v(kb_of(j + 1));
                st = st_next;
                if (PAIR && j + 1 == n0) {  // the next block opens the second group
#pragma unroll
                    for (int b = 0; b < D / 32; b++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            po[b][r] = o[b][r];
                            o[b][r] = 0.f;
                        }
                    pm = m_i;
                    pl = l_i;
                    m_i = -INFINITY;
                    l_i = 0.f;
                }
            }
        };
        int j = 0;
        for (; j + 1 < n; j++) step(j, std::true_type{});
        step(j, std::false_type{});
    }

    // merge: every wave's state of every group into LDS, then each wave a quarter of the rows
    auto xo_of = [&](int gi) { return reinterpret_cast<float(*)[D / 2][64]>(lds_v + gi * ANW * (D / 2) * 64); };
    auto xm_of = [&](int gi) { return reinterpret_cast<float(*)[2][64]>(lds_q + gi * ANW * 2 * 64); };
    auto put = [&](int gi, const f32x16 (&so)[D / 32], float sm, float sl) {
        float(*xo)[D / 2][64] = xo_of(gi);
        float(*xm)[2][64] = xm_of(gi);
#pragma unroll
        for (int b = 0; b < D / 32; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) xo[wave][b * 16 + r][lane] = so[b][r];
        xm[wave][0][lane] = sm;
        xm[wave][1][lane] = sl;
    };
    PITON_PHASE(2);
    // every V copy into the slabs has landed before the LDS is reused for the merge
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();  // every wave is done with its slab and the Q tiles
    const bool second = PAIR && n1 > 0;  // the running state is the second group's
    put(second ? 1 : 0, o, m_i, l_i);
    if (PAIR && ng > 1) put(second ? 0 : 1, po, pm, pl);
    __syncthreads();
    for (int gi = 0; gi < ng; gi++) {
        const int qi = (gi ? qg1 : qg0) * AQG + l31;
        merge_quarter<D>(xo_of(gi), xm_of(gi),
                         g.o + bi * g.s_ob + h * g.s_oh + (int64_t)qi * g.s_om, qi < n_ctx);
    }
    PITON_PHASE(3);
    PITON_PHASE_END(kPhaseAttnFast, g.phase);
}

template <int D>
static void launch_d(int kl, const AttnArgs &g, dim3 grid, hipStream_t st) {
    if (kl == K_VEC_D) PITON_LAUNCH((attn_fwd_kernel_f32<D, K_VEC_D>), grid, dim3(64 * ANW), 0, st, g);
    else PITON_LAUNCH((attn_fwd_kernel_f32<D, K_SCALAR>), grid, dim3(64 * ANW), 0, st, g);
}

// One new query per (batch, head) against keys 0 .. n_keys-1 of a cache (the decode step of a
// KV-cached decoder): one 256-thread workgroup per (batch, head).
//   * scores: D/16 consecutive lanes share a key, 16 head dims each (four float4 loads of the
//     key row), and add their partial dot products with lane exchanges; the scores go to LDS;
//   * the maximum and the sum of exps over the keys reduce across the workgroup (DPP within a
//     wave, then the four wave results through LDS);
//   * P V: thread (g, d) sums p_j V[j][d] over the keys j = g mod 256/D with coalesced V rows;
//     the 256/D partial sums of a dim add in a fixed order.
constexpr int kMaxDecodeKeys = 8192;

struct DecodeArgs {
    const float *q, *k, *v;
    float *o;
    float scale;  // sm_scale * log2(e)
    int64_t s_qb, s_qh, s_kb, s_kh, s_kn, s_vb, s_vh, s_vn, s_ob, s_oh;
    int n_keys, n_heads, head_dim;
    PhaseRecord *phase;  // the launch's phase-trace records (diagnostics builds; null otherwise)
};

// Holds the arguments read after the scores (the scale, the output and its strides) in scalar
// registers from the start: the compiler would otherwise load them from the kernarg segment
// where they are first used, one more memory round trip on the critical path.
__device__ __forceinline__ void keep_decode_args(DecodeArgs &g) {
    g.scale = sgpr_keep(g.scale);
    g.o = sgpr_keep(g.o);
    g.s_ob = sgpr_keep(g.s_ob);
    g.s_oh = sgpr_keep(g.s_oh);
}

template <class Op>
__device__ __forceinline__ float block_reduce4(float v, Op op, float *red) {
    v = wave_reduce(v, op);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return op(op(red[0], red[1]), op(red[2], red[3]));
}

template <int D, bool VEC>
__global__ __launch_bounds__(256) void attn_decode_kernel(DecodeArgs g) {
    keep_decode_args(g);
    __shared__ float p[kMaxDecodeKeys];
    __shared__ float red[8];
    __shared__ float part[256];
    constexpr int TPK = D / 16, KPP = 256 / TPK, KG = 256 / D;
    const int t = threadIdx.x;
    const int64_t bh = blockIdx.x, b = bh / g.n_heads, h = bh % g.n_heads;
    const float *qp = g.q + b * g.s_qb + h * g.s_qh;
    const float *kp = g.k + b * g.s_kb + h * g.s_kh;
    const float *vp = g.v + b * g.s_vb + h * g.s_vh;
    const int n_keys = g.n_keys, head_dim = g.head_dim;

    // this lane's 16 dims of the query (scaled), and of each key it scores
    const int sub = t % TPK, kslot = t / TPK, d0 = 16 * sub;
    const bool dims_ok = d0 < head_dim;  // head_dim is a multiple of 16
    float q16[16];
#pragma unroll
    for (int i = 0; i < 16; i++) q16[i] = dims_ok ? qp[d0 + i] * g.scale : 0.f;
    float mloc = -INFINITY;
    for (int j0 = 0; j0 < n_keys; j0 += KPP) {
        const int j = j0 + kslot;
        float sc = 0.f;
        if (j < n_keys && dims_ok) {
            const float *kr = kp + (int64_t)j * g.s_kn + d0;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                float4 f;
                if constexpr (VEC) f = *reinterpret_cast<const float4 *>(kr + 4 * c);
                else f = make_float4(kr[4 * c], kr[4 * c + 1], kr[4 * c + 2], kr[4 * c + 3]);
                sc = fmaf(q16[4 * c], f.x, sc);
                sc = fmaf(q16[4 * c + 1], f.y, sc);
                sc = fmaf(q16[4 * c + 2], f.z, sc);
                sc = fmaf(q16[4 * c + 3], f.w, sc);
            }
        }
#pragma unroll
        for (int o = 1; o < TPK; o <<= 1) sc += __shfl_xor(sc, o);  // the key's TPK lanes are consecutive
        if (j < n_keys) {
            if (sub == 0) p[j] = sc;
            mloc = fmaxf(mloc, sc);
        }
    }
    const float m = block_reduce4(mloc, MaxOp(), red);  // its barrier also publishes the scores
    float lsum = 0.f;
    for (int j = t; j < n_keys; j += 256) {
        const float e = __builtin_amdgcn_exp2f(p[j] - m);
        p[j] = e;
        lsum += e;
    }
    const float inv = 1.0f / block_reduce4(lsum, SumOp(), red + 4);  // and publishes the exps

    const int d = t % D, kg = t / D;
    float acc = 0.f;
    if (d < head_dim) {
        const float *vc = vp + d;
#pragma unroll 4
        for (int j = kg; j < n_keys; j += KG) acc = fmaf(p[j], vc[(int64_t)j * g.s_vn], acc);
    }
    part[t] = acc;
    __syncthreads();
    if (t < D && t < head_dim) {
        float v = part[t];
#pragma unroll
        for (int w = 1; w < KG; w++) v += part[w * D + t];
        g.o[b * g.s_ob + h * g.s_oh + t] = v * inv;
    }
}

// Short caches (n_keys <= 256, head_dim <= 64: a decoder with a small context): the same
// arithmetic in the same order as attn_decode_kernel, so the two give identical bits, but every
// K and V element the workgroup needs is requested before any of it is used: one memory round
// trip instead of one per key chunk plus a chain of V loads behind the softmax.
constexpr int kShortDecodeKeys = 256;
#ifndef PITON_DECODE_SHORT
#define PITON_DECODE_SHORT 1
#endif

template <int D, bool VEC>
__global__ __launch_bounds__(256) void attn_decode_short(DecodeArgs g) {
    keep_decode_args(g);
    static_assert(D <= 64, "short decode holds K and V in registers for head_dim <= 64");
    __shared__ float p[kShortDecodeKeys];
    __shared__ float red[8];
    __shared__ float part[256];
    constexpr int TPK = D / 16, KPP = 256 / TPK, KG = 256 / D;
    constexpr int NIT = kShortDecodeKeys / KPP, NV = kShortDecodeKeys / KG;
    const int t = threadIdx.x;
    const int64_t bh = blockIdx.x, b = bh / g.n_heads, h = bh % g.n_heads;
    const float *qp = g.q + b * g.s_qb + h * g.s_qh;
    const float *kp = g.k + b * g.s_kb + h * g.s_kh;
    const float *vp = g.v + b * g.s_vb + h * g.s_vh;
    const int n_keys = g.n_keys, head_dim = g.head_dim;
    const int sub = t % TPK, kslot = t / TPK, d0 = 16 * sub;
    const bool dims_ok = d0 < head_dim;
    const int d = t % D, kg = t / D;
    const bool d_ok = d < head_dim;
    PITON_PHASE_VARS;
    PITON_PHASE(0);

    f32x4 kv[NIT][4];
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int j = it * KPP + kslot;
        const float *kr = kp + (int64_t)j * g.s_kn + d0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            f32x4 f = {0.f, 0.f, 0.f, 0.f};
            if (j < n_keys && dims_ok) {
                if constexpr (VEC) f = *reinterpret_cast<const f32x4 *>(kr + 4 * c);
                else f = f32x4{kr[4 * c], kr[4 * c + 1], kr[4 * c + 2], kr[4 * c + 3]};
            }
            kv[it][c] = f;
        }
    }
    // V through a descriptor bounded at the last key's row: rows past it read as zeros, so the
    // loads need no per-key predicate. The whole offset is the per-lane one (the descriptor's
    // range check does not cover `soffset`); the host checks it fits 31 bits.
    const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(vp), (short)0,
                                                      (int)(((int64_t)(n_keys - 1) * g.s_vn + head_dim) * 4), 0x00020000);
    const int vo = (int)((d + (int64_t)kg * g.s_vn) * 4), vstep = (int)(KG * g.s_vn * 4);
    float vv[NV];
#pragma unroll
    for (int i = 0; i < NV; i++)
        vv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, vo + i * vstep, 0, 0));
    float q16[16];
#pragma unroll
    for (int i = 0; i < 16; i++) q16[i] = dims_ok ? qp[d0 + i] * g.scale : 0.f;

    PITON_PHASE_WAIT_LOADS();
    PITON_PHASE(1);
    float mloc = -INFINITY;
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int j = it * KPP + kslot;
        float sc = 0.f;
        if (j < n_keys && dims_ok) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                sc = fmaf(q16[4 * c], kv[it][c][0], sc);
                sc = fmaf(q16[4 * c + 1], kv[it][c][1], sc);
                sc = fmaf(q16[4 * c + 2], kv[it][c][2], sc);
                sc = fmaf(q16[4 * c + 3], kv[it][c][3], sc);
            }
        }
#pragma unroll
        for (int o = 1; o < TPK; o <<= 1) sc += __shfl_xor(sc, o);
        if (j < n_keys) {
            if (sub == 0) p[j] = sc;
            mloc = fmaxf(mloc, sc);
        }
    }
    for (int j = n_keys + t; j < kShortDecodeKeys; j += 256) p[j] = 0.f;  // weights of absent keys
    const float m = block_reduce4(mloc, MaxOp(), red);
    PITON_PHASE(2);
    float lsum = 0.f;
    for (int j = t; j < n_keys; j += 256) {
        const float e = __builtin_amdgcn_exp2f(p[j] - m);
        p[j] = e;
        lsum += e;
    }
    const float inv = 1.0f / block_reduce4(lsum, SumOp(), red + 4);

    // keys past n_keys add fmaf(+0, +0, acc) = acc (acc starts at +0 and never becomes -0), so
    // the sum equals attn_decode_kernel's, which skips them
    float acc = 0.f;
    if (d_ok) {
#pragma unroll
        for (int i = 0; i < NV; i++) acc = fmaf(p[kg + KG * i], vv[i], acc);
    }
    part[t] = acc;
    __syncthreads();
    if (t < D && t < head_dim) {
        float v = part[t];
#pragma unroll
        for (int w = 1; w < KG; w++) v += part[w * D + t];
        g.o[b * g.s_ob + h * g.s_oh + t] = v * inv;
    }
    PITON_PHASE(3);
    PITON_PHASE_END(kPhaseAttnDecodeShort, g.phase);
}

static int attn_launch(AttnArgs g, int64_t batch, int64_t n_heads, int32_t head_dim, hipStream_t st) {
    g.q_vec = aligned16(g.q) && g.s_qm % 4 == 0 && g.s_qh % 4 == 0 && g.s_qb % 4 == 0 && head_dim % 4 == 0;
    g.v_vec = aligned16(g.v) && g.s_vn % 4 == 0 && g.s_vh % 4 == 0 && g.s_vb % 4 == 0 && head_dim % 4 == 0;
    const int kl = (g.s_kk == 1 && g.s_kn % 4 == 0 && g.s_kh % 4 == 0 && g.s_kb % 4 == 0 && aligned16(g.k) &&
                    head_dim % 4 == 0) ? K_VEC_D : K_SCALAR;
    g.nqg = (int)((g.n_ctx + AQG - 1) / AQG);
    g.nbh = (int)(batch * n_heads);
    g.phase = phase_slot();
    dim3 grid((unsigned)((int64_t)g.nqg * g.nbh));
    // the fast kernel: exact head_dim, contiguous aligned rows that do not overlap, and every
    // byte offset it forms (rows up to n_ctx + 3 * ANW * 32, the loads a few blocks past the
    // end included) within 31 bits
    const int64_t smax = std::max(g.s_qm, std::max(g.s_kn, g.s_vn));
    const bool fast = (head_dim == 32 || head_dim == 64) && kl == K_VEC_D && g.q_vec && g.v_vec &&
                      aligned16(g.o) && g.s_om % 4 == 0 && g.s_oh % 4 == 0 && g.s_ob % 4 == 0 &&
                      g.s_qm >= head_dim && g.s_kn >= head_dim && g.s_vn >= head_dim &&
                      ((g.n_ctx + 3 * ANW * ABN + AQG) * smax + head_dim) * 4 < (1LL << 31);
    bool pair = false;
    if (fast && g.causal && g.nqg > 1) {
        const int64_t pairs = (int64_t)g.nbh * ((g.nqg + 1) / 2);
        pair = PITON_ATTN_PAIR_MODE == 1 || (PITON_ATTN_PAIR_MODE == 2 && pairs <= 2 * (int64_t)device_cu_count());
        if (pair) grid = dim3((unsigned)pairs);
    }
    if (fast && head_dim == 64) {
        if (pair) PITON_LAUNCH((attn_fwd_fast<64, true>), grid, dim3(64 * ANW), 0, st, g);
        else PITON_LAUNCH((attn_fwd_fast<64, false>), grid, dim3(64 * ANW), 0, st, g);
    } else if (fast) {
        if (pair) PITON_LAUNCH((attn_fwd_fast<32, true>), grid, dim3(64 * ANW), 0, st, g);
        else PITON_LAUNCH((attn_fwd_fast<32, false>), grid, dim3(64 * ANW), 0, st, g);
    }
    else if (head_dim <= 32) launch_d<32>(kl, g, grid, st);
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
    PITON_REQUIRE(n_ctx < (1LL << 31) - 64, PITON_EUNSUPPORTED, "attn_fwd: N_CTX %lld too large", (long long)n_ctx);
    PITON_REQUIRE(sat_mul(sat_mul(batch, n_heads), (n_ctx + 31) / 32) <= 0x7FFFFFFF, PITON_EUNSUPPORTED,
                  "attn_fwd: %lld x %lld heads x N_CTX %lld exceed one grid", (long long)batch, (long long)n_heads,
                  (long long)n_ctx);
    return PITON_OK;
}

}  // namespace piton

PITON_PHASE_TU(attention)

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
               stride_vh, stride_vn, stride_oh, stride_om, n_ctx, 0, 0, 0, 0, n_heads, head_dim, causal ? 1 : 0, 0, 0, 0, 0};
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
               head_dim, causal ? 1 : 0, 0, 0, 0, 0};
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
    PITON_REQUIRE(batch == 0 || n_heads == 0 || (q && k && v && out), PITON_EINVAL, "attn_decode: null pointer");
    PITON_REQUIRE(sat_mul(batch, n_heads) <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "attn_decode: too many heads");
    int rc = require_device();
    if (rc) return rc;
    if (batch * n_heads == 0) return PITON_OK;
    DecodeArgs g{q, k, v, out, sm_scale * 1.44269504088896341f, stride_qb, stride_qh, stride_kb, stride_kh, stride_kn,
                 stride_vb, stride_vh, stride_vn, stride_ob, stride_oh, (int)n_keys, (int)n_heads, head_dim,
                 phase_slot()};
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(batch * n_heads)), block(256);
    const bool vec = aligned16(k) && stride_kn % 4 == 0 && stride_kh % 4 == 0 && stride_kb % 4 == 0;
#define PITON_DEC(KERNEL, D)                                                                                        \
    do {                                                                                                            \
        if (vec) PITON_LAUNCH((KERNEL<D, true>), grid, block, 0, st, g);                                      \
        else PITON_LAUNCH((KERNEL<D, false>), grid, block, 0, st, g);                                         \
    } while (0)
    // short caches: every V offset the kernel forms (up to 256 rows and 64 dims) within 31 bits
    const bool short_cache = PITON_DECODE_SHORT && n_keys <= kShortDecodeKeys && stride_vn >= 0 &&
                             ((int64_t)kShortDecodeKeys * stride_vn + 64) * 4 < 0x7FFFFFFF;
    if (head_dim <= 32 && short_cache) PITON_DEC(attn_decode_short, 32);
    else if (head_dim == 64 && short_cache) PITON_DEC(attn_decode_short, 64);
    else if (head_dim <= 32) PITON_DEC(attn_decode_kernel, 32);
    else if (head_dim == 64) PITON_DEC(attn_decode_kernel, 64);
    else PITON_DEC(attn_decode_kernel, 128);
#undef PITON_DEC
    rc = check_launch("attn_decode");
    if (rc == PITON_OK) clear_error();
    return rc;
}

}  // extern "C"
