// fp32 GEMM on CDNA4 matrix cores: matmul_kernel (examples/kernels.py:18-57) and
// dense_layer_kernel (examples/nn_kernels.py:23-74).
//
// Design (gfx950):
//   * workgroup = 256 threads = 4 wavefronts in a 2x2 grid; workgroup tile 128x128, each wave
//     owns 64x64 = 2x2 blocks of v_mfma_f32_32x32x2_f32 (16 accumulators per lane per block);
//   * K advances in tiles of 32: global -> registers (prefetch of tile k+1 while tile k is
//     multiplied) -> LDS (one buffer: a barrier after the tile's reads, one after its refill;
//     33 KB of LDS lets three workgroups share a CU, which hides the barriers better than two
//     workgroups with double-buffered LDS) -> MFMA operands;
//   * LDS holds A transposed (As[k][m]) and B as is (Bs[k][n]); an MFMA operand is then 32
//     consecutive floats per half-wave (lanes 0-31 read row k, lanes 32-63 row k+1), free of
//     bank conflicts; A's row stride is odd so the transposing writes spread over the banks;
//   * each operand has three loaders chosen on the host: float4 along its contiguous
//     dimension (either orientation) when the strides and base allow 16-byte loads, else
//     scalar loads with runtime strides (the ragged / padded / odd-stride cases);
//   * rows past M and columns past N load zeros and are never stored; the K tail loads zeros,
//     so the stored elements equal sum_k A[m,k] B[k,n] exactly as the reference's masks give;
//   * tile order: workgroups renumbered so each XCD gets a contiguous run of logical ids,
//     then the reference's GROUP_SIZE_M grouping (kernels.py:28-36) on those ids.
#include <string>
#include <type_traits>

#include "common.h"

namespace piton {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 32, GTHREADS = 256;
constexpr int kStrideAT = GBM + 1;  // As[k][m]: odd row stride for the transposing writes
constexpr int kStrideB = GBN + 4;   // Bs[k][n]: 16-byte aligned rows for float4 writes
constexpr int kStrideBT = GBN + 1;  // Bs[k][n] written from k-contiguous B

enum : int { VEC_ROW = 0, VEC_COL = 1, SCALAR = 2 };

struct GemmArgs {
    const float *a, *b;
    float *c;
    int64_t M, N, K;
    int64_t s_am, s_ak, s_bk, s_bn, s_cm, s_cn;
    int group_m;
    const float *bias;  // dense epilogue (nullable)
    int relu;
    const float *res;   // residual added after bias / ReLU (nullable), element (m, n) at m*s_rm + n
    int64_t s_rm;
    int a_kfast, b_nfast;  // scalar loaders: which index runs fastest across threads
    float ln_eps;          // small-row kernel with LN: rows of A are layer-normalised first
    int tile0;             // register-direct kernel: the logical id of the launch's first tile
    PhaseRecord *phase;    // split kernel: the launch's phase-trace records (diagnostics builds; null otherwise)
};

// Holds the epilogue's arguments (C and its strides, bias, ReLU, residual; the layernorm's eps)
// in scalar registers
// from the kernel's start: otherwise the compiler reloads them from the kernarg segment at the
// epilogue, one more memory round trip at the end of every launch.
__device__ __forceinline__ void keep_epilogue_args(GemmArgs &g) {
    g.c = sgpr_keep(g.c);
    g.s_cm = sgpr_keep(g.s_cm);
    g.s_cn = sgpr_keep(g.s_cn);
    g.bias = sgpr_keep(g.bias);
    g.relu = sgpr_keep(g.relu);
    g.res = sgpr_keep(g.res);
    g.s_rm = sgpr_keep(g.s_rm);
    g.ln_eps = sgpr_keep(g.ln_eps);
}

// Loads the A tile (GBM x GBK at m0, k0) into 16 registers per thread.
// A_L == VEC_ROW: k contiguous; VEC_COL: m contiguous; SCALAR: any strides.
template <int A_L>
__device__ __forceinline__ void load_a(const GemmArgs &g, int t, int64_t m0, int64_t k0, float (&r)[16]) {
    if constexpr (A_L == VEC_ROW) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int row = (t >> 3) + 32 * i, kq = t & 7;
            int64_t m = m0 + row, k = k0 + 4 * kq;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < g.M && k < g.K) v = *reinterpret_cast<const float4 *>(g.a + m * g.s_am + k);
            r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
        }
    } else if constexpr (A_L == VEC_COL) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int kk = (t >> 5) + 8 * i, mq = t & 31;
            int64_t m = m0 + 4 * mq, k = k0 + kk;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < g.M && k < g.K) v = *reinterpret_cast<const float4 *>(g.a + m + k * g.s_ak);
            r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int idx = t + GTHREADS * i;
            int row = g.a_kfast ? idx >> 5 : idx & 127;
            int kk = g.a_kfast ? idx & 31 : idx >> 7;
            int64_t m = m0 + row, k = k0 + kk;
            r[i] = (m < g.M && k < g.K) ? g.a[m * g.s_am + k * g.s_ak] : 0.f;
        }
    }
}

// Interior tiles of row-major A and B (every row, column and k of the tile in bounds): the
// same loads as load_a / load_b for VEC_ROW, unguarded, from per-thread pointers that advance
// by one K tile per iteration.
__device__ __forceinline__ void load_a_interior(const float *pa, int64_t s_am, float (&r)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = *reinterpret_cast<const float4 *>(pa + 32 * i * s_am);
        r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
    }
}

__device__ __forceinline__ void load_b_interior(const float *pb, int64_t s_bk, float (&r)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = *reinterpret_cast<const float4 *>(pb + 8 * i * s_bk);
        r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
    }
}

template <int A_L>
__device__ __forceinline__ void store_a(const GemmArgs &g, int t, float (&As)[GBK][kStrideAT], const float (&r)[16]) {
    if constexpr (A_L == VEC_ROW) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int row = (t >> 3) + 32 * i, kq = t & 7;
#pragma unroll
            for (int j = 0; j < 4; j++) As[4 * kq + j][row] = r[4 * i + j];
        }
    } else if constexpr (A_L == VEC_COL) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int kk = (t >> 5) + 8 * i, mq = t & 31;
#pragma unroll
            for (int j = 0; j < 4; j++) As[kk][4 * mq + j] = r[4 * i + j];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int idx = t + GTHREADS * i;
            int row = g.a_kfast ? idx >> 5 : idx & 127;
            int kk = g.a_kfast ? idx & 31 : idx >> 7;
            As[kk][row] = r[i];
        }
    }
}

// B tile (GBK x GBN at k0, n0). B_L == VEC_ROW: n contiguous; VEC_COL: k contiguous.
template <int B_L>
__device__ __forceinline__ void load_b(const GemmArgs &g, int t, int64_t k0, int64_t n0, float (&r)[16]) {
    if constexpr (B_L == VEC_ROW) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int kk = (t >> 5) + 8 * i, nq = t & 31;
            int64_t k = k0 + kk, n = n0 + 4 * nq;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < g.K && n < g.N) v = *reinterpret_cast<const float4 *>(g.b + k * g.s_bk + n);
            r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
        }
    } else if constexpr (B_L == VEC_COL) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int col = (t >> 3) + 32 * i, kq = t & 7;
            int64_t k = k0 + 4 * kq, n = n0 + col;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < g.K && n < g.N) v = *reinterpret_cast<const float4 *>(g.b + k + n * g.s_bn);
            r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int idx = t + GTHREADS * i;
            int col = g.b_nfast ? idx & 127 : idx >> 5;
            int kk = g.b_nfast ? idx >> 7 : idx & 31;
            int64_t k = k0 + kk, n = n0 + col;
            r[i] = (k < g.K && n < g.N) ? g.b[k * g.s_bk + n * g.s_bn] : 0.f;
        }
    }
}

template <int B_L, int SB>
__device__ __forceinline__ void store_b(const GemmArgs &g, int t, float (&Bs)[GBK][SB], const float (&r)[16]) {
    if constexpr (B_L == VEC_ROW) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int kk = (t >> 5) + 8 * i, nq = t & 31;
            *reinterpret_cast<float4 *>(&Bs[kk][4 * nq]) = make_float4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
        }
    } else if constexpr (B_L == VEC_COL) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int col = (t >> 3) + 32 * i, kq = t & 7;
#pragma unroll
            for (int j = 0; j < 4; j++) Bs[4 * kq + j][col] = r[4 * i + j];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int idx = t + GTHREADS * i;
            int col = g.b_nfast ? idx & 127 : idx >> 5;
            int kk = g.b_nfast ? idx >> 7 : idx & 31;
            Bs[kk][col] = r[i];
        }
    }
}

// LDS stages of the K loop: 1 (two barriers per tile, 33 KB of LDS: three workgroups per CU)
// measured 4-5 % faster at 4096^3 than 2 (one barrier, 67 KB: two workgroups per CU)
#ifndef PITON_GEMM_STAGES
#define PITON_GEMM_STAGES 1
#endif
constexpr int kStages = PITON_GEMM_STAGES;

// FULL: row-major A and B, M and N multiples of 128 and K of 32, so every tile is interior and
// every K tile whole. Without the guarded paths the kernel fits 128 registers and runs four
// workgroups per CU (4096^3: the 1024 tiles in one generation; 3 % faster than three per CU).
// Layouts with a scalar (any-stride) loader need more registers: two workgroups per CU.
template <int A_L, int B_L, bool FULL>
__global__ __launch_bounds__(GTHREADS) __attribute__((amdgpu_waves_per_eu(
    kStages == 1 ? (FULL ? 4 : (A_L == SCALAR || B_L == SCALAR) ? 2 : 3) : 1)))
void gemm_f32_kernel(GemmArgs g) {
    keep_epilogue_args(g);
    constexpr int SB = (B_L == VEC_ROW) ? kStrideB : kStrideBT;
    __shared__ float As[kStages][GBK][kStrideAT];
    __shared__ float Bs[kStages][GBK][SB];

    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l31 = lane & 31;

    // tile order: XCD-contiguous logical id, then GROUP_SIZE_M grouping (kernels.py:28-36)
    const int num_pid_m = (int)((g.M + GBM - 1) / GBM);
    const int num_pid_n = (int)((g.N + GBN - 1) / GBN);
    const int pid = xcd_logical_id(blockIdx.x, gridDim.x, kXcdCount);
    const int in_group = g.group_m * num_pid_n;
    const int group_id = pid / in_group;
    const int first_m = group_id * g.group_m;
    const int gsize = min(num_pid_m - first_m, g.group_m);
    const int pid_m = first_m + (pid % in_group) % gsize;
    const int pid_n = (pid % in_group) / gsize;
    const int64_t m0 = (int64_t)pid_m * GBM, n0 = (int64_t)pid_n * GBN;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    float ra[16], rb[16];
    const int nk = (int)((g.K + GBK - 1) / GBK);
    // row-major A and B on an interior tile: unguarded loads through advancing pointers for every
    // K tile that lies wholly inside K (the last partial one takes the guarded loaders)
    constexpr bool kRowMajor = A_L == VEC_ROW && B_L == VEC_ROW;
    static_assert(!FULL || kRowMajor, "FULL needs row-major A and B");
    const bool interior = FULL || (kRowMajor && m0 + GBM <= g.M && n0 + GBN <= g.N);
    const int nk_full = FULL ? nk : (int)(g.K / GBK);
    const float *pa = g.a + (m0 + (t >> 3)) * g.s_am + 4 * (t & 7);
    const float *pb = g.b + (int64_t)(t >> 5) * g.s_bk + n0 + 4 * (t & 31);
    if (FULL || (kRowMajor && interior && nk_full > 0)) {
        load_a_interior(pa, g.s_am, ra);
        load_b_interior(pb, g.s_bk, rb);
    } else {
        load_a<A_L>(g, t, m0, 0, ra);
        load_b<B_L>(g, t, 0, n0, rb);
    }
    store_a<A_L>(g, t, As[0], ra);
    store_b<B_L, SB>(g, t, Bs[0], rb);
    __syncthreads();

    for (int kt = 0; kt < nk; kt++) {
        const int cur = kStages == 1 ? 0 : kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            if (FULL || (kRowMajor && interior && kt + 1 < nk_full)) {
                pa += GBK;
                pb += GBK * g.s_bk;
                load_a_interior(pa, g.s_am, ra);
                load_b_interior(pb, g.s_bk, rb);
            } else {
                load_a<A_L>(g, t, m0, (int64_t)(kt + 1) * GBK, ra);
                load_b<B_L>(g, t, (int64_t)(kt + 1) * GBK, n0, rb);
            }
        }
#pragma unroll
        for (int s = 0; s < GBK / 2; s++) {
            const int kk = 2 * s + half;
            const float a0 = As[cur][kk][wm * 64 + l31];
            const float a1 = As[cur][kk][wm * 64 + 32 + l31];
            const float b0 = Bs[cur][kk][wn * 64 + l31];
            const float b1 = Bs[cur][kk][wn * 64 + 32 + l31];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        if constexpr (kStages == 1) __syncthreads();  // every wave is done reading the tile
        if (more) {
            store_a<A_L>(g, t, As[kStages == 1 ? 0 : cur ^ 1], ra);
            store_b<B_L, SB>(g, t, Bs[kStages == 1 ? 0 : cur ^ 1], rb);
        }
        __syncthreads();
    }

    // epilogue: accumulator r of a 32x32 block holds row 8*(r/4) + 4*half + r%4, column l31
#pragma unroll
    for (int mb = 0; mb < 2; mb++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            const int64_t col = n0 + wn * 64 + nb * 32 + l31;
            if (!FULL && col >= g.N) continue;
            const float bias = g.bias ? g.bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t row = m0 + wm * 64 + mb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (FULL || row < g.M) {
                    float v = acc[mb][nb][r];
                    if (g.bias) v += bias;
                    if (g.relu && v < 0.f) v = 0.f;  // NaN passes, as np.maximum(NaN, 0)
                    if (g.res) v += g.res[row * g.s_rm + col];
                    g.c[row * g.s_cm + col * g.s_cn] = v;
                }
            }
        }
}

// whole-tile shapes (row- or column-major operands) take the register-direct kernel below (1)
// or the LDS kernel (0)
#ifndef PITON_GEMM_DIRECT
#define PITON_GEMM_DIRECT 1
#endif

// Whole-tile shapes without LDS: every wave loads its own MFMA operands from memory straight
// into registers, so there is no LDS staging and no barrier, and the waves of a workgroup run
// independently. Within a K tile of 32, lane half h supplies k = 16h + s at MFMA step s (the
// contraction order inside the tile is free as long as A and B agree), which makes a row-major
// A's operands 16 consecutive floats of the lane's row (four 16-byte loads) and a row-major B's
// 16 rows of its column (one 4-byte load per row, 128 contiguous bytes per half-wave).
// Operands of tile k+1 are loaded while tile k multiplies (two register sets, the loop unrolled
// by two). Buffer descriptors carry the matrices (each < 2 GiB); every load lies inside them.
// The plain loop (ONE_GEN false, 146 VGPRs, three workgroups per CU) ran 4096^3 ~5 % faster
// than the LDS kernel, whose two barriers per K tile left the matrix pipe idle 14 % of the
// time; grids of more tiles than CUs now run as one launch per generation of one workgroup per
// CU on the interleaved form (launch_gemm), which is faster again.
#ifndef PITON_GEMM_DIRECT_KT
#define PITON_GEMM_DIRECT_KT 32
#endif
#ifndef PITON_GEMM_DIRECT_WAVES
#define PITON_GEMM_DIRECT_WAVES 3
#endif
// K per register tile: 32 (146 VGPRs, three workgroups per CU) and 16 (114 VGPRs, four per
// CU) measured the same; 32 is the default
constexpr int DKT = PITON_GEMM_DIRECT_KT;
constexpr int DKH = DKT / 2;               // k per lane half per tile
#ifndef PITON_GEMM_ONE_GEN_WAVES
#define PITON_GEMM_ONE_GEN_WAVES 2
#endif
#ifndef PITON_GEMM_DIRECT_MB
#define PITON_GEMM_DIRECT_MB 2
#endif
#ifndef PITON_GEMM_DIRECT_NB
#define PITON_GEMM_DIRECT_NB 2
#endif
// 32 x 32 blocks per wave: DMB x DNB (2 x 2: a 128 x 128 workgroup tile), or DMB x DNB_WIDE in
// the wide form (2 x 4: 128 x 256, one wave per SIMD with its accumulators in AGPRs). Measured
// with one launch per generation, 4096^3: 2 x 2 0.93 of peak, 2 x 4 0.946, 4 x 2 0.90.
#ifndef PITON_GEMM_WIDE
#define PITON_GEMM_WIDE 1
#endif
constexpr int DMB = PITON_GEMM_DIRECT_MB, DNB = PITON_GEMM_DIRECT_NB, DNB_WIDE = 2 * DNB;
constexpr int DBM = 64 * DMB, DBN = 64 * DNB;                           // workgroup tile (2 x 2 waves)
// ONE_GEN: the launch has at most one workgroup per CU (a wave alone on its SIMD): the next
// tile's loads are interleaved with this tile's products, one after each MFMA, as in the split
// kernel (2048^3: 163 -> 141 us). With several workgroups per CU the other waves hide the loads
// and the interleave only slows the wave down (4096^3: 1.02 -> 1.42 ms), so it is off there.
// AKC / BKC: A / B is contiguous along K (A row-major, B column-major). A K-contiguous operand
// is read as float4 chunks along k (lane half h holds k = 16 h + s for s = 0..15); an M- or
// N-contiguous one one element per k, coalesced across the lanes' 32 consecutive rows or
// columns. Either way lane (h, l31) supplies the same k at step s, so every layout runs the same
// MFMA sequence and gives the same bits. NBW: 32 x 32 blocks per wave along N (DNB, or DNB_WIDE
// in one-generation launches); each output element's k order does not depend on it either.
template <bool ONE_GEN, bool AKC, bool BKC, int NBW>
__global__ __launch_bounds__(GTHREADS) __attribute__((amdgpu_waves_per_eu(
    ONE_GEN ? (NBW > DNB ? 1 : PITON_GEMM_ONE_GEN_WAVES) : PITON_GEMM_DIRECT_WAVES)))
void gemm_direct_kernel(GemmArgs g) {
    keep_epilogue_args(g);
    static_assert(ONE_GEN || NBW == DNB, "the wide form runs one workgroup per CU");
    constexpr int WNB = NBW, WBN = 64 * NBW;  // blocks per wave along N, workgroup tile columns
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l31 = lane & 31;

    const int num_pid_m = (int)(g.M / DBM);
    const int num_pid_n = (int)(g.N / WBN);
    const int pid = g.tile0 + xcd_logical_id(blockIdx.x, gridDim.x, kXcdCount);
    const int in_group = g.group_m * num_pid_n;
    const int group_id = pid / in_group;
    const int first_m = group_id * g.group_m;
    const int gsize = min(num_pid_m - first_m, g.group_m);
    const int pid_m = first_m + (pid % in_group) % gsize;
    const int pid_n = (pid % in_group) / gsize;
    const int64_t m0 = (int64_t)pid_m * DBM, n0 = (int64_t)pid_n * WBN;

    // descriptors bounded at each matrix's last element (whole tiles: every load is inside)
    const auto ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(g.a), (short)0,
                                                      (int)(((g.M - 1) * g.s_am + (g.K - 1) * g.s_ak + 1) * 4), 0x00020000);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(g.b), (short)0,
                                                      (int)(((g.K - 1) * g.s_bk + (g.N - 1) * g.s_bn + 1) * 4), 0x00020000);
    // the contiguous axis has stride 1 (the host checks it): a compile-time constant here
    const int64_t s_am = AKC ? g.s_am : 1, s_ak = AKC ? 1 : g.s_ak;
    const int64_t s_bk = BKC ? 1 : g.s_bk, s_bn = BKC ? g.s_bn : 1;
    // per-lane byte offsets of the block's row (A) or column (B) at the lane half's first k
    uint32_t va[DMB], vb[WNB];
#pragma unroll
    for (int i = 0; i < DMB; i++)
        va[i] = (uint32_t)(((m0 + wm * 32 * DMB + i * 32 + l31) * s_am + (int64_t)(DKH * half) * s_ak) * 4);
#pragma unroll
    for (int i = 0; i < WNB; i++)
        vb[i] = (uint32_t)(((int64_t)(DKH * half) * s_bk + (n0 + wn * 32 * WNB + i * 32 + l31) * s_bn) * 4);
    const uint32_t sak4 = (uint32_t)(s_ak * 4), sbk4 = (uint32_t)(s_bk * 4);

    constexpr int AQ = AKC ? DKH / 4 : DKH, BQ = BKC ? DKH / 4 : DKH;  // loads per block and K tile
    struct Ops {
        std::conditional_t<AKC, f32x4, float> a[DMB][AQ];
        std::conditional_t<BKC, f32x4, float> b[WNB][BQ];
    };
    auto load = [&](int kt, Ops &o) {
        const int ka = (int)((uint32_t)kt * DKT * sak4), kb = (int)((uint32_t)kt * DKT * sbk4);
#pragma unroll
        for (int i = 0; i < DMB; i++)
#pragma unroll
            for (int q = 0; q < AQ; q++) {
                if constexpr (AKC)
                    o.a[i][q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(va[i] + 16 * q), ka, 0));
                else
                    o.a[i][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ra, (int)va[i], ka + q * (int)sak4, 0));
            }
#pragma unroll
        for (int q = 0; q < BQ; q++)
#pragma unroll
            for (int i = 0; i < WNB; i++) {
                if constexpr (BKC)
                    o.b[i][q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, (int)(vb[i] + 16 * q), kb, 0));
                else
                    o.b[i][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, (int)vb[i], kb + q * (int)sbk4, 0));
            }
    };
    auto aval = [](const Ops &o, int i, int s) {
        if constexpr (AKC) return o.a[i][s >> 2][s & 3];
        else return o.a[i][s];
    };
    auto bval = [](const Ops &o, int j, int s) {
        if constexpr (BKC) return o.b[j][s >> 2][s & 3];
        else return o.b[j][s];
    };
    f32x16 acc[DMB][WNB];
#pragma unroll
    for (int i = 0; i < DMB; i++)
#pragma unroll
        for (int j = 0; j < WNB; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    auto mul = [&](const Ops &o) {
#pragma unroll
        for (int s = 0; s < DKH; s++)
#pragma unroll
            for (int i = 0; i < DMB; i++)
#pragma unroll
                for (int j = 0; j < WNB; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(aval(o, i, s), bval(o, j, s), acc[i][j], 0, 0, 0);
    };
    // K % (2 DKT) == 0: the tiles come in pairs. The last pair's prefetch loads the last tile
    // again (never used) rather than a tile past K: every load stays inside the matrices, which
    // also keeps the uniform offsets in `soffset` legal (the descriptor's range check covers the
    // per-lane offset only)
    const int nk = (int)(g.K / DKT);
    constexpr int DLOADS = DMB * AQ + WNB * BQ, DMFMAS = DKH * DMB * WNB;
    auto interleave = [&]() {
        if constexpr (ONE_GEN) {
#pragma unroll
            for (int i = 0; i < DMFMAS; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // one MFMA
                if (i < DLOADS) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one VMEM read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    Ops o0, o1;
    load(0, o0);
    for (int kt = 0; kt < nk; kt += 2) {
        load(kt + 1, o1);
        mul(o0);
        interleave();
        load(min(kt + 2, nk - 1), o0);
        mul(o1);
        interleave();
    }

    // accumulator r of a 32x32 block holds row 8*(r/4) + 4*half + r%4, column l31
#pragma unroll
    for (int mb = 0; mb < DMB; mb++)
#pragma unroll
        for (int nb = 0; nb < WNB; nb++) {
            const int64_t col = n0 + wn * 32 * WNB + nb * 32 + l31;
            const float bias = g.bias ? g.bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t row = m0 + wm * 32 * DMB + mb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                float v = acc[mb][nb][r];
                if (g.bias) v += bias;
                if (g.relu && v < 0.f) v = 0.f;  // NaN passes, as np.maximum(NaN, 0)
                if (g.res) v += g.res[row * g.s_rm + col];
                g.c[row * g.s_cm + col * g.s_cn] = v;
            }
        }
}

// Shapes with too few 128 x 128 tiles to fill the chip (config 2's 512^3 has 16 and 1024^3 64
// for 256 CUs) or with ragged edges: a workgroup owns a 32 NB x 32 NBN tile and its KS waves
// split K, each wave computing the whole tile, NB x NBN blocks of v_mfma_f32_32x32x2_f32, over
// the K tiles kt = wave, wave + KS, ... (interleaved, so the waves read neighbouring k together).
// Operands go from memory straight into registers as in the direct kernel (the same k order
// inside a K tile of 32: lane half h supplies k = 16 h + s at step s), through buffer
// descriptors bounded at each matrix's last element. The K tail (k >= K inside the last tile,
// which may hold padding or the next row or column) reads as zeros, as the reference's K mask
// makes it: a row-major A's values there are masked (16-byte chunks by their offset, an
// unaligned row's values after its shift), a column-major B's chunks take an offset past the
// bound; a column-major A's elements (columns at least M floats apart) and a row-major B's rows
// past K (rows at least N floats apart) lie past the bound already. Rows of A past M and columns
// of B past N feed only rows and columns of C that are not stored. The KS partial tiles meet in
// LDS and add in wave order (fixed: the result does not depend on timing); the epilogue (bias,
// ReLU, residual) then stores rows < M and columns < N.
// AM: A's layout. A_ROW16: row-major, rows 16-byte aligned (16-byte loads along k). A_ROW:
// row-major, each lane's 16 consecutive A values sit r = (row start) mod 4 floats past a 16-byte
// boundary, the same r for every K tile: the lane loads the five aligned 16-byte chunks that
// cover them and picks the four-way shift in registers (5 loads and about 50 selects per block
// instead of 16 loads). A_COL: column-major (stride 1 along M), one float per k, coalesced over
// the lanes' 32 rows. BKC: B column-major (stride 1 along K, 16-byte aligned, K % 4 == 0),
// 16-byte loads along k; otherwise B has stride 1 along N and loads one float per k.
#ifndef PITON_SPLIT_MAX_WAVES
#define PITON_SPLIT_MAX_WAVES 4
#endif
#ifndef PITON_SPLIT_WAVES_PER_CU
#define PITON_SPLIT_WAVES_PER_CU 8
#endif
// the wide 64 x 128 tile of the split kernel (0: square tiles only)
#ifndef PITON_SPLIT_WIDE
#define PITON_SPLIT_WIDE 1
#endif
// the direct kernel takes whole-tile shapes with at least this many 128 x 128 tiles per CU
// grids with more tiles than CUs run as one launch per generation of one tile per CU (0: one
// launch of the multi-workgroup kernel, PITON_GEMM_DIRECT_WAVES workgroups per CU)
#ifndef PITON_GEMM_GEN_LAUNCHES
#define PITON_GEMM_GEN_LAUNCHES 1
#endif
#ifndef PITON_DIRECT_TILES_PER_CU
#define PITON_DIRECT_TILES_PER_CU 1
#endif
constexpr int kMaxSplitWaves = PITON_SPLIT_MAX_WAVES;
enum SplitA { A_ROW16 = 0, A_ROW = 1, A_COL = 2 };

template <int NB, int NBN, int KS, int AM, bool BKC, bool TAIL>
__global__ __launch_bounds__(64 * KS) void gemm_split_kernel(GemmArgs g) {
    constexpr bool AVEC = AM == A_ROW16;
    constexpr int TB = 32 * NB, TBN = 32 * NBN;  // tile rows and columns
    constexpr int NACC = NB * NBN * 16;          // accumulator registers per lane
    // the partial tiles: [wave][group of four accumulators][lane], 16 bytes per lane and group
    __shared__ f32x4 red[KS > 1 ? KS : 1][NACC / 4][64];
    keep_epilogue_args(g);
    // the wave index is uniform: readfirstlane makes the K loop, which starts at it, a scalar loop
    const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const int half = lane >> 5, l31 = lane & 31;
    PITON_PHASE_VARS;
    PITON_PHASE(0);

    const int num_pid_m = (int)((g.M + TB - 1) / TB);
    const int num_pid_n = (int)((g.N + TBN - 1) / TBN);
    const int pid = xcd_logical_id(blockIdx.x, gridDim.x, kXcdCount);
    const int in_group = g.group_m * num_pid_n;
    const int group_id = pid / in_group;
    const int first_m = group_id * g.group_m;
    const int gsize = min(num_pid_m - first_m, g.group_m);
    const int pid_m = first_m + (pid % in_group) % gsize;
    const int pid_n = (pid % in_group) / gsize;
    const int64_t m0 = (int64_t)pid_m * TB, n0 = (int64_t)pid_n * TBN;

    // the stride along each operand's contiguous axis is 1 (the host checks it)
    const int64_t s_am = AM == A_COL ? 1 : g.s_am, s_ak = AM == A_COL ? g.s_ak : 1;
    const int64_t s_bk = BKC ? 1 : g.s_bk, s_bn = BKC ? g.s_bn : 1;
    // bounded at the last element of each matrix: offsets at or past the bound read as zero. A
    // row-major A's descriptor starts at the 16-byte boundary at or below A (inside A's
    // allocation, whose start is aligned) and its bound is rounded up to whole 16-byte chunks (the
    // last chunk lies in the page of A's last element), so a 16-byte load is either wholly inside
    // or wholly outside.
    const int off0 = AM == A_COL ? 0 : (int)((reinterpret_cast<uintptr_t>(g.a) >> 2) & 3);  // A's first float past the boundary
    const float *a_al = g.a - off0;
    const int64_t a_end = off0 + (g.M - 1) * s_am + (g.K - 1) * s_ak + 1;  // floats from a_al
    const int64_t a_bound = ((a_end + 3) & ~(int64_t)3) * 4;                              // bytes
    const int64_t b_bound = ((g.K - 1) * s_bk + (g.N - 1) * s_bn + 1) * 4;
    uint32_t va[NB], vb[NBN];
    int ra_shift[NB];  // A_ROW: this lane's row start past its 16-byte boundary, in floats
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const int64_t e0 = off0 + (m0 + i * 32 + l31) * s_am + 16 * half * s_ak;
        ra_shift[i] = (int)(e0 & 3);
        va[i] = (uint32_t)((AM == A_COL ? e0 : e0 & ~(int64_t)3) * 4);
    }
#pragma unroll
    for (int j = 0; j < NBN; j++) vb[j] = (uint32_t)(((int64_t)(16 * half) * s_bk + (n0 + j * 32 + l31) * s_bn) * 4);
    const uint32_t sak4 = (uint32_t)(s_ak * 4), sbk4 = (uint32_t)(s_bk * 4);
    const int nk = (int)((g.K + 31) / 32);
    // per-lane offsets that do not change from tile to tile: one float per k of a column-major A
    // (va[i] is va[0] + 128 i) and of a row-major B (vb[j] is vb[0] + 128 j): the block offsets
    // go in the instructions' immediate offsets
    uint32_t vas[AM == A_COL ? 16 : 1], vbs[BKC ? 1 : 16];
    if constexpr (AM == A_COL) {
#pragma unroll
        for (int s = 0; s < 16; s++) vas[s] = va[0] + s * sak4;
    }
    if constexpr (!BKC) {
#pragma unroll
        for (int s = 0; s < 16; s++) vbs[s] = vb[0] + s * sbk4;
    }

    constexpr int AW = AM == A_ROW ? 20 : 16;  // A floats a lane loads per block and tile
    struct Ops {
        float a[NB][AW];
        float b[NBN][16];
    };
    // A tile's loads go through descriptors whose base is advanced to the tile and whose bound
    // shrinks by as much (scalar arithmetic only: with K % 32 == 0 the loop has no vector address
    // arithmetic), so the range check, which covers the per-lane offset, still ends each at its
    // matrix's last element: offsets at or past it read as zero. Tiles past the last one (a wave's
    // K tiles come in pairs) read through a bound of 0: zeros. TAIL (K % 32 != 0), inside the
    // last tile, k >= K: a column-major A's and a row-major B's elements lie past the bound; a
    // row-major A's 16-byte chunks and a column-major B's get an offset past the bound (2^31) by a
    // select against the tile's remaining k (a compare and a select per chunk, no branch: control
    // flow in the loop makes the compiler copy the accumulators out of AGPRs each iteration).
    constexpr uint32_t kOut = 0x80000000u;
    auto rsrc = [&](const float *base, int64_t bound, uint32_t step4, int kt) {
        const int64_t shift = (int64_t)kt * 32 * step4;  // past the last tile the base is never read
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(reinterpret_cast<const char *>(base) + shift),
                                                 (short)0, scalar_lt_select(kt, nk, (int)(bound - shift)),
                                                 0x00020000);
    };
    // PIN keeps the loads in source order with scheduling barriers (A first, then B step by step).
    auto load = [&](int kt, Ops &o, auto pin) {
        const auto ra = rsrc(a_al, a_bound, sak4, kt);
        const auto rb = rsrc(g.b, b_bound, sbk4, kt);
        const int rem = (int)(g.K - (int64_t)kt * 32) - 16 * half;  // TAIL: this lane's k below K in the tile
        // TAIL: the offset of a chunk of four k starting c past the lane's first k of the tile
        auto chunk = [&](uint32_t off, int c) -> int { return (int)(!TAIL || c < rem ? off : kOut); };
        auto pinned = [&]() {
            if constexpr (decltype(pin)::value) __builtin_amdgcn_sched_barrier(0);
        };
#pragma unroll
        for (int i = 0; i < NB; i++) {
            if constexpr (AM == A_COL) {
                // columns no closer than M floats apart (the host checks it): (m, k) with k >= K
                // lies at or past (K - 1) s_ak + M, the bound
#pragma unroll
                for (int s = 0; s < 16; s++) {
                    o.a[i][s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ra, (int)(vas[s] + 128 * i), 0, 0));
                    pinned();
                }
            } else {
                // A_ROW16: four chunks of four k; A_ROW: the five chunks holding k0 - r .. k0 - r + 19
#pragma unroll
                for (int q = 0; q < (AVEC ? 4 : 5); q++) {
                    const int off = AVEC ? chunk(va[i] + 16 * q, 4 * q) : (int)(va[i] + 16 * q);
                    const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
#pragma unroll
                    for (int e = 0; e < 4; e++) o.a[i][4 * q + e] = v[e];
                    pinned();
                }
            }
        }
        if constexpr (BKC) {
#pragma unroll
            for (int j = 0; j < NBN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x4 v =
                        __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, chunk(vb[j] + 16 * q, 4 * q), 0, 0));
#pragma unroll
                    for (int e = 0; e < 4; e++) o.b[j][4 * q + e] = v[e];
                    pinned();
                }
        } else {
#pragma unroll
            for (int s = 0; s < 16; s++)
#pragma unroll
                for (int j = 0; j < NBN; j++) {
                    o.b[j][s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, (int)(vbs[s] + 128 * j), 0, 0));
                    pinned();
                }
        }
    };
    using Pin = std::true_type;
    using Free = std::false_type;
    f32x16 acc[NB][NBN];
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
        for (int j = 0; j < NBN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    // A_ROW: the lane's 16 values of block i: window[s + r], zero where k0 + s >= K
    auto a_vals = [&](const Ops &o, int i, int kt, float (&v)[16]) {
        if constexpr (AM != A_ROW) {
#pragma unroll
            for (int s = 0; s < 16; s++) v[s] = o.a[i][s];
        } else {
            // bitwise blends with all-ones / all-zero masks (v_bfi): a select between two array
            // elements becomes a dynamic index, which moves the array to scratch memory
            const int r = ra_shift[i];
            const int64_t nvalid = g.K - ((int64_t)kt * 32 + 16 * half);
            const uint32_t m1 = 0u - (uint32_t)(r & 1), m2 = 0u - (uint32_t)((r >> 1) & 1);
            uint32_t t0[18];
#pragma unroll
            for (int s = 0; s < 18; s++) {
                const uint32_t x0 = __float_as_uint(o.a[i][s]), x1 = __float_as_uint(o.a[i][s + 1]);
                t0[s] = x0 ^ ((x0 ^ x1) & m1);
            }
#pragma unroll
            for (int s = 0; s < 16; s++) {
                const uint32_t x = t0[s] ^ ((t0[s] ^ t0[s + 2]) & m2);
                v[s] = __uint_as_float(x & (0u - (uint32_t)(s < nvalid)));
            }
        }
    };
    auto mul = [&](const Ops &o, int kt) {
        float av[NB][16];
#pragma unroll
        for (int i = 0; i < NB; i++) a_vals(o, i, kt, av[i]);
#pragma unroll
        for (int s = 0; s < 16; s++)
#pragma unroll
            for (int i = 0; i < NB; i++)
#pragma unroll
                for (int j = 0; j < NBN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], o.b[j][s], acc[i][j], 0, 0, 0);
    };
    // this wave's K tiles: wave, wave + KS, ...; the next one is in flight while one multiplies.
    // Tiles come in pairs with no condition between loads and products (a conditional product
    // lets the compiler sink its loads next to it, ending the prefetch): a tile past the last
    // one reads zeros for A (k >= K) and B (rows past K) and adds exact zeros; the prefetch
    // after the last pair is never used.
    // The scheduling barriers keep each tile's loads together ahead of the other tile's products
    // (left free, the scheduler moves every load next to its first use to save registers).
    // Each half-step issues the next tile's loads between this tile's products, PITON_SPLIT_LPM
    // loads after each MFMA from the first one on (a wave alone on its SIMD otherwise stops the
    // matrix pipe while it issues a tile's worth of loads), and the scheduling barriers keep the
    // halves apart. One load per MFMA measured best (1024^3: 22.3 us; two 23.0, three 23.8; all
    // loads ahead of the products 27.6).
#ifndef PITON_SPLIT_LPM
#define PITON_SPLIT_LPM 1
#endif

    // 32 x 32 tiles (NB = 1): 20 loads against 16 MFMAs, two after each so that every load is in
    // flight before the tile's last product (512^3: 6.04 -> 5.72 us; 64 x 64 tiles keep one:
    // 1024^3 20.9 against 21.7 us with two, 22.4 with three)
    constexpr int LOADS = NB * (AM == A_ROW16 ? 4 : AM == A_ROW ? 5 : 16) + NBN * (BKC ? 4 : 16);
    constexpr int MFMAS = 16 * NB * NBN, LPM = NB == 1 ? 2 : PITON_SPLIT_LPM;
    // PRECISE: each product waits only for its own operands (the compiler's counts) instead of
    // the whole tile at each half's start, and the next tile's loads go out from product
    // LOAD_START on. Measured per layout: faster on 32 x 32 tiles (512^3 5.46 -> 5.30 us, 768^2
    // x 2048 32.1 -> 30.8) and, loads from the 17th product on, on 64 x 64 tiles with B
    // column-major (1024^3 20.7 -> 20.1); slower on 64 x 64 tiles with B row-major (1024^3 19.6
    // -> 20.8, 1024^2 x 4096 61.9 -> 68.1).
    constexpr bool PRECISE = NB == 1 || BKC;
    constexpr int LOAD_START = NB == 2 && BKC ? 16 : 0;
    auto interleave = [&]() {
#pragma unroll
        for (int i = 0; i < MFMAS; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            if (i >= LOAD_START && (i - LOAD_START) * LPM < LOADS)
                __builtin_amdgcn_sched_group_barrier(0x020, LPM, 0);  // LPM VMEM reads
        }
    };
    // Without PRECISE each half starts with every load of its tile landed (vmcnt(0)): its tile's
    // loads went out during the other half. With PRECISE the prologue's loads land before the
    // loop (else the compiler's counts at the loop head merge the prologue's load order with the
    // loop's and wait for nearly all of them) and each product then waits for its own operands.
    // The prologue's loads go out in source order on 32 x 32 tiles (a wave has few K tiles, and
    // the first products start when their operands arrive: 512^3 5.72 -> 5.6 us); on 64 x 64
    // tiles that order measured slower in the loop that follows (1024^2 x 4096: 77 against 69 us,
    // the same instructions in another register assignment), so the compiler orders them.
    Ops o0, o1;
    if constexpr (NB == 1) load(wave, o0, Pin());
    else load(wave, o0, Free());
    if constexpr (PRECISE) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    PITON_PHASE_WAIT_LOADS();
    PITON_PHASE(1);
    for (int kt = wave; kt < nk; kt += 2 * KS) {
        if constexpr (!PRECISE) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_sched_barrier(0);
        load(kt + KS, o1, Free());
        mul(o0, kt);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!PRECISE) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_sched_barrier(0);
        load(kt + 2 * KS, o0, Free());
        mul(o1, kt + KS);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
    }

    PITON_PHASE(2);
    // accumulator r of a 32x32 block holds row 8*(r/4) + 4*half + r%4, column l31
    auto store = [&](int i, int j, int r, int ln, float v) {
        const int64_t row = m0 + i * 32 + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
        const int64_t col = n0 + j * 32 + (ln & 31);
        if (row >= g.M || col >= g.N) return;
        if (g.bias) v += g.bias[col];
        if (g.relu && v < 0.f) v = 0.f;  // NaN passes, as np.maximum(NaN, 0)
        if (g.res) v += g.res[row * g.s_rm + col];
        g.c[row * g.s_cm + col * g.s_cn] = v;
    };
    if constexpr (KS == 1) {
#pragma unroll
        for (int i = 0; i < NB; i++)
#pragma unroll
            for (int j = 0; j < NBN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) store(i, j, r, lane, acc[i][j][r]);
    } else {
#pragma unroll
        for (int i = 0; i < NB; i++)
#pragma unroll
            for (int j = 0; j < NBN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    red[wave][(i * NBN + j) * 4 + q][lane] =
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        // an LDS-only barrier: the partials are in LDS; nothing here waits for other memory
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kWaitcntLgkm0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        __builtin_amdgcn_sched_barrier(0);
        // wave w finishes the groups w, w + KS, ... of four accumulators, every partial read
        // first; the partials add in wave order
        constexpr int GPW = NACC / 4 / KS;  // groups per wave
        f32x4 part[GPW][KS];
#pragma unroll
        for (int u = 0; u < GPW; u++)
#pragma unroll
            for (int w = 0; w < KS; w++) part[u][w] = red[w][wave + KS * u][lane];
#pragma unroll
        for (int u = 0; u < GPW; u++) {
            const int x = wave + KS * u;  // group: block x / 4, accumulators 4 (x % 4) .. + 3
            f32x4 v = part[u][0];
#pragma unroll
            for (int w = 1; w < KS; w++) v += part[u][w];
#pragma unroll
            for (int e = 0; e < 4; e++) store((x >> 2) / NBN, (x >> 2) % NBN, 4 * (x & 3) + e, lane, v[e]);
        }
    }
    PITON_PHASE(3);
    PITON_PHASE_END(kPhaseGemmSplit, g.phase);
}

// First index of the largest of x[r, 0:n] (numpy argmax rule: the first NaN wins), one wave
// per row: each lane scans elements lane, lane + 64, ..., then the (value, index) pairs combine
// across the wave with argmax_combine (common.h), whose result does not depend on the order.

__global__ __launch_bounds__(256) void argmax_rows_kernel(const float *x, int64_t rows, int64_t ld, int n, int32_t *out) {
    out = sgpr_keep(out);  // read with the other arguments, not reloaded at the store
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;  // whole wavefront leaves together
    const float *row = x + r * ld;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = lane; i < n; i += 64) argmax_combine(bv, bi, row[i], i);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        const float v2 = __shfl_xor(bv, s);
        const int i2 = __shfl_xor(bi, s);
        argmax_combine(bv, bi, v2, i2);
    }
    if (lane == 0) out[r] = bi;
}

// Y = X W (+ bias, ReLU, + residual) for at most 64 rows (a decode step's batch): the big
// kernel would give such a product a handful of 128 x 128 tiles walking K serially. Here a
// workgroup owns one 16-row tile and 16 columns (v_mfma_f32_16x16x4f32; the grid is column
// blocks x row tiles, so a 64 x 256 product spreads over 64 CUs: with all four row tiles in
// one workgroup the product was MFMA-bound on 16 CUs, 2.4 us per 256 of K); its 16 waves
// split K, and each lane group of 16 lanes takes a contiguous quarter of its wave's K range
// (the MFMA's 4-deep k index is permuted that way), so a lane walks consecutive k. With K a
// multiple of 256 and 16-byte X rows, a lane loads X as float4 (four k at once) and the loads
// of the next four k are in flight while the current four multiply. The 16 partial tiles sum
// in a fixed order through LDS: results do not depend on timing.
constexpr int SMN = 16;        // columns per workgroup
constexpr int SMWAVES = 16;    // waves splitting K
typedef float f32x4v __attribute__((ext_vector_type(4)));

// LN: Y = LN(X) W (...), LN(x) = (x - mean) * (1 / sqrt(var + eps)) over the K columns of each
// row with the statistics computed exactly as layernorm_rows_kernel computes them for a
// 16-byte-aligned row (per lane (x0 + x1) + (x2 + x3) over its float4 chunks, DPP wave sums,
// a second pass of fmaf squares): the product sees the very values the separate layernorm
// would have written. Needs the FAST layout.
template <bool FAST, bool LN, int KQ = 0>
__global__ __launch_bounds__(64 * SMWAVES) void gemm_small_m_kernel(GemmArgs g) {
    keep_epilogue_args(g);
    static_assert(!LN || FAST, "LN needs the FAST layout");
    __shared__ float part[SMWAVES][4][64];  // [wave][accumulator][lane]: 16 KiB
    __shared__ float stats[16][2];          // LN: mean and 1/sqrt(var + eps) of the tile's rows
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, grp = lane >> 4, c16 = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * SMN, n = n0 + c16;
    const int64_t m0 = (int64_t)blockIdx.y * 16;  // this workgroup's 16-row tile
    const int64_t kq = (g.K + 4 * SMWAVES - 1) / (4 * SMWAVES);  // k per lane group
    const int64_t kbeg = (int64_t)(wave * 4 + grp) * kq;
    const bool n_ok = n < g.N;
    const int64_t m = m0 + c16;  // the A row this lane supplies
    const bool m_ok = m < g.M;
    f32x4v acc = f32x4v{0.f, 0.f, 0.f, 0.f};
    // the epilogue's bias and residual, requested with the operands (epilogue_loads): thread
    // (r, lane) = (t / 64, t % 64) < 256 finishes output (m0 + 4*grp + r, n), and only it reads
    // and writes that element (so a residual that is the output itself is read before it is
    // written)
    const int er = t >> 6;
    const int64_t emo = m0 + 4 * grp + er;
    const bool e_ok = t < 256 && emo < g.M && n_ok;
    float e_bias = 0.f, e_res = 0.f;
    auto epilogue_loads = [&]() {
        e_bias = (e_ok && g.bias) ? g.bias[n] : 0.f;
        e_res = (e_ok && g.res) ? g.res[emo * g.s_rm + n] : 0.f;
    };
    float ln_mean = 0.f, ln_inv = 1.f;
    // LN: wave w computes the statistics of row m0 + w (K % 256 == 0, so a lane's chunks are
    // lane + 64c); a row of up to 1024 columns stays in registers for the variance pass
    auto ln_stats = [&]() {
        constexpr int MAXC = 4;
        const int64_t mr = m0 + wave;
        if (mr < g.M) {
            const f32x4v *src = reinterpret_cast<const f32x4v *>(g.a + mr * g.s_am);
            const int64_t nch = g.K / 4;
            float sum = 0.f, q = 0.f, mean;
            if (nch <= 64 * MAXC) {
                f32x4v ch[MAXC];
#pragma unroll
                for (int c = 0; c < MAXC; c++)
                    if (lane + 64 * c < nch) ch[c] = src[lane + 64 * c];
#pragma unroll
                for (int c = 0; c < MAXC; c++)
                    if (lane + 64 * c < nch) sum += (ch[c][0] + ch[c][1]) + (ch[c][2] + ch[c][3]);
                mean = wave_reduce(sum, SumOp()) / (float)g.K;
#pragma unroll
                for (int c = 0; c < MAXC; c++)
                    if (lane + 64 * c < nch) {
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float d = ch[c][j] - mean;
                            q = fmaf(d, d, q);
                        }
                    }
            } else {
                for (int64_t ci = lane; ci < nch; ci += 64) {
                    const f32x4v f = src[ci];
                    sum += (f[0] + f[1]) + (f[2] + f[3]);
                }
                mean = wave_reduce(sum, SumOp()) / (float)g.K;
                for (int64_t ci = lane; ci < nch; ci += 64) {
                    const f32x4v f = src[ci];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float d = f[j] - mean;
                        q = fmaf(d, d, q);
                    }
                }
            }
            const float var = wave_reduce(q, SumOp()) / (float)g.K;
            if (lane == 0) {
                stats[wave][0] = mean;
                stats[wave][1] = 1.0f / sqrtf(var + g.ln_eps);
            }
        }
        __syncthreads();
        if (m_ok) {
            ln_mean = stats[c16][0];
            ln_inv = stats[c16][1];
        }
    };
    if constexpr (FAST) {
        // kq % 4 == 0 and every k of the range < K; rows past M and columns past N read zeros
        const float *wp = g.b + (n_ok ? n : 0) + kbeg * g.s_bk;
        const float *xp = g.a + (m_ok ? m : 0) * g.s_am + kbeg;
        // the raw loads; the normalisation (LN) and the row mask are applied by `ready`
        auto load = [&](int64_t s, f32x4v &xa, float (&wb)[4]) {
            xa = *reinterpret_cast<const f32x4v *>(xp + s);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float w = wp[(s + j) * g.s_bk];
                wb[j] = n_ok ? w : 0.f;
            }
        };
        auto ready = [&](f32x4v &xa) {
            if constexpr (LN) {
#pragma unroll
                for (int j = 0; j < 4; j++) xa[j] = (xa[j] - ln_mean) * ln_inv;
            }
            xa = m_ok ? xa : f32x4v{0.f, 0.f, 0.f, 0.f};
        };
        auto mul = [&](const f32x4v &xa, const float (&wb)[4]) {
#pragma unroll
            for (int j = 0; j < 4; j++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[j], wb[j], acc, 0, 0, 0);
        };
        if constexpr (KQ > 0) {
            // K = 64 KQ: the lane group's whole k range is requested at once, one memory round
            // trip, and the bias and residual after it (a wait for these covers them all)
            f32x4v xa[KQ / 4];
            float wb[KQ / 4][4];
#pragma unroll
            for (int c = 0; c < KQ / 4; c++) load(4 * c, xa[c], wb[c]);
            __builtin_amdgcn_sched_barrier(0);
            epilogue_loads();
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (LN) ln_stats();
#pragma unroll
            for (int c = 0; c < KQ / 4; c++) {
                ready(xa[c]);
                mul(xa[c], wb[c]);
            }
        } else {
            epilogue_loads();
            f32x4v xa0, xa1;
            float wb0[4], wb1[4];
            load(0, xa0, wb0);  // in flight while the LN statistics are computed
            if constexpr (LN) ln_stats();
            for (int64_t s = 0; s < kq; s += 8) {
                if (s + 4 < kq) load(s + 4, xa1, wb1);
                ready(xa0);
                mul(xa0, wb0);
                if (s + 4 >= kq) break;
                if (s + 8 < kq) load(s + 8, xa0, wb0);
                ready(xa1);
                mul(xa1, wb1);
            }
        }
    } else {
        epilogue_loads();
        const float *wp = g.b + n;
        for (int64_t s = 0; s < kq; s++) {
            const int64_t k = kbeg + s;
            const bool k_ok = k < g.K;
            const float bv = (k_ok && n_ok) ? wp[k * g.s_bk] : 0.f;
            const float av = (k_ok && m_ok) ? g.a[m * g.s_am + k] : 0.f;
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
        }
    }
    // accumulator r holds row m0 + 4*grp + r, column n0 + c16
#pragma unroll
    for (int r = 0; r < 4; r++) part[wave][r][lane] = acc[r];
    __syncthreads();
    if (t >= 256) return;
    // thread (r, lane) = (t / 64, t % 64) finishes one output: the 16 partials in wave order
    const int r = t >> 6;
    const int64_t mo = m0 + 4 * grp + r;
    if (mo >= g.M || !n_ok) return;
    float v = part[0][r][lane];
#pragma unroll
    for (int w = 1; w < SMWAVES; w++) v += part[w][r][lane];
    if (g.bias) v += e_bias;
    if (g.relu && v < 0.f) v = 0.f;  // NaN passes, as np.maximum(NaN, 0)
    if (g.res) v += e_res;
    g.c[mo * g.s_cm + n] = v;
}

// the FAST small-M kernel, with the whole K range of a lane group loaded at once where K is
// 256, 512 or 1024 (the decoder's products: 1024 in one round trip instead of two)
template <bool LN>
static void launch_small_m(const GemmArgs &g, dim3 grid, dim3 block, hipStream_t st) {
    const int64_t kq = g.K / (4 * SMWAVES);
    auto name = [](int q) {
        static const char *n[2][4] = {{"gemm_small_m_kernel<true, false, 0>", "gemm_small_m_kernel<true, false, 4>",
                                       "gemm_small_m_kernel<true, false, 8>", "gemm_small_m_kernel<true, false, 16>"},
                                      {"gemm_small_m_kernel<true, true, 0>", "gemm_small_m_kernel<true, true, 4>",
                                       "gemm_small_m_kernel<true, true, 8>", "gemm_small_m_kernel<true, true, 16>"}};
        return n[LN ? 1 : 0][q];
    };
    if (kq == 4) PITON_LAUNCH_NAMED((gemm_small_m_kernel<true, LN, 4>), name(1), grid, block, 0, st, g);
    else if (kq == 8) PITON_LAUNCH_NAMED((gemm_small_m_kernel<true, LN, 8>), name(2), grid, block, 0, st, g);
    else if (kq == 16) PITON_LAUNCH_NAMED((gemm_small_m_kernel<true, LN, 16>), name(3), grid, block, 0, st, g);
    else PITON_LAUNCH_NAMED((gemm_small_m_kernel<true, LN, 0>), name(0), grid, block, 0, st, g);
}

static int layout_a(const GemmArgs &g) {
    if (g.s_ak == 1 && g.s_am % 4 == 0 && g.K % 4 == 0 && aligned16(g.a)) return VEC_ROW;
    if (g.s_am == 1 && g.s_ak % 4 == 0 && g.M % 4 == 0 && aligned16(g.a)) return VEC_COL;
    return SCALAR;
}
static int layout_b(const GemmArgs &g) {
    if (g.s_bn == 1 && g.s_bk % 4 == 0 && g.N % 4 == 0 && aligned16(g.b)) return VEC_ROW;
    if (g.s_bk == 1 && g.s_bn % 4 == 0 && g.K % 4 == 0 && aligned16(g.b)) return VEC_COL;
    return SCALAR;
}

// The split kernel's tile (NB blocks of 32 per side), waves per workgroup and operand layouts
// for a shape, or nb = 0 when it does not apply. Tiles of 64 when there are at least as many as
// CUs, else of 32; then the waves double (up to kMaxSplitWaves) until the launch has
// PITON_SPLIT_WAVES_PER_CU waves per CU, as long as each wave keeps at least two K tiles
// (8 per CU: 1536^3 103 -> 88 us against 4; the other shapes measured the same).
struct SplitPlan {
    int nb, ks;
    int64_t tiles;
    int am;    // SplitA: A's layout
    bool bkc;  // B column-major
    int nbn;   // blocks of 32 columns per tile (nb, or 2 nb: the wide tile)
};
static SplitPlan plan_split(const GemmArgs &g, int cus) {
    SplitPlan p{0, 0, 0, A_ROW16, false, 0};
    if (g.K <= 0 || g.M <= 0 || g.N <= 0) return p;
    // A with stride 1 along K (16-byte loads where its rows are 16-byte aligned and K % 4 == 0) or
    // along M with columns at least M floats apart; B with stride 1 along N and rows at least N
    // floats apart, or with stride 1 along K, 16-byte aligned columns and K % 4 == 0
    if (g.s_ak == 1 && g.s_am > 0) p.am = g.s_am % 4 == 0 && g.K % 4 == 0 && aligned16(g.a) ? A_ROW16 : A_ROW;
    else if (g.s_am == 1 && g.s_ak >= g.M) p.am = A_COL;
    else return p;
    // (a row-major B's rows no closer than N floats apart: then the rows past K of the last K
    // tile lie past the descriptor's bound and read as zeros)
    if (g.s_bn == 1 && g.s_bk >= g.N) p.bkc = false;
    else if (g.s_bk == 1 && g.s_bn > 0 && g.s_bn % 4 == 0 && g.K % 4 == 0 && aligned16(g.b)) p.bkc = true;
    else return p;
    auto tiles2 = [&](int64_t tm, int64_t tn) { return sat_mul((g.M + tm - 1) / tm, (g.N + tn - 1) / tn); };
    auto tiles = [&](int64_t tb) { return tiles2(tb, tb); };
    const int64_t nk = (g.K + 31) / 32;
#ifndef PITON_SPLIT_NB_MAX
#define PITON_SPLIT_NB_MAX 2
#endif
    const int nb = PITON_SPLIT_NB_MAX > 1 && tiles(64) >= cus ? 2 : 1;
    const int64_t nt = tiles(32 * nb);
    int ks = 1;
    // (eight waves only on 64 x 64 tiles: their reduction gives each wave two groups of four
    // accumulators; a 32 x 32 tile has four groups)
    const int ks_max = nb == 2 ? kMaxSplitWaves : min(kMaxSplitWaves, 4);
    while (ks < ks_max && nt * ks < PITON_SPLIT_WAVES_PER_CU * (int64_t)cus && 4 * ks <= nk) ks *= 2;
    // every byte offset a lane forms (the prefetch past the last tile included) stays below 2^31
    const int64_t tb = 32 * nb, kpad = g.K + 32 * (2 * ks + 3);  // the farthest prefetch: tile nk - 1 + 2 ks
    if (sat_add(sat_mul(g.M + tb, g.s_am), sat_mul(kpad, g.s_ak)) >= (1LL << 29) - 4 ||
        sat_add(sat_mul(kpad, g.s_bk), sat_mul(g.N + tb, g.s_bn)) >= (1LL << 29) || nt > 0x7FFFFFFF)
        return p;
    p.nb = nb, p.ks = ks, p.tiles = nt, p.nbn = nb;
    // the wide tile, 64 x 128: where 64 x 64 tiles would put two workgroups on some CUs and the
    // 64 x 128 ones fit one per CU (the ragged 1000 x 1800 x 700: 464 against 240), four waves
    // splitting K give each SIMD one wave with the same MFMA work as two waves of the square
    // tile, and the wave's 2 x 4 blocks need 0.56 loads per product instead of 0.63
    const int64_t ntw = tiles2(64, 128);
    // (measured with B row-major: 2048 x 768 x 256 15.9 -> 15.4 us, 1024 x 2048 x 256 16.3 ->
    // 15.8; the same on the ragged shape with 16-byte aligned rows, 33.0 -> 32.2 with A's row
    // stride 703; B column-major measured slower and keeps the square tile)
    if (nb == 2 && ks == 4 && nt > cus && ntw <= cus && p.am != A_COL && !p.bkc && PITON_SPLIT_WIDE &&
        sat_add(sat_mul(kpad, g.s_bk), sat_mul(g.N + 128, g.s_bn)) < (1LL << 29)) {
        p.nbn = 4;
        p.tiles = ntw;
    }
    return p;
}

// the recorded name of gemm_split_kernel<NB, NBN, KS, AM, BKC, TAIL>, with its parameters' values
template <int NB, int NBN, int KS, int AM, bool BKC, bool TAIL>
static const char *split_name() {
    static const std::string name = "gemm_split_kernel<" + std::to_string(NB) + ", " + std::to_string(NBN) + ", " +
                                    std::to_string(KS) + ", " +
                                    (AM == A_ROW16 ? "A_ROW16" : AM == A_ROW ? "A_ROW" : "A_COL") + ", " +
                                    (BKC ? "true" : "false") + ", " + (TAIL ? "true" : "false") + ">";
    return name.c_str();
}

template <int NB, int NBN, int KS, int AM, bool BKC>
static void launch_split_one(const GemmArgs &g, unsigned nwg, hipStream_t st) {
    if (g.K % 32 == 0)
        PITON_LAUNCH_NAMED((gemm_split_kernel<NB, NBN, KS, AM, BKC, false>), (split_name<NB, NBN, KS, AM, BKC, false>()),
                           dim3(nwg), dim3(64 * KS), 0, st, g);
    else
        PITON_LAUNCH_NAMED((gemm_split_kernel<NB, NBN, KS, AM, BKC, true>), (split_name<NB, NBN, KS, AM, BKC, true>()),
                           dim3(nwg), dim3(64 * KS), 0, st, g);
}

template <int NB, int NBN, int KS>
static void launch_split_ks(const GemmArgs &g, int am, bool bkc, unsigned nwg, hipStream_t st) {
    if (am == A_ROW16 && !bkc) launch_split_one<NB, NBN, KS, A_ROW16, false>(g, nwg, st);
    else if (am == A_ROW16) launch_split_one<NB, NBN, KS, A_ROW16, true>(g, nwg, st);
    else if (am == A_ROW && !bkc) launch_split_one<NB, NBN, KS, A_ROW, false>(g, nwg, st);
    else if (am == A_ROW) launch_split_one<NB, NBN, KS, A_ROW, true>(g, nwg, st);
    else if (!bkc) launch_split_one<NB, NBN, KS, A_COL, false>(g, nwg, st);
    else launch_split_one<NB, NBN, KS, A_COL, true>(g, nwg, st);
}

template <int NB>
static void launch_split_nb(const GemmArgs &g, const SplitPlan &sp, unsigned nwg, hipStream_t st) {
    if (sp.ks == 1) launch_split_ks<NB, NB, 1>(g, sp.am, sp.bkc, nwg, st);
    else if (sp.ks == 2) launch_split_ks<NB, NB, 2>(g, sp.am, sp.bkc, nwg, st);
#if PITON_SPLIT_MAX_WAVES > 4
    else if (NB == 2 && sp.ks == 8) launch_split_ks<2, 2, 8>(g, sp.am, sp.bkc, nwg, st);
#endif
    else if (NB == 2 && sp.nbn == 4) launch_split_ks<2, 4, 4>(g, sp.am, sp.bkc, nwg, st);
    else launch_split_ks<NB, NB, 4>(g, sp.am, sp.bkc, nwg, st);
}

template <int A_L>
static void launch_b(int bl, const GemmArgs &g, int nwg, hipStream_t st) {
    if (bl == VEC_ROW) PITON_LAUNCH((gemm_f32_kernel<A_L, VEC_ROW, false>), dim3(nwg), dim3(GTHREADS), 0, st, g);
    else if (bl == VEC_COL) PITON_LAUNCH((gemm_f32_kernel<A_L, VEC_COL, false>), dim3(nwg), dim3(GTHREADS), 0, st, g);
    else PITON_LAUNCH((gemm_f32_kernel<A_L, SCALAR, false>), dim3(nwg), dim3(GTHREADS), 0, st, g);
}

// one_gen: no more tiles than CUs; akc / bkc: A / B contiguous along K; wide: 128 x 256 tiles
// (one-generation launches only)
static void launch_direct(bool one_gen, bool wide, bool akc, bool bkc, const GemmArgs &g, unsigned tiles,
                          hipStream_t st) {
    const dim3 grid(tiles), block(GTHREADS);
    if (wide) {
        if (akc && !bkc) PITON_LAUNCH((gemm_direct_kernel<true, true, false, DNB_WIDE>), grid, block, 0, st, g);
        else if (akc) PITON_LAUNCH((gemm_direct_kernel<true, true, true, DNB_WIDE>), grid, block, 0, st, g);
        else if (!bkc) PITON_LAUNCH((gemm_direct_kernel<true, false, false, DNB_WIDE>), grid, block, 0, st, g);
        else PITON_LAUNCH((gemm_direct_kernel<true, false, true, DNB_WIDE>), grid, block, 0, st, g);
    } else if (one_gen) {
        if (akc && !bkc) PITON_LAUNCH((gemm_direct_kernel<true, true, false, DNB>), grid, block, 0, st, g);
        else if (akc) PITON_LAUNCH((gemm_direct_kernel<true, true, true, DNB>), grid, block, 0, st, g);
        else if (!bkc) PITON_LAUNCH((gemm_direct_kernel<true, false, false, DNB>), grid, block, 0, st, g);
        else PITON_LAUNCH((gemm_direct_kernel<true, false, true, DNB>), grid, block, 0, st, g);
    } else {
        if (akc && !bkc) PITON_LAUNCH((gemm_direct_kernel<false, true, false, DNB>), grid, block, 0, st, g);
        else if (akc) PITON_LAUNCH((gemm_direct_kernel<false, true, true, DNB>), grid, block, 0, st, g);
        else if (!bkc) PITON_LAUNCH((gemm_direct_kernel<false, false, false, DNB>), grid, block, 0, st, g);
        else PITON_LAUNCH((gemm_direct_kernel<false, false, true, DNB>), grid, block, 0, st, g);
    }
}

// split_ok: shapes that give the direct kernel fewer 128 x 128 tiles than CUs, or that are not
// whole tiles, take the split kernel when each operand has stride 1 along one axis (its k order differs from the LDS kernel's, so
// the dense entry, whose bits the fused digits chain reproduces, keeps the LDS kernel)
static int launch_gemm(GemmArgs g, hipStream_t st, const char *what, bool split_ok) {
    if (g.M == 0 || g.N == 0) return PITON_OK;
    const int64_t tiles = sat_mul((g.M + GBM - 1) / GBM, (g.N + GBN - 1) / GBN);
    PITON_REQUIRE(tiles <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "%s: %lld tiles exceed one grid", what, (long long)tiles);
    // a group taller than the tile rows orders tiles exactly as a group of all of them does;
    // the clamp keeps group_m * num_pid_n within the tile count (no 32-bit overflow in the kernels)
    const int group_user = g.group_m;
    const int64_t num_pid_m = (g.M + GBM - 1) / GBM;
    if (g.group_m > num_pid_m) g.group_m = (int)num_pid_m;
    g.a_kfast = llabs(g.s_ak) <= llabs(g.s_am);
    g.b_nfast = llabs(g.s_bn) <= llabs(g.s_bk);
    const int al = layout_a(g), bl = layout_b(g);
    const int nwg = (int)tiles;
    const bool whole = al == VEC_ROW && bl == VEC_ROW && g.M % GBM == 0 && g.N % GBN == 0 && g.K % GBK == 0 && g.K > 0;
    // the direct kernel takes either layout of each operand (row- or column-major, 16-byte
    // vectors along the contiguous axis) with whole tiles; it addresses elements by 32-bit byte
    // offsets from the matrix base: positive strides and every element within 2^31 bytes
    const bool vec_layouts = (al == VEC_ROW || al == VEC_COL) && (bl == VEC_ROW || bl == VEC_COL);
    const bool direct = PITON_GEMM_DIRECT && vec_layouts && g.K > 0 && g.M % DBM == 0 && g.N % DBN == 0 &&
                        g.K % (2 * DKT) == 0 && g.s_am > 0 && g.s_ak > 0 && g.s_bk > 0 && g.s_bn > 0 &&
                        sat_add(sat_mul(g.M - 1, g.s_am), sat_mul(g.K - 1, g.s_ak)) < (1LL << 29) &&
                        sat_add(sat_mul(g.K - 1, g.s_bk), sat_mul(g.N - 1, g.s_bn)) < (1LL << 29);
    const bool akc = al == VEC_ROW, bkc = bl == VEC_COL;  // the operands contiguous along K
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    // the direct kernel's tiles: 128 x 128, or 128 x 256 when that takes as many generations of
    // one tile per CU as half as many (each wide tile is twice the work; 3072^3 keeps 128 x 128:
    // 288 wide tiles would take two generations, the second with 32 tiles, against three of 576)
    const int64_t ntiles = direct ? (g.M / DBM) * (g.N / DBN) : 0;
    const int64_t wtiles = direct && g.N % (64 * DNB_WIDE) == 0 ? (g.M / DBM) * (g.N / (64 * DNB_WIDE)) : 0;
    auto gens = [&](int64_t t) { return (t + cus - 1) / cus; };
    const bool wide = PITON_GEMM_WIDE && PITON_GEMM_GEN_LAUNCHES && wtiles > 0 && ntiles > cus &&
                      2 * gens(wtiles) == gens(ntiles);
    const int64_t dtiles = wide ? wtiles : ntiles;
    const SplitPlan sp =
        split_ok && !(direct && ntiles >= PITON_DIRECT_TILES_PER_CU * cus) ? plan_split(g, cus) : SplitPlan{0, 0, 0};
    if (sp.nb > 0) {
        // the split kernel's group order runs over its own tile rows
        const int64_t rows = (g.M + 32 * sp.nb - 1) / (32 * sp.nb);
        GemmArgs gs = g;
        gs.group_m = (int)(group_user > rows ? rows : group_user);
        gs.phase = phase_slot();
        if (sp.nb == 2) launch_split_nb<2>(gs, sp, (unsigned)sp.tiles, st);
        else launch_split_nb<1>(gs, sp, (unsigned)sp.tiles, st);
    } else if (direct) {
        // more tiles than CUs: one launch per generation of (at most) one tile per CU, each on the
        // one-generation kernel (`tile0` = the launch's first logical tile). One wave per SIMD
        // with the next tile's loads interleaved into the products keeps the matrix pipe busier
        // than three workgroups per CU running the plain loop (4096^3: 0.90 -> 0.93 of peak)
        if (PITON_GEMM_GEN_LAUNCHES && ntiles > cus) {
            for (int64_t t0 = 0; t0 < dtiles; t0 += cus) {
                GemmArgs part = g;
                part.tile0 = (int)t0;
                launch_direct(true, wide, akc, bkc, part, (unsigned)(dtiles - t0 < cus ? dtiles - t0 : cus), st);
            }
        } else {
            launch_direct(ntiles <= cus, false, akc, bkc, g, (unsigned)ntiles, st);
        }
    } else if (whole)
        PITON_LAUNCH((gemm_f32_kernel<VEC_ROW, VEC_ROW, true>), dim3(nwg), dim3(GTHREADS), 0, st, g);
    else if (al == VEC_ROW) launch_b<VEC_ROW>(bl, g, nwg, st);
    else if (al == VEC_COL) launch_b<VEC_COL>(bl, g, nwg, st);
    else launch_b<SCALAR>(bl, g, nwg, st);
    return check_launch(what);
}

}  // namespace piton

PITON_PHASE_TU(matmul)

extern "C" {

int32_t piton_mi355x_matmul(const float *a, const float *b, float *c, int64_t M, int64_t N, int64_t K,
                            int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                            int64_t stride_cm, int64_t stride_cn, int32_t group_size_m, void *stream) {
    using namespace piton;
    PITON_REQUIRE(M >= 0 && N >= 0 && K >= 0, PITON_EINVAL, "matmul: negative size M=%lld N=%lld K=%lld",
                  (long long)M, (long long)N, (long long)K);
    PITON_REQUIRE(group_size_m >= 1, PITON_EINVAL, "matmul: GROUP_SIZE_M must be >= 1, got %d", group_size_m);
    PITON_REQUIRE((M == 0 || N == 0) || c != nullptr, PITON_EINVAL, "matmul: null C");
    PITON_REQUIRE((M == 0 || N == 0 || K == 0) || (a != nullptr && b != nullptr), PITON_EINVAL, "matmul: null A or B");
    PITON_REQUIRE(aligned4(a) && aligned4(b) && aligned4(c), PITON_EINVAL, "matmul: pointers must be 4-byte aligned");
    int rc = require_device();
    if (rc) return rc;
    GemmArgs g{a, b, c, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn,
               group_size_m, nullptr, 0, nullptr, 0, 0, 0};
    rc = launch_gemm(g, (hipStream_t)stream, "matmul", true);
    if (rc == PITON_OK) clear_error();
    return rc;
}

int32_t piton_mi355x_dense(const float *x, const float *w, const float *bias, float *y, int64_t M, int64_t N,
                           int64_t K, int32_t add_bias, int32_t relu, int32_t *argmax_out, int32_t n_classes,
                           void *stream) {
    using namespace piton;
    PITON_REQUIRE(M >= 0 && N > 0 && K > 0, PITON_EINVAL, "dense: bad size M=%lld N=%lld K=%lld",
                  (long long)M, (long long)N, (long long)K);
    PITON_REQUIRE(x && w && y, PITON_EINVAL, "dense: null X, W or Y");
    PITON_REQUIRE(!add_bias || bias, PITON_EINVAL, "dense: ADD_BIAS with a null bias");
    PITON_REQUIRE(!argmax_out || (n_classes >= 1 && n_classes <= N), PITON_EINVAL,
                  "dense: n_classes %d outside [1, N=%lld]", n_classes, (long long)N);
    PITON_REQUIRE(aligned4(x) && aligned4(w) && aligned4(y) && aligned4(bias), PITON_EINVAL,
                  "dense: pointers must be 4-byte aligned");
    int rc = require_device();
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    GemmArgs g{x, w, y, M, N, K, K, 1, N, 1, N, 1, 1, add_bias ? bias : nullptr, relu ? 1 : 0, nullptr, 0, 0, 0};
    rc = launch_gemm(g, st, "dense", false);
    if (rc) return rc;
    if (argmax_out && M > 0) {
        PITON_REQUIRE((M + 3) / 4 <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "dense: M=%lld too large", (long long)M);
        PITON_LAUNCH(argmax_rows_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, y, M, N, n_classes,
                           argmax_out);
        rc = check_launch("dense argmax");
        if (rc) return rc;
    }
    clear_error();
    return PITON_OK;
}

int32_t piton_mi355x_linear(const float *x, int64_t ldx, const float *w, const float *bias, const float *residual,
                            int64_t ldr, float *y, int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t relu,
                            void *stream) {
    using namespace piton;
    PITON_REQUIRE(M >= 0 && N > 0 && K > 0, PITON_EINVAL, "linear: bad size M=%lld N=%lld K=%lld", (long long)M,
                  (long long)N, (long long)K);
    PITON_REQUIRE(ldx >= K && ldy >= N && (!residual || ldr >= N), PITON_EINVAL,
                  "linear: row strides (%lld, %lld, %lld) shorter than the rows", (long long)ldx, (long long)ldy,
                  (long long)ldr);
    PITON_REQUIRE(M == 0 || (x && w && y), PITON_EINVAL, "linear: null X, W or Y");
    PITON_REQUIRE(aligned4(x) && aligned4(w) && aligned4(y) && aligned4(bias) && aligned4(residual), PITON_EINVAL,
                  "linear: pointers must be 4-byte aligned");
    int rc = require_device();
    if (rc) return rc;
    GemmArgs g{x, w, y, M, N, K, ldx, 1, N, 1, ldy, 1, 1, bias, relu ? 1 : 0, residual, ldr, 0, 0, 0.f};
    if (M > 0 && M <= 64) {
        PITON_REQUIRE((N + SMN - 1) / SMN <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "linear: N=%lld too large", (long long)N);
        const dim3 grid((unsigned)((N + SMN - 1) / SMN), (unsigned)((M + 15) / 16)), block(64 * SMWAVES);
        if (K % (16 * SMWAVES) == 0 && ldx % 4 == 0 && aligned16(x))
            launch_small_m<false>(g, grid, block, (hipStream_t)stream);
        else
            PITON_LAUNCH((gemm_small_m_kernel<false, false>), grid, block, 0, (hipStream_t)stream, g);
        rc = check_launch("linear");
    } else {
        rc = launch_gemm(g, (hipStream_t)stream, "linear", true);
    }
    if (rc == PITON_OK) clear_error();
    return rc;
}

int32_t piton_mi355x_linear_ln(const float *x, int64_t ldx, float eps, const float *w, const float *bias,
                               const float *residual, int64_t ldr, float *y, int64_t ldy, int64_t M, int64_t N,
                               int64_t K, int32_t relu, void *stream) {
    using namespace piton;
    PITON_REQUIRE(M >= 0 && N > 0 && K > 0, PITON_EINVAL, "linear_ln: bad size M=%lld N=%lld K=%lld", (long long)M,
                  (long long)N, (long long)K);
    PITON_REQUIRE(ldx >= K && ldy >= N && (!residual || ldr >= N), PITON_EINVAL,
                  "linear_ln: row strides (%lld, %lld, %lld) shorter than the rows", (long long)ldx, (long long)ldy,
                  (long long)ldr);
    PITON_REQUIRE(M == 0 || (x && w && y), PITON_EINVAL, "linear_ln: null X, W or Y");
    PITON_REQUIRE(aligned4(x) && aligned4(w) && aligned4(y) && aligned4(bias) && aligned4(residual), PITON_EINVAL,
                  "linear_ln: pointers must be 4-byte aligned");
    PITON_REQUIRE(M <= 64 && K % (16 * SMWAVES) == 0 && ldx % 4 == 0 && aligned16(x), PITON_EUNSUPPORTED,
                  "linear_ln: needs M <= 64, K %% 256 == 0 and 16-byte X rows (M=%lld K=%lld ldx=%lld)",
                  (long long)M, (long long)K, (long long)ldx);
    PITON_REQUIRE((N + SMN - 1) / SMN <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "linear_ln: N=%lld too large", (long long)N);
    int rc = require_device();
    if (rc) return rc;
    if (M == 0) return PITON_OK;
    GemmArgs g{x, w, y, M, N, K, ldx, 1, N, 1, ldy, 1, 1, bias, relu ? 1 : 0, residual, ldr, 0, 0, eps};
    const dim3 grid((unsigned)((N + SMN - 1) / SMN), (unsigned)((M + 15) / 16)), block(64 * SMWAVES);
    launch_small_m<true>(g, grid, block, (hipStream_t)stream);
    rc = check_launch("linear_ln");
    if (rc == PITON_OK) clear_error();
    return rc;
}

int32_t piton_mi355x_argmax_rows(const float *x, int64_t rows, int64_t ld, int64_t n, int32_t *out, void *stream) {
    using namespace piton;
    PITON_REQUIRE(rows >= 0 && n >= 1 && ld >= n, PITON_EINVAL, "argmax_rows: rows=%lld n=%lld ld=%lld",
                  (long long)rows, (long long)n, (long long)ld);
    PITON_REQUIRE(rows == 0 || (x && out), PITON_EINVAL, "argmax_rows: null pointer");
    int rc = require_device();
    if (rc) return rc;
    if (rows == 0) return PITON_OK;
    PITON_REQUIRE(n <= 0x7FFFFFFF && (rows + 3) / 4 <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "argmax_rows: too large");
    PITON_LAUNCH(argmax_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, x,
                       rows, ld, (int)n, out);
    rc = check_launch("argmax_rows");
    if (rc == PITON_OK) clear_error();
    return rc;
}

}  // extern "C"
