// The digits MLP chain (examples/digits_model.py:120-139: three dense_layer_kernel launches,
// examples/nn_kernels.py:23-74, then the argmax of the first ten logits) in one launch.
//
// The digits networks (64 -> 128 -> 64 -> 10 or 16) take mlp3_rows16_kernel below: 16 rows per
// workgroup on 16x16x4 MFMAs. Other sizes take mlp3_kernel: a workgroup of four waves takes 32
// rows through all three layers with the activations in LDS: layer l's 32-column output tiles go
// to waves round-robin, each computed as one v_mfma_f32_32x32x2_f32 chain over the whole K in
// ascending k pairs -- the order the dense GEMM uses -- then bias, ReLU (hidden layers) and the
// fp32 store, so its logits are the three dense launches' logits bit for bit. The A operand (the
// previous layer's rows) comes from LDS (row pitch 257: conflict-free), the B operand (weights,
// L2-resident after the first workgroups) from memory, a chunk of 32 k pairs loaded ahead of
// its MFMAs. The argmax follows numpy's rule (first index of the maximum; a NaN wins), the rule
// of the dense entry's fused argmax.
#include "common.h"

namespace piton {

constexpr int MLP_ROWS = 32, MLP_PITCH = 257, MLP_MAXK = 256;

// out[row][col] for the 32 x n output of one layer: in[32][k] (LDS) times w[k][n] (+ b, ReLU)
__device__ __forceinline__ void mlp_layer(const float (*in)[MLP_PITCH], int k, const float *w, const float *b, int n,
                                          bool relu, float (*out)[MLP_PITCH]) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, l31 = lane & 31;
    const int ntiles = (n + 31) / 32, steps = k / 2;
    for (int tile = wave; tile < ntiles; tile += 4) {
        const int col = 32 * tile + l31;
        const bool col_ok = col < n;
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0.f;
        for (int s0 = 0; s0 < steps; s0 += 32) {
            float bw[32];
#pragma unroll
            for (int u = 0; u < 32; u++) {
                // an unconditional load from a clamped (valid) address, then the select: a
                // conditional load becomes a branch whose join waits for it, one load at a time
                const bool ok = s0 + u < steps && col_ok;
                const int kk = ok ? 2 * (s0 + u) + half : 0, cc = ok ? col : 0;
                const float v = w[(int64_t)kk * n + cc];
                bw[u] = ok ? v : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 32; u++)
                if (s0 + u < steps) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(in[l31][2 * (s0 + u) + half], bw[u], acc,
                                                                                0, 0, 0);
        }
        // accumulator r: row 8*(r/4) + 4*half + r%4, column col
        const float bias = (b && col_ok) ? b[col] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float v = acc[r];
            if (b) v += bias;
            if (relu && v < 0.f) v = 0.f;  // NaN passes, as np.maximum(NaN, 0)
            if (col_ok) out[8 * (r >> 2) + 4 * half + (r & 3)][col] = v;  // the next layer reads k < n only
        }
    }
}

__global__ __launch_bounds__(256) void mlp3_kernel(const float *x, int64_t M, const float *w1, const float *b1,
                                                   const float *w2, const float *b2, const float *w3, const float *b3,
                                                   int k0, int n1, int n2, int n3, float *logits, int32_t *pred,
                                                   int n_classes) {
    __shared__ float buf[2][MLP_ROWS][MLP_PITCH];
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * MLP_ROWS;
    // the workgroup's 32 input rows (rows past M read zeros)
    for (int idx = t; idx < MLP_ROWS * k0; idx += 256) {
        const int row = idx / k0, kk = idx % k0;
        const bool ok = r0 + row < M;
        const float v = x[(ok ? r0 + row : 0) * k0 + kk];  // unconditional, as the weights
        buf[0][row][kk] = ok ? v : 0.f;
    }
    __syncthreads();
    mlp_layer(buf[0], k0, w1, b1, n1, true, buf[1]);
    __syncthreads();
    mlp_layer(buf[1], n1, w2, b2, n2, true, buf[0]);
    __syncthreads();
    mlp_layer(buf[0], n2, w3, b3, n3, false, buf[1]);
    __syncthreads();
    // logits and the argmax of the first n_classes: thread t < 32 takes row t
    for (int idx = t; idx < MLP_ROWS * n3; idx += 256) {
        const int row = idx / n3, c = idx % n3;
        if (r0 + row < M && logits) logits[(r0 + row) * n3 + c] = buf[1][row][c];
    }
    if (t < MLP_ROWS && r0 + t < M && pred) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int c = 0; c < n_classes; c++) argmax_combine(bv, bi, buf[1][t][c], c);
        pred[r0 + t] = bi;
    }
}

// The digits networks (K0 -> N1 -> N2 -> N3, K0, N1 and N2 multiples of 64, N3 <= 16) in one
// launch of 16-row workgroups on v_mfma_f32_16x16x4f32: 1797 rows make 113 workgroups (32-row
// tiles on 32x32x2 MFMAs made 57, leaving 199 of 256 CUs idle), and a layer's MFMA chain is
// 16-32 products of 32 cycles instead of 32-64 of 64. Four waves:
//   layer 1: wave w owns the 16-column tiles w, w + 4, ... of N1; layer 2 the same over N2;
//   layer 3 (one tile): wave 0;
// each tile is one MFMA chain over the whole K, lane group g (lanes 16g .. 16g + 15) feeding
// k = g K/4 + s at step s (the four k of a step are any four, so long as A and B agree), so a
// lane reads consecutive k: x as float4, the activations as 16-byte LDS reads. Every weight,
// bias and input a wave needs is requested at the start, before the first product, as
// unconditional loads from clamped addresses followed by selects (a conditional load becomes a
// branch whose join waits for it). The activations pass between layers through LDS behind
// barriers that wait on LDS only. The k order differs from the dense GEMM's, so the logits
// differ from three dense launches by rounding (each within the float32 error bound of the
// chain); the argmax follows numpy's rule (first index of the maximum; a NaN wins).
__device__ __forceinline__ void mlp_lds_barrier() {
    asm volatile("" ::: "memory");  // no LDS store sinks below the barrier
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWaitcntLgkm0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    __builtin_amdgcn_sched_barrier(0);
}

template <int K0, int N1, int N2, int N3>
__global__ __launch_bounds__(256) void mlp3_rows16_kernel(const float *x, int64_t M, const float *w1, const float *b1,
                                                          const float *w2, const float *b2, const float *w3,
                                                          const float *b3, float *logits, int32_t *pred,
                                                          int n_classes, PhaseRecord *phase) {
    static_assert(K0 % 64 == 0 && N1 % 64 == 0 && N2 % 64 == 0 && N3 >= 1 && N3 <= 16 && K0 <= 256 && N1 <= 256 &&
                      N2 <= 256,
                  "layer sizes of the 16-row kernel");
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    constexpr int P1 = N1 / 64, P2 = N2 / 64;          // column tiles per wave in layers 1 and 2
    constexpr int S1 = K0 / 4, S2 = N1 / 4, S3 = N2 / 4;  // MFMA steps of each layer
    constexpr int H1P = N1 + 4, H2P = N2 + 4;           // LDS row pitches (16-byte rows)
    __shared__ __align__(16) float h1[16][H1P];
    __shared__ __align__(16) float h2[16][H2P];
    __shared__ float lg[16][17];
    const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const int grp = lane >> 4, c16 = lane & 15;
    const int64_t r0 = (int64_t)blockIdx.x * 16;
    // the epilogue's arguments, read with the others at the start
    logits = sgpr_keep(logits);
    pred = sgpr_keep(pred);
    n_classes = sgpr_keep(n_classes);
    PITON_PHASE_VARS;
    PITON_PHASE(0);
    // the row this lane supplies to layer 1's A operand: a row past M reads row M - 1 instead
    // (an output row depends on its own input row only, and rows past M are never stored)
    const int64_t row = r0 + c16 < M ? r0 + c16 : M - 1;

    // -- every operand requested up front, in the order of use (the first products wait for x
    // and W1 only) --
    f32x4v xa[S1 / 4];
    const f32x4v *xp = reinterpret_cast<const f32x4v *>(x + row * K0 + S1 * grp);
#pragma unroll
    for (int q = 0; q < S1 / 4; q++) xa[q] = xp[q];
    float wb1[P1][S1], wb2[P2][S2], wb3[S3], bias1[P1], bias2[P2];
#pragma unroll
    for (int p = 0; p < P1; p++) {
        const int col = 16 * (wave + 4 * p) + c16;
#pragma unroll
        for (int s = 0; s < S1; s++) wb1[p][s] = w1[(S1 * grp + s) * N1 + col];
        bias1[p] = (b1 ? b1 : w1)[col];  // a null bias reads a weight, which the epilogue discards
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < P2; p++) {
        const int col = 16 * (wave + 4 * p) + c16;
#pragma unroll
        for (int s = 0; s < S2; s++) wb2[p][s] = w2[(S2 * grp + s) * N2 + col];
        bias2[p] = (b2 ? b2 : w2)[col];
    }
    __builtin_amdgcn_sched_barrier(0);
    // layer 3's operands (used by wave 0 only; loaded by every wave, so no branch waits on them).
    // Columns past N3 read column N3 - 1: an output column depends on its own weight column
    // only, and those columns are neither stored nor ranked
    const bool c3_ok = c16 < N3;
    const int c3 = c3_ok ? c16 : N3 - 1;
#pragma unroll
    for (int s = 0; s < S3; s++) wb3[s] = w3[(S3 * grp + s) * N3 + c3];
    const float bias3 = (b3 ? b3 : w3)[c3];
    __builtin_amdgcn_sched_barrier(0);
    PITON_PHASE_WAIT_LOADS();
    PITON_PHASE(1);

    // -- layer 1: rows of x times W1 (+ b1, ReLU) into h1 --
    f32x4v acc1[P1];
#pragma unroll
    for (int p = 0; p < P1; p++) acc1[p] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < S1 / 4; q++) {
        const f32x4v a = xa[q];
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int p = 0; p < P1; p++)
                acc1[p] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], wb1[p][4 * q + e], acc1[p], 0, 0, 0);
    }
    // accumulator r of a tile: row 4 * grp + r, column 16 * tile + c16
#pragma unroll
    for (int p = 0; p < P1; p++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = acc1[p][r] + (b1 ? bias1[p] : 0.f);
            if (v < 0.f) v = 0.f;  // NaN passes, as np.maximum(NaN, 0)
            h1[4 * grp + r][16 * (wave + 4 * p) + c16] = v;
        }
    mlp_lds_barrier();

    // -- layer 2: h1 W2 (+ b2, ReLU) into h2 --
    f32x4v acc2[P2];
#pragma unroll
    for (int p = 0; p < P2; p++) acc2[p] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < S2 / 4; q++) {
        const f32x4v a = *reinterpret_cast<const f32x4v *>(&h1[c16][S2 * grp + 4 * q]);
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int p = 0; p < P2; p++)
                acc2[p] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], wb2[p][4 * q + e], acc2[p], 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < P2; p++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = acc2[p][r] + (b2 ? bias2[p] : 0.f);
            if (v < 0.f) v = 0.f;
            h2[4 * grp + r][16 * (wave + 4 * p) + c16] = v;
        }
    mlp_lds_barrier();
    PITON_PHASE(2);
    if (wave != 0) {  // wave-uniform; no barrier follows
        PITON_PHASE(3);
        PITON_PHASE_END(kPhaseMlp, phase);
        return;
    }

    // -- layer 3 (wave 0): h2 W3 + b3, the logits and the argmax of the first n_classes --
    f32x4v acc3 = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < S3 / 4; q++) {
        const f32x4v a = *reinterpret_cast<const f32x4v *>(&h2[c16][S3 * grp + 4 * q]);
#pragma unroll
        for (int e = 0; e < 4; e++) acc3 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], wb3[4 * q + e], acc3, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float v = acc3[r] + (b3 ? bias3 : 0.f);
        const int64_t orow = r0 + 4 * grp + r;
        if (logits && c3_ok && orow < M) logits[orow * N3 + c16] = v;
        lg[4 * grp + r][c16] = v;
    }
    wave_lds_sync();
    if (lane < 16 && r0 + lane < M && pred) {
        float lv[N3];
#pragma unroll
        for (int c = 0; c < N3; c++) lv[c] = lg[lane][c];
        // in class order, numpy's rule is: the first NaN wins, else a strictly larger value
        // (selects only: the general combine's branches cost more than the ten comparisons)
        float bv = lv[0];
        int bi = 0;
#pragma unroll
        for (int c = 1; c < N3; c++) {
            const bool take = c < n_classes && bv == bv && (lv[c] != lv[c] || lv[c] > bv);
            bv = take ? lv[c] : bv;
            bi = take ? c : bi;
        }
        pred[r0 + lane] = bi;
    }
    PITON_PHASE(3);
    PITON_PHASE_END(kPhaseMlp, phase);
}

}  // namespace piton

PITON_PHASE_TU(mlp)

extern "C" int32_t piton_mi355x_mlp3(const float *x, int64_t M, const float *w1, const float *b1, const float *w2,
                                     const float *b2, const float *w3, const float *b3, int64_t k0, int64_t n1,
                                     int64_t n2, int64_t n3, float *logits, int32_t *pred, int32_t n_classes,
                                     void *stream) {
    using namespace piton;
    PITON_REQUIRE(M >= 0, PITON_EINVAL, "mlp3: negative M");
    PITON_REQUIRE(k0 >= 2 && k0 % 2 == 0 && k0 <= MLP_MAXK && n1 >= 2 && n1 % 2 == 0 && n1 <= MLP_MAXK && n2 >= 2 &&
                      n2 % 2 == 0 && n2 <= MLP_MAXK && n3 >= 1 && n3 <= MLP_MAXK,
                  PITON_EUNSUPPORTED, "mlp3: layer sizes %lld -> %lld -> %lld -> %lld outside even sizes <= 256",
                  (long long)k0, (long long)n1, (long long)n2, (long long)n3);
    PITON_REQUIRE(!pred || (n_classes >= 1 && n_classes <= n3), PITON_EINVAL, "mlp3: n_classes %d outside [1, %lld]",
                  n_classes, (long long)n3);
    PITON_REQUIRE(M == 0 || (x && w1 && w2 && w3 && (logits || pred)), PITON_EINVAL, "mlp3: null pointer");
    PITON_REQUIRE(aligned4(x) && aligned4(w1) && aligned4(w2) && aligned4(w3) && aligned4(b1) && aligned4(b2) &&
                      aligned4(b3) && aligned4(logits),
                  PITON_EINVAL, "mlp3: pointers must be 4-byte aligned");
    int rc = require_device();
    if (rc) return rc;
    if (M == 0) return PITON_OK;
    const int64_t wgs = (M + MLP_ROWS - 1) / MLP_ROWS, wgs16 = (M + 15) / 16;
    PITON_REQUIRE(wgs16 <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "mlp3: M=%lld too large", (long long)M);
    // the digits networks (ten logits, or the trained model's sixteen) with 16-byte aligned
    // input rows: 16-row tiles; other sizes: 32-row tiles, the dense GEMM's bits
    const bool digits = k0 == 64 && n1 == 128 && n2 == 64 && (n3 == 10 || n3 == 16) && aligned16(x);
    if (digits && n3 == 10)
        PITON_LAUNCH((mlp3_rows16_kernel<64, 128, 64, 10>), dim3((unsigned)wgs16), dim3(256), 0, (hipStream_t)stream,
                     x, M, w1, b1, w2, b2, w3, b3, logits, pred, n_classes, phase_slot());
    else if (digits)
        PITON_LAUNCH((mlp3_rows16_kernel<64, 128, 64, 16>), dim3((unsigned)wgs16), dim3(256), 0, (hipStream_t)stream,
                     x, M, w1, b1, w2, b2, w3, b3, logits, pred, n_classes, phase_slot());
    else
        PITON_LAUNCH(mlp3_kernel, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, x, M, w1, b1, w2, b2, w3,
                     b3, (int)k0, (int)n1, (int)n2, (int)n3, logits, pred, n_classes);
    rc = check_launch("mlp3");
    if (rc == PITON_OK) clear_error();
    return rc;
}
