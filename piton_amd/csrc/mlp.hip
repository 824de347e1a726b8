// The digits MLP chain (examples/digits_model.py:120-139: three dense_layer_kernel launches,
// examples/nn_kernels.py:23-74, then the argmax of the first ten logits) in one launch.
//
// A workgroup of four waves takes 32 rows through all three layers with the activations in
// LDS: layer l's 32-column output tiles go to waves round-robin, each computed as one
// v_mfma_f32_32x32x2_f32 chain over the whole K in ascending k pairs -- the order the dense
// GEMM uses -- then bias, ReLU (hidden layers) and the fp32 store, so the logits are the three
// dense launches' logits bit for bit. The A operand (the previous layer's rows) comes from LDS
// (row pitch 257: conflict-free), the B operand (weights, L2-resident after the first
// workgroups) from memory, a chunk of 32 k pairs loaded ahead of its MFMAs. (Staging all three
// weight matrices in LDS first measured slower: 24.5 us against 15.9.) The argmax follows
// numpy's rule (first index of the maximum; a NaN wins), the rule of the dense entry's fused
// argmax. 1797 rows: 57 workgroups instead of three launches of 15 tiles each.
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

// mlp_layer for a layer whose sizes are known at compile time, with the B operands already in
// registers: wr[p][u] is weight row 2u + half, column 32*(wave + 4p) + l31 (0 past n). The same
// MFMA chain and epilogue as mlp_layer, so the same values.
template <int K, int N, int P>
__device__ __forceinline__ void mlp_layer_regs(const float (*in)[MLP_PITCH], const float (&wr)[P][K / 2],
                                               const float *b, bool relu, float (*out)[MLP_PITCH]) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, l31 = lane & 31;
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int tile = wave + 4 * p;
        if (tile >= (N + 31) / 32) break;  // wave-uniform
        const int col = 32 * tile + l31;
        const bool col_ok = col < N;
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0.f;
#pragma unroll
        for (int u = 0; u < K / 2; u++)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(in[l31][2 * u + half], wr[p][u], acc, 0, 0, 0);
        const float bias = (b && col_ok) ? b[col] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float v = acc[r];
            if (b) v += bias;
            if (relu && v < 0.f) v = 0.f;
            if (col_ok) out[8 * (r >> 2) + 4 * half + (r & 3)][col] = v;
        }
    }
}

// The wave's B operands of one layer (its tiles wave, wave + 4, ...), requested without waiting
template <int K, int N, int P>
__device__ __forceinline__ void mlp_load_weights(const float *w, float (&wr)[P][K / 2]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, l31 = lane & 31;
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int col = 32 * (wave + 4 * p) + l31;
        const bool ok = col < N;
#pragma unroll
        for (int u = 0; u < K / 2; u++) {
            const float v = w[(int64_t)(2 * u + half) * N + (ok ? col : 0)];  // unconditional, as in mlp_layer
            wr[p][u] = ok ? v : 0.f;
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

// mlp3_kernel for layer sizes fixed at compile time: every wave requests the weights of all its
// tiles of all three layers at the start, beside the input rows, so the chain waits for memory
// once instead of once per layer and weight chunk.
template <int K0, int N1, int N2, int N3>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2)))
void mlp3_fixed_kernel(const float *x, int64_t M, const float *w1, const float *b1, const float *w2, const float *b2,
                       const float *w3, const float *b3, float *logits, int32_t *pred, int n_classes) {
    static_assert(K0 % 2 == 0 && N1 % 2 == 0 && N2 % 2 == 0 && K0 <= MLP_MAXK && N1 <= MLP_MAXK &&
                      N2 <= MLP_MAXK && N3 <= MLP_MAXK, "even sizes within the LDS tiles");
    constexpr int P1 = ((N1 + 31) / 32 + 3) / 4, P2 = ((N2 + 31) / 32 + 3) / 4, P3 = ((N3 + 31) / 32 + 3) / 4;
    __shared__ float buf[2][MLP_ROWS][MLP_PITCH];
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * MLP_ROWS;
    float wr1[P1][K0 / 2], wr2[P2][N1 / 2], wr3[P3][N2 / 2];
    mlp_load_weights<K0, N1, P1>(w1, wr1);
    mlp_load_weights<N1, N2, P2>(w2, wr2);
    mlp_load_weights<N2, N3, P3>(w3, wr3);
#pragma unroll
    for (int idx = t; idx < MLP_ROWS * K0; idx += 256) {
        const int row = idx / K0, kk = idx % K0;
        const bool ok = r0 + row < M;
        const float v = x[(ok ? r0 + row : 0) * K0 + kk];
        buf[0][row][kk] = ok ? v : 0.f;
    }
    __syncthreads();
    mlp_layer_regs<K0, N1, P1>(buf[0], wr1, b1, true, buf[1]);
    __syncthreads();
    mlp_layer_regs<N1, N2, P2>(buf[1], wr2, b2, true, buf[0]);
    __syncthreads();
    mlp_layer_regs<N2, N3, P3>(buf[0], wr3, b3, false, buf[1]);
    __syncthreads();
#pragma unroll
    for (int idx = t; idx < MLP_ROWS * N3; idx += 256) {
        const int row = idx / N3, c = idx % N3;
        if (r0 + row < M && logits) logits[(r0 + row) * N3 + c] = buf[1][row][c];
    }
    if (t < MLP_ROWS && r0 + t < M && pred) {
        // every logit of the row read first (one LDS round trip), then combined in class order
        float lv[N3];
#pragma unroll
        for (int c = 0; c < N3; c++) lv[c] = buf[1][t][c];
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int c = 0; c < N3; c++)
            if (c < n_classes) argmax_combine(bv, bi, lv[c], c);
        pred[r0 + t] = bi;
    }
}

}  // namespace piton

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
    const int64_t wgs = (M + MLP_ROWS - 1) / MLP_ROWS;
    PITON_REQUIRE(wgs <= 0x7FFFFFFF, PITON_EUNSUPPORTED, "mlp3: M=%lld too large", (long long)M);
    // the digits networks (ten logits, or the trained model's sixteen)
    if (k0 == 64 && n1 == 128 && n2 == 64 && n3 == 10)
        PITON_LAUNCH((mlp3_fixed_kernel<64, 128, 64, 10>), dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, x,
                     M, w1, b1, w2, b2, w3, b3, logits, pred, n_classes);
    else if (k0 == 64 && n1 == 128 && n2 == 64 && n3 == 16)
        PITON_LAUNCH((mlp3_fixed_kernel<64, 128, 64, 16>), dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, x,
                     M, w1, b1, w2, b2, w3, b3, logits, pred, n_classes);
    else
        PITON_LAUNCH(mlp3_kernel, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, x, M, w1, b1, w2, b2, w3,
                     b3, (int)k0, (int)n1, (int)n2, (int)n3, logits, pred, n_classes);
    rc = check_launch("mlp3");
    if (rc == PITON_OK) clear_error();
    return rc;
}
