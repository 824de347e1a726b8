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
                const int kk = 2 * (s0 + u) + half;
                bw[u] = (s0 + u < steps && col_ok) ? w[(int64_t)kk * n + col] : 0.f;
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

__device__ __forceinline__ void mlp_argmax_combine(float &v, int &i, float v2, int i2) {
    const bool n1 = v != v, n2 = v2 != v2;
    const bool take = (n1 && n2) ? i2 < i : n2 ? true : n1 ? false : (v2 > v || (v2 == v && i2 < i));
    if (take) {
        v = v2;
        i = i2;
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
        buf[0][row][kk] = r0 + row < M ? x[(r0 + row) * k0 + kk] : 0.f;
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
        for (int c = 0; c < n_classes; c++) mlp_argmax_combine(bv, bi, buf[1][t][c], c);
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
    PITON_LAUNCH(mlp3_kernel, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, x, M, w1, b1, w2, b2, w3,
                       b3, (int)k0, (int)n1, (int)n2, (int)n3, logits, pred, n_classes);
    rc = check_launch("mlp3");
    if (rc == PITON_OK) clear_error();
    return rc;
}
