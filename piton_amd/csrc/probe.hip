// The sustained fp32 MFMA rate of the device this library runs on, measured beside the
// datasheet's 157.3 TFLOP/s (which assumes the 2.4 GHz peak engine clock): each wave issues
// `iters` x 32 v_mfma_f32_32x32x2_f32 (64 clocks each) in two independent accumulator chains at
// two waves per SIMD, so the matrix pipe never waits on a result; the caller times the launch.
// Diagnostics only: no reference kernel corresponds to it.
#include "common.h"

namespace piton {

__global__ __launch_bounds__(256) void mfma_probe_kernel(float *out, int iters, float a, float b) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    f32x16 c0, c1;
#pragma unroll
    for (int r = 0; r < 16; r++) c0[r] = c1[r] = 0.f;
    const float x = a + 1e-7f * (float)threadIdx.x, y = b;
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int s = 0; s < 16; s++) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(y, x, c1, 0, 0, 0);
        }
    }
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r++) s += c0[r] + c1[r];
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;  // keeps the chains live
}

}  // namespace piton

extern "C" int32_t piton_mi355x_mfma_probe(float *out, int64_t workgroups, int32_t iters, void *stream) {
    using namespace piton;
    PITON_REQUIRE(workgroups >= 1 && workgroups <= (1 << 20), PITON_EINVAL, "mfma_probe: workgroups %lld outside [1, 2^20]",
                  (long long)workgroups);
    PITON_REQUIRE(iters >= 1, PITON_EINVAL, "mfma_probe: iters %d < 1", iters);
    PITON_REQUIRE(out && aligned4(out), PITON_EINVAL, "mfma_probe: out must be a 4-byte aligned pointer");
    int rc = require_device();
    if (rc) return rc;
    PITON_LAUNCH(mfma_probe_kernel, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream, out, iters, 1.0f,
                 1e-9f);
    rc = check_launch("mfma_probe");
    if (rc == PITON_OK) clear_error();
    return rc;
}
