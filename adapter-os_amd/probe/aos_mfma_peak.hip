/*
 * aos_mfma_peak.hip — achievable dense bf16 matrix-core throughput on this GPU, for the bench's
 * prefill roofline (measured beside the datasheet peak).
 *
 * Every wave issues chains of v_mfma_f32_32x32x16_bf16 on 8 independent accumulators (no memory
 * traffic in the loop); the grid fills every SIMD with two waves. The accumulators are folded and
 * written once per wave so nothing is optimised away.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

namespace {

constexpr int CHAINS = 8;

__global__ void __launch_bounds__(256, 2) mfma_loop(bf16x8 a, bf16x8 b, int iters, float *out) {
  f32x16 acc[CHAINS];
#pragma unroll
  for (int k = 0; k < CHAINS; ++k) acc[k] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < CHAINS; ++k) acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[k], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < CHAINS; ++k)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[k][v];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

/* Runs the loop on `blocks` workgroups of 4 waves, `iters` iterations; returns the dense bf16
 * TFLOP/s of the best of `reps` timed launches (after one warm-up), or a negative value on a HIP
 * error. */
extern "C" double aos_mfma_peak_tflops(int blocks, int iters, int reps) {
  float *out = nullptr;
  if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) return -1.0;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0;
  bf16x8 a, b;
  for (int k = 0; k < 8; ++k) {
    a[k] = (__bf16)(0.001f * (k + 1));
    b[k] = (__bf16)(0.002f * (k + 1));
  }
  double best = 0.0;
  for (int r = 0; r <= reps; ++r) {
    hipExtLaunchKernelGGL(mfma_loop, dim3(blocks), dim3(256), 0, 0, e0, e1, 0, a, b, iters, out);
    if (hipEventSynchronize(e1) != hipSuccess) return -1.0;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return -1.0;
    const double flops = (double)blocks * 4 * iters * CHAINS * (2.0 * 32 * 32 * 16);
    const double tf = flops / (ms * 1e-3) / 1e12;
    if (r > 0 && tf > best) best = tf;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipFree(out);
  return best;
}
