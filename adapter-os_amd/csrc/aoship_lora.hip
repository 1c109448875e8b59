/*
 * aoship_lora.hip — LoRA shrink S = coef * (X . A^T) on the matrix cores.
 *
 * The MLX forward computes each adapter's delta as ((x @ A^T) @ B^T) * (scale * blend)
 * (mlx_cpp_wrapper_real.cpp:3394-3419). Here the first product ("shrink", rank r outputs per
 * adapter) is computed once per call for every adapter in the union of the tokens' rings, with
 * the token's coefficient folded in; the second product ("expand") runs inside the base-layer
 * kernels as extra K steps of the same accumulators.
 *
 * Grid: (column tiles of 32 = (adapter, rank row) pairs, 1, K chunks); one wavefront computes a
 * 32-token x 32-column tile over its K chunk with v_mfma_f32_32x32x16_bf16, then the chunks are
 * summed in chunk order by the last workgroup to finish that tile (deterministic).
 *
 * The column-tile-0 workgroups also write the activation group half-sums xs2 used by the int4
 * bias term of the base GEMV.
 */
#include "aoship_device.h"
#include "aoship_internal.h"
#include "aoship_union.h"

namespace {

__global__ void __launch_bounds__(64) aos_shrink_kernel(aos_shrink_params p) {
  __shared__ uint32_t bits[AOS_UNION_WORDS];
  __shared__ uint16_t list[256];
  __shared__ int cnt;
  const int lane = threadIdx.x;
  const int ct = blockIdx.x;
  const int mod = blockIdx.y;
  const int kchunk = blockIdx.z;
  const aos_lora_tab &tab = p.tab[mod];
  const int U = tab.rpad > 0 ? aos_build_union(p.rings, 0, p.T, tab, bits, list, &cnt) : 0;
  const int rpad = tab.rpad;
  const bool do_mma = rpad > 0 && ct * 32 < U * rpad;
  const bool do_xs = (ct == 0) && (mod == 0) && (p.xs2 != nullptr);
  if (!do_mma && !do_xs) return;

  const int G = p.in >> 6;
  const int g0 = (int)((long)kchunk * G / p.kc);
  const int g1 = (int)((long)(kchunk + 1) * G / p.kc);
  const int i = lane & 31, c = lane >> 5;
  const int col = ct * 32 + i;
  const int u = rpad > 0 ? col / rpad : 0;
  const int j = rpad > 0 ? col % rpad : 0;
  const uint16_t *arow = (do_mma && u < U) ? tab.A[list[u]] + (size_t)j * p.in : nullptr;
  const uint16_t *xrow = (i < p.T) ? p.x + (size_t)i * p.in : nullptr;

  f32x16 acc = {};
  for (int g = g0; g < g1; ++g) {
    float hs[2] = {0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int k0 = 64 * g + 16 * st + 8 * c;
      u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
      if (xrow) a = *(const u32x4 *)(xrow + k0);
      if (arow) b = *(const u32x4 *)(arow + k0);
      if (do_mma) acc = aos_mfma32(a, b, acc);
      if (do_xs) {
        float s = hs[st >> 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s += aos_bf16_to_f32((uint16_t)(a[e] & 0xffffu));
          s += aos_bf16_to_f32((uint16_t)(a[e] >> 16));
        }
        hs[st >> 1] = s;
      }
    }
    if (do_xs) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float other = aos_shfl_f(hs[h], lane + 32 < 64 ? lane + 32 : lane);
        if (c == 0 && i < p.T) p.xs2[(size_t)i * (2 * G) + 2 * g + h] = hs[h] + other;
      }
    }
  }
  if (!do_mma) return;

  if (p.kc > 1) {
    const int slot = mod * p.n_col_tiles + ct;
    float *part = p.part + ((size_t)slot * p.kc + kchunk) * (16 * 64);
#pragma unroll
    for (int v = 0; v < 16; ++v) part[v * 64 + lane] = acc[v];
    uint32_t old = 0;
    __syncthreads();
    if (lane == 0) {
      aos_fence_release();
      old = __hip_atomic_fetch_add(&p.counters[slot], 1u, __ATOMIC_ACQ_REL,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    old = aos_shfl(old, 0);
    if (old != (uint32_t)p.kc - 1u) return;
    aos_fence_acquire();
    if (lane == 0) p.counters[slot] = 0u;
    f32x16 tot = {};
    for (int kk = 0; kk < p.kc; ++kk) {
      const float *pp = p.part + ((size_t)slot * p.kc + kk) * (16 * 64);
#pragma unroll
      for (int v = 0; v < 16; ++v) tot[v] += pp[v * 64 + lane];
    }
    acc = tot;
  }

  /* Epilogue: S[t][col] = coef(t, adapter) * acc (bfloat16). */
  const int stride = p.umax * rpad;
  if (u < U) {
    const int a = list[u];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = aos_acc_m(v, lane);
      if (m < p.T) {
        float cf = aos_coef(p.rings[m], a, tab);
        p.S[mod][(size_t)m * stride + col] = aos_f32_to_bf16(cf * acc[v]);
      }
    }
  }
}

}  // namespace

extern "C" int aos_launch_shrink(const aos_shrink_params *p, void *stream) {
  dim3 grid(p->n_col_tiles, p->nmod, p->kc);
  hipLaunchKernelGGL(aos_shrink_kernel, grid, dim3(64), 0, (hipStream_t)stream, *p);
  return (int)hipGetLastError();
}
