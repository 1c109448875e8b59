/*
 * aoship_gemv.hip — decode path (T <= 32 tokens): int4 GEMV + fused LoRA expand (+ SwiGLU).
 *
 * Computes, per output row o and token t, the MLX forward's
 *   linear(x, W) + apply_lora(x)                    (mlx_cpp_wrapper_real.cpp:3372-3419)
 * and in SwiGLU mode h = (g * sigmoid(g)) * u for the gate/up pair (:3509-3522).
 *
 * HBM-bound design for gfx950:
 *   - weights stream in the q4-tile layout: one 16-byte load per lane brings a full 1 KiB
 *     (32 rows x 64 K) chunk, i.e. one quantisation group of 32 rows;
 *   - nibbles become bfloat16 (128 + q) with one and-or per pair (exact), and
 *     v_mfma_f32_32x32x16_bf16 forms t = sum (128 + q) x per group with the tokens as the M
 *     dimension (padded to 32); the group's scale and bias are applied to the accumulator:
 *         y += s * t + (b - 128 s) * sum(x over the group)
 *     so no per-element dequantisation arithmetic is needed;
 *   - K is split across the W waves of a workgroup and across ks workgroups per row block; the
 *     partials are summed in a fixed order (waves through LDS, workgroups by the last one to
 *     finish), so results are bit-identical run to run with no floating-point atomics;
 *   - the LoRA expand sum_u S[t, u] B_u[o, :] runs as extra MFMA K steps on the reduced
 *     accumulator, before the SwiGLU / store epilogue.
 */
#include "aoship_device.h"
#include "aoship_internal.h"
#include "aoship_union.h"

namespace {

template <int NV>
__device__ __forceinline__ void group_step(const u32x4 &wv, uint32_t sbv, const uint16_t *xrow,
                                           int xoff, const float *xs2, int T, int g, int G2,
                                           int lane, float (&acc)[NV]) {
  f32x16 t = {};
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    u32x4 a = {0u, 0u, 0u, 0u};
    if (xrow) a = *(const u32x4 *)(xrow + xoff + 8 * st);
    t = aos_mfma32(a, aos_q4_magic(wv[st]), t);
  }
  const float s = aos_f16_to_f32(sbv & 0xffffu);
  const float b = aos_f16_to_f32(sbv >> 16);
  const float bp = fmaf(-128.0f, s, b);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int m = aos_acc_m(v, lane);
    float xs = 0.0f;
    if (m < T) xs = xs2[(size_t)m * G2 + 2 * g] + xs2[(size_t)m * G2 + 2 * g + 1];
    acc[v] = fmaf(s, t[v], fmaf(bp, xs, acc[v]));
  }
}

/* LoRA expand: acc += S[t, :] . B_u[row, :] over the union list. */
__device__ __forceinline__ f32x16 lora_expand(f32x16 acc, const aos_lora_tab &tab,
                                              const uint16_t *S, int stride, int T,
                                              const uint16_t *list, int U, int row, int lane) {
  const int rpad = tab.rpad;
  if (rpad == 0) return acc;
  const int i = lane & 31, c = lane >> 5;
  for (int u = 0; u < U; ++u) {
    const uint16_t *brow = tab.B[list[u]] + (size_t)row * rpad;
    for (int j0 = 0; j0 < rpad; j0 += 16) {
      u32x4 a = {0u, 0u, 0u, 0u};
      if (i < T) a = *(const u32x4 *)(S + (size_t)i * stride + u * rpad + j0 + 8 * c);
      u32x4 b = *(const u32x4 *)(brow + j0 + 8 * c);
      acc = aos_mfma32(a, b, acc);
    }
  }
  return acc;
}

template <int NV, bool SW, int W>
__global__ void __launch_bounds__(64 * W) aos_gemv_kernel(aos_gemv_params p) {
  constexpr int NA = SW ? 2 : 1;
  __shared__ float red[W][NA * NV][64];
  __shared__ uint32_t bits[AOS_UNION_WORDS];
  __shared__ uint16_t list0[256], list1[256];
  __shared__ int cnt;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rb = blockIdx.x, ksi = blockIdx.y;
  /* Union lists for the expand (every workgroup builds them; only the last one uses them). */
  int U0 = 0, U1 = 0;
  if (p.tab0.rpad > 0) U0 = aos_build_union(p.rings, 0, p.T, p.tab0, bits, list0, &cnt);
  if (SW && p.tab1.rpad > 0) U1 = aos_build_union(p.rings, 0, p.T, p.tab1, bits, list1, &cnt);
  const int G = p.w0.G, G2 = 2 * G, in = p.w0.in;
  const int s_tot = p.ks * W, s_idx = ksi * W + wave;
  const int g0 = (int)((long)s_idx * G / s_tot), g1 = (int)((long)(s_idx + 1) * G / s_tot);
  const int i = lane & 31, c = lane >> 5;
  const uint16_t *xrow = (i < p.T) ? p.x + (size_t)i * in : nullptr;

  float acc0[NV], acc1[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    acc0[v] = 0.0f;
    acc1[v] = 0.0f;
  }
  const u32x4 *q0 = (const u32x4 *)p.w0.qt + (size_t)rb * G * 64 + lane;
  const uint32_t *s0 = p.w0.sb + (size_t)rb * G * 32 + (lane & 31);
  const u32x4 *q1 = SW ? (const u32x4 *)p.w1.qt + (size_t)rb * G * 64 + lane : nullptr;
  const uint32_t *s1 = SW ? p.w1.sb + (size_t)rb * G * 32 + (lane & 31) : nullptr;

  for (int g = g0; g < g1; ++g) {
    const u32x4 wv0 = q0[(size_t)g * 64];
    const uint32_t sb0 = s0[(size_t)g * 32];
    u32x4 wv1;
    uint32_t sb1 = 0;
    if (SW) {
      wv1 = q1[(size_t)g * 64];
      sb1 = s1[(size_t)g * 32];
    }
    const int xoff = 64 * g + 32 * c;
    group_step<NV>(wv0, sb0, xrow, xoff, p.xs2, p.T, g, G2, lane, acc0);
    if (SW) group_step<NV>(wv1, sb1, xrow, xoff, p.xs2, p.T, g, G2, lane, acc1);
  }

  /* Fixed-order reduction over the waves of this workgroup. */
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    red[wave][v][lane] = acc0[v];
    if (SW) red[wave][NV + v][lane] = acc1[v];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float a0 = red[0][v][lane], a1 = SW ? red[0][NV + v][lane] : 0.0f;
    for (int w = 1; w < W; ++w) {
      a0 += red[w][v][lane];
      if (SW) a1 += red[w][NV + v][lane];
    }
    acc0[v] = a0;
    acc1[v] = a1;
  }

  /* Fixed-order reduction over the ks workgroups of this row block: the last to arrive sums. */
  if (p.ks > 1) {
    float *part = p.part + ((size_t)rb * p.ks + ksi) * (NA * NV * 64);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      part[v * 64 + lane] = acc0[v];
      if (SW) part[(NV + v) * 64 + lane] = acc1[v];
    }
    uint32_t old = 0;
    if (lane == 0) {
      aos_fence_release();
      old = __hip_atomic_fetch_add(&p.counters[rb], 1u, __ATOMIC_ACQ_REL,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    old = aos_shfl(old, 0);
    if (old != (uint32_t)p.ks - 1u) return;
    aos_fence_acquire();
    if (lane == 0) p.counters[rb] = 0u;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      acc0[v] = 0.0f;
      acc1[v] = 0.0f;
    }
    for (int k = 0; k < p.ks; ++k) {
      const float *pp = p.part + ((size_t)rb * p.ks + k) * (NA * NV * 64);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        acc0[v] += pp[v * 64 + lane];
        if (SW) acc1[v] += pp[(NV + v) * 64 + lane];
      }
    }
  }

  /* LoRA expand on the full accumulators. */
  const int row = rb * 32 + (lane & 31);
  f32x16 f0 = {}, f1 = {};
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    f0[v] = acc0[v];
    f1[v] = acc1[v];
  }
  if (U0 > 0) f0 = lora_expand(f0, p.tab0, p.S0, p.umax * p.tab0.rpad, p.T, list0, U0, row, lane);
  if (SW && U1 > 0)
    f1 = lora_expand(f1, p.tab1, p.S1, p.umax * p.tab1.rpad, p.T, list1, U1, row, lane);

  const int out = p.w0.out;
  if (!SW) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int m = aos_acc_m(v, lane);
      if (m < p.T) p.y[(size_t)m * out + row] = aos_f32_to_bf16(f0[v]);
    }
  } else {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int m = aos_acc_m(v, lane);
      const float gt = f0[v], up = f1[v];
      const float sg = 1.0f / (1.0f + expf(-gt));
      const uint16_t hb = aos_f32_to_bf16((gt * sg) * up);
      float hs = aos_bf16_to_f32(hb);
      /* half-group sum over the 32 rows of this block (lanes of the same half) */
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) hs = hs + aos_shfl_f(hs, lane ^ o);
      if (m < p.T) {
        p.y[(size_t)m * out + row] = hb;
        if ((lane & 31) == 0) p.ys2[(size_t)m * (out / 32) + rb] = hs;
      }
    }
  }
}

template <int NV>
int launch_nv(const aos_gemv_params *p, int swiglu, int waves, hipStream_t st) {
  dim3 grid(p->w0.RB, p->ks);
  if (swiglu) {
    hipLaunchKernelGGL((aos_gemv_kernel<NV, true, 4>), grid, dim3(256), 0, st, *p);
  } else {
    if (waves == 4)
      hipLaunchKernelGGL((aos_gemv_kernel<NV, false, 4>), grid, dim3(256), 0, st, *p);
    else
      hipLaunchKernelGGL((aos_gemv_kernel<NV, false, 8>), grid, dim3(512), 0, st, *p);
  }
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int aos_launch_gemv(const aos_gemv_params *p, int swiglu, void *stream) {
  hipStream_t st = (hipStream_t)stream;
  const int T = p->T;
  const int waves = p->waves;
  if (waves != 4 && waves != 8) return (int)hipErrorInvalidValue;
  if (swiglu && waves != 4) return (int)hipErrorInvalidValue;
  if (T <= 1) return launch_nv<1>(p, swiglu, waves, st);
  if (T <= 2) return launch_nv<2>(p, swiglu, waves, st);
  if (T <= 4) return launch_nv<4>(p, swiglu, waves, st);
  if (T <= 8) return launch_nv<4>(p, swiglu, waves, st);
  if (T <= 16) return launch_nv<8>(p, swiglu, waves, st);
  return launch_nv<16>(p, swiglu, waves, st);
}
