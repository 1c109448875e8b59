/*
 * aoship_union.h — the distinct adapters used by a tile of tokens, and each token's coefficient.
 *
 * Ring slot s of token t contributes adapter a = adapter_indices[s] when s < top_k, its Q15 gate
 * q > 0 and the adapter has this module (prepare_lora_for_ring skips q <= 0 and unknown handles:
 * crates/adapteros-lora-mlx-ffi/src/backend.rs:398-428). The union is listed in ascending adapter
 * index; every workgroup that needs it recomputes it, so all of them agree.
 *
 * coefficient(t, a) = scale[a] * (float(q) / 32767.0f), the product the MLX forward forms as
 * mod.scale * blend_weights[i] (mlx_cpp_wrapper_real.cpp:3410, backend.rs:417).
 */
#ifndef AOSHIP_UNION_H
#define AOSHIP_UNION_H

#include "aoship_device.h"
#include "aoship_internal.h"

#define AOS_UNION_WORDS (AOS_MAX_ADAPTERS / 32)

__device__ __forceinline__ bool aos_slot_active(const aoship_ring_t &r, int s,
                                                const aos_lora_tab &tab, int *a_out,
                                                int *q_out) {
  if (s >= (int)r.top_k || s >= 8) return false;
  int q = r.gates_q15[s];
  int a = r.adapter_indices[s];
  if (q <= 0 || a >= tab.n) return false;
  if (tab.A[a] == nullptr || tab.B[a] == nullptr) return false;
  *a_out = a;
  *q_out = q;
  return true;
}

/* Build the ascending union list over tokens [t0, t1) in LDS. All threads of the block must
 * call it. bits: AOS_UNION_WORDS words of LDS; list: LDS array. Returns U. */
__device__ int aos_build_union(const aoship_ring_t *rings, int t0, int t1, const aos_lora_tab &tab,
                               uint32_t *bits, uint16_t *list, int *s_count) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int words = (tab.n + 31) >> 5;
  for (int w = tid; w < words; w += nt) bits[w] = 0u;
  __syncthreads();
  const int entries = (t1 - t0) * 8;
  for (int e = tid; e < entries; e += nt) {
    const aoship_ring_t &r = rings[t0 + (e >> 3)];
    int a, q;
    if (aos_slot_active(r, e & 7, tab, &a, &q)) atomicOr(&bits[a >> 5], 1u << (a & 31));
  }
  __syncthreads();
  if (tid == 0) {
    int u = 0;
    for (int w = 0; w < words; ++w) {
      uint32_t m = bits[w];
      while (m) {
        int b = __builtin_ctz(m);
        m &= m - 1u;
        list[u++] = (uint16_t)((w << 5) + b);
      }
    }
    *s_count = u;
  }
  __syncthreads();
  return *s_count;
}

__device__ __forceinline__ float aos_coef(const aoship_ring_t &r, int a, const aos_lora_tab &tab) {
  float c = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    int aa, q;
    if (aos_slot_active(r, s, tab, &aa, &q) && aa == a) {
      float blend = (float)q / 32767.0f;
      c += tab.scale[a] * blend; /* a repeated slot contributes twice, as in apply_lora */
    }
  }
  return c;
}

#endif
