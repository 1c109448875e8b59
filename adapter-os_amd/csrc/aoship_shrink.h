/*
 * aoship_shrink.h — the decode path's LoRA shrink and adapter plan as device functions.
 *
 * The MLX forward computes each adapter's delta as ((x @ A^T) @ B^T) * (scale * blend)
 * (mlx_cpp_wrapper_real.cpp:3394-3419; blend = q / 32767 from prepare_lora_for_ring,
 * crates/adapteros-lora-mlx-ffi/src/backend.rs:398-428). The first product ("shrink",
 * S = x . A^T) is computed once per call, unscaled, in float32; the base-layer kernels add the
 * second product ("expand") as extra matrix-core steps with each token's coefficient applied to
 * S on the fly.
 *
 * The shrink is a skinny GEMM (T <= 32 tokens, a few hundred rank rows, K = in_features) bound by
 * reading the bf16 A rows, so it is built like the int4 GEMV: 32-row blocks, K split over the
 * waves of a workgroup and over ks workgroups, a register ring keeping D groups of A in flight
 * per wave, x staged once per workgroup in LDS, v_mfma_f32_32x32x16_bf16 with the tokens as M,
 * and a fixed-order reduction (waves in LDS, workgroups by the last one to finish). S and the
 * plan are read by later launches, or, in a fused launch, by the GEMV workgroups of the same
 * grid: S and the plan are therefore stored with device-scope (cache-coherent) stores.
 */
#ifndef AOSHIP_SHRINK_H
#define AOSHIP_SHRINK_H

#include "aoship_device.h"
#include "aoship_internal.h"

namespace aos_shrink {

constexpr int XE = 4;

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* The plan's per-adapter inputs (bound flags, scales, the listed pointer tables) staged in LDS by
 * a workgroup that builds the plan right after routing (at most AOS_PLAN_TABS_N adapters): it loads
 * them before it routes, so that building the plan afterwards needs only the rings. */
#define AOS_PLAN_TABS_N 64
struct PlanTabs {
  uint32_t bound[AOS_PLAN_TABS_N];
  float scale[AOS_PLAN_TABS_N];
  uint64_t ptr[AOS_PLAN_NPTR][AOS_PLAN_TABS_N];
};

/* Thread a's entries (a < n): loaded into registers first (relaxed atomic loads, which the compiler
 * does not move down to their use), stored to LDS later, so that the loads overlap other work. */
struct PlanTabRegs {
  uint32_t bound;
  float scale;
  uint64_t ptr[AOS_PLAN_NPTR];
};

__device__ __forceinline__ PlanTabRegs plan_tabs_fetch(const aos_plan_params &pp) {
  PlanTabRegs r = {};
  const int a = threadIdx.x;
  if (a < pp.n && a < AOS_PLAN_TABS_N) {
    r.bound = __hip_atomic_load(pp.bound + a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    r.scale = __hip_atomic_load(pp.scale + a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int k = 0; k < AOS_PLAN_NPTR; ++k)
      if (pp.ptab[k])
        r.ptr[k] = __hip_atomic_load((const uint64_t *)(pp.ptab[k] + a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return r;
}

__device__ __forceinline__ void plan_tabs_store(const aos_plan_params &pp, const PlanTabRegs &r, PlanTabs *lt) {
  const int a = threadIdx.x;
  if (a < pp.n && a < AOS_PLAN_TABS_N) {
    lt->bound[a] = r.bound;
    lt->scale[a] = r.scale;
#pragma unroll
    for (int k = 0; k < AOS_PLAN_NPTR; ++k) lt->ptr[k][a] = r.ptr[k];
  }
}

/* Plan of one call, built by a whole workgroup: ring slot s of token t contributes adapter
 * a = adapter_indices[s] when s < top_k, its gate q > 0 and the adapter is bound
 * (backend.rs:409-425 skips q <= 0 and unknown handles). coef[t][u] = sum over such slots of
 * scale[a] * (float(q) / 32767.0f), the product mod.scale * blend_weights[i] of the MLX
 * forward. */
/* lt: the per-adapter inputs staged in LDS (NULL: read from memory). own_rings: the rings were written
 * by this workgroup (plain loads see them after its barriers); otherwise they are read with
 * device-scope loads. */
__device__ __forceinline__ void build_plan(const aos_plan_params &pp, const PlanTabs *lt = nullptr,
                                           bool own_rings = false) {
  __shared__ uint32_t bits[AOS_MAX_ADAPTERS / 32];
  __shared__ uint16_t list[AOS_PLAN_MAXU];
  __shared__ int cntU;
  __shared__ aoship_ring_t rs[AOS_DECODE_MAX_T];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int words = (pp.n + 31) >> 5;
  for (int w = tid; w < words; w += nt) bits[w] = 0u;
  /* the rings, with device-scope loads (the router may have written them in this launch) */
  for (int w = tid; w < pp.T * 10; w += nt)
    ((uint32_t *)rs)[w] = own_rings ? ((const uint32_t *)pp.rings)[w]
                                    : __hip_atomic_load((const uint32_t *)pp.rings + w, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  for (int e = tid; e < pp.T * 8; e += nt) {
    const aoship_ring_t &r = rs[e >> 3];
    const int s = e & 7;
    const int a = r.adapter_indices[s];
    if (s < (int)r.top_k && r.gates_q15[s] > 0 && a < pp.n && (lt ? lt->bound[a] != 0u : pp.bound[a] != 0))
      atomicOr(&bits[a >> 5], 1u << (a & 31));
  }
  __syncthreads();
  if (tid == 0) {
    int u = 0;
    for (int w = 0; w < words; ++w) {
      uint32_t m = bits[w];
      while (m) {
        const int b = __builtin_ctz(m);
        m &= m - 1u;
        list[u] = (uint16_t)((w << 5) + b);
        __hip_atomic_store(&pp.plan->list[u], list[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ++u;
      }
    }
    cntU = u;
    __hip_atomic_store(&pp.plan->U, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const int U = cntU;
  /* the union's row pointers in the listed tables: thread tid's entries (slot tid of each
   * table) load here and are stored after the coefficients; slots past the threads loop at the
   * end. Tables are indexed by constants only (a variable index would copy the kernel's
   * arguments to private memory). */
  uint64_t pv[AOS_PLAN_NPTR];
#pragma unroll
  for (int k = 0; k < AOS_PLAN_NPTR; ++k) {
    pv[k] = 0;
    if (tid < U && pp.ptab[k]) pv[k] = lt ? lt->ptr[k][list[tid]] : (uint64_t)aos_gld_ptr(pp.ptab[k] + list[tid]);
  }
  for (int idx = tid; idx < pp.T * U; idx += nt) {
    const int t = idx / U, u = idx - t * U;
    const int a = list[u];
    const aoship_ring_t &r = rs[t];
    float c = 0.0f;
    for (int s = 0; s < 8; ++s) {
      if (s < (int)r.top_k && r.adapter_indices[s] == a && r.gates_q15[s] > 0) {
        const float blend = (float)r.gates_q15[s] / 32767.0f;
        c += (lt ? lt->scale[a] : pp.scale[a]) * blend;
      }
    }
    aos_publish(&pp.plan->coef[t][u], c);
  }
#pragma unroll
  for (int k = 0; k < AOS_PLAN_NPTR; ++k) {
    if (!pp.ptab[k]) continue;
    if (tid < U) __hip_atomic_store(&pp.plan->ptr[k][tid], pv[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int u = tid + nt; u < U; u += nt)
      __hip_atomic_store(&pp.plan->ptr[k][u], (uint64_t)aos_gld_ptr(pp.ptab[k] + list[u]), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

/* Row blocks of 32 over the modules' rank rows. */
__device__ __forceinline__ int shrink_rows(const aos_shrink_params &p) {
  return p.n_rb[0] + (p.nmod > 1 ? p.n_rb[1] : 0) + (p.nmod > 2 ? p.n_rb[2] : 0);
}

/* One workgroup of the shrink: row block lrb (lrb == shrink_rows(p): the plan workgroup, when
 * plan_build is set), K split ksi. Returns true in wave 0 of the workgroup that completes the row
 * block (the one that stored its S, or split 0 of a row block with nothing to compute, or of the
 * plan), false elsewhere. */
template <int NV, int W, int D>
__device__ __forceinline__ bool shrink_block(const aos_shrink_params &p, int lrb, int ksi, unsigned char *smem) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rb_total = shrink_rows(p);
  if (lrb == rb_total) {
    if (ksi == 0 && p.plan_build.plan) build_plan(p.plan_build);
    return ksi == 0;
  }
  const int rb_global = lrb;
  int m = 0;
  while (m < p.nmod - 1 && lrb >= p.n_rb[m]) {
    lrb -= p.n_rb[m];
    ++m;
  }
  const aos_lora_tab &tab = p.tab[m];
  const int rpad = tab.rpad;
  const int nslots = p.all_mode ? tab.n : (p.plan->U < AOS_PLAN_MAXU ? p.plan->U : AOS_PLAN_MAXU);
  /* uniform for every K split of this row block */
  if (rpad == 0 || lrb * 32 >= nslots * rpad) return ksi == 0;

  const int T = p.T, in = p.in, G = in >> 6;
  const int i = lane & 31, c = lane >> 5;
  const int col = lrb * 32 + i;
  const int u = col / rpad, j = col - u * rpad;
  const uint16_t *arow = p.zero_row;
  bool valid = false;
  if (u < nslots) {
    const int a = p.all_mode ? u : p.plan->list[u];
    const uint16_t *A = tab.A[a];
    if (A) {
      arow = A + (size_t)j * in;
      valid = true;
    }
  }

  const int gw0 = (int)((long)ksi * G / p.ks), gw1 = (int)((long)(ksi + 1) * G / p.ks);
  const int GR = gw1 - gw0;
  const int ga = gw0 + wave * GR / W, gb = gw0 + (wave + 1) * GR / W, ng = gb - ga;

  /* x staging (first loads ahead of the ring), then the ring of A rows. Lanes without a valid
   * row read the zero buffer at a fixed offset. */
  const int xchunks = GR * 8, nx = T * xchunks;
  u32x4 xv[XE];
#pragma unroll
  for (int jx = 0; jx < XE; ++jx) {
    int idx = tid + jx * 64 * W;
    idx = idx < nx ? idx : idx % nx; /* surplus lanes re-read chunks spread over x (a single
                                      * clamped chunk would be one cache line hit by every lane) */
    const int t = idx / xchunks, r = idx - t * xchunks;
    xv[jx] = *(const u32x4 *)(p.x + (size_t)t * in + (size_t)gw0 * 64 + r * 8);
  }
  /* lane half c takes elements 32c + 8st .. +7 of each group, as the staged x fragments do; a
   * wave without a group (possible when the LDS budget forces more K splits than the geometry's
   * groups per wave allow) reads the zero row and adds nothing */
  const bool streams = valid && ng > 0;
  const uint16_t *ap = streams ? arow + (size_t)ga * 64 + 32 * c : p.zero_row;
  const int astep = streams ? 64 : 0;
  const int sstep = streams ? 8 : 0;
  u32x4 ring[D][4];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int jj = d < ng ? d : (ng > 0 ? ng - 1 : 0);
#pragma unroll
    for (int st = 0; st < 4; ++st) ring[d][st] = aos_gld16(ap + (size_t)jj * astep + sstep * st);
  }
  uint16_t *xl = (uint16_t *)(smem + 128);
  const int xstride = GR * 64;
  if (tid < 32) ((uint32_t *)smem)[tid] = 0u;
#pragma unroll
  for (int jx = 0; jx < XE; ++jx) {
    const int idx = tid + jx * 64 * W;
    if (idx < nx) {
      const int t = idx / xchunks, r = idx - t * xchunks;
      *(u32x4 *)(xl + (size_t)t * xstride + r * 8) = xv[jx];
    }
  }
  for (int idx = tid + XE * 64 * W; idx < nx; idx += 64 * W) {
    const int t = idx / xchunks, r = idx - t * xchunks;
    *(u32x4 *)(xl + (size_t)t * xstride + r * 8) =
        *(const u32x4 *)(p.x + (size_t)t * in + (size_t)gw0 * 64 + r * 8);
  }
  lds_barrier();

  const int xbase = i < T ? 128 + i * xstride * 2 + 64 * c : 0;
  const int xmult = i < T ? 128 : 0;
  f32x16 acc = {};
  for (int base = 0; base < ng; base += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int jg = base + d;
      if (jg < ng) {
        const int gl = ga + jg - gw0;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const u32x4 a = *(const u32x4 *)(smem + xbase + (size_t)gl * xmult + 16 * st);
          acc = aos_mfma32(a, ring[d][st], acc);
        }
      }
      int jn = jg + D;
      jn = jn < ng ? jn : ng - 1;
#pragma unroll
      for (int st = 0; st < 4; ++st) ring[d][st] = aos_gld16(ap + (size_t)jn * astep + sstep * st);
    }
  }

  /* fixed-order reduction: waves through LDS, then the K splits */
  float *red = (float *)smem;
  lds_barrier();
#pragma unroll
  for (int v = 0; v < NV; ++v) red[(wave * NV + v) * 64 + lane] = acc[v];
  if (NV < 16) aos_mfma_hold(acc);
  lds_barrier();
  if (wave != 0) return false;
  float tot[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float s = red[v * 64 + lane];
    for (int w = 1; w < W; ++w) s += red[(w * NV + v) * 64 + lane];
    tot[v] = s;
  }
  if (p.ks > 1) {
    float *part = p.part + ((size_t)rb_global * p.ks + ksi) * (NV * 64);
#pragma unroll
    for (int v = 0; v < NV; ++v) aos_publish(part + v * 64 + lane, tot[v]);
    uint32_t old = 0;
    if (lane == 0) old = aos_arrive(&p.counters[rb_global]);
    old = aos_shfl(old, 0);
    if (old != (uint32_t)p.ks - 1u) return false;
    if (lane == 0) aos_reset(&p.counters[rb_global]);
#pragma unroll
    for (int v = 0; v < NV; ++v) tot[v] = 0.0f;
    /* partials are read 8 at a time (all loads in flight together) and summed in order */
    for (int k0 = 0; k0 < p.ks; k0 += 8) {
      float vals[8][NV];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int k = k0 + kk < p.ks ? k0 + kk : p.ks - 1;
        const float *pp = p.part + ((size_t)rb_global * p.ks + k) * (NV * 64);
#pragma unroll
        for (int v = 0; v < NV; ++v) vals[kk][v] = aos_collect(pp + v * 64 + lane);
      }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        if (k0 + kk < p.ks) {
#pragma unroll
          for (int v = 0; v < NV; ++v) tot[v] += vals[kk][v];
        }
    }
  }
  /* S[t][col] (float32, unscaled); absent adapters give zero columns */
  if (u < nslots) {
    float *S = p.S[m];
    const int stride = p.s_stride[m];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int mt = aos_acc_m(v, lane);
      if (mt < T) aos_publish(&S[(size_t)mt * stride + col], valid ? tot[v] : 0.0f);
    }
  }
  return true;
}

}  // namespace aos_shrink

#endif
