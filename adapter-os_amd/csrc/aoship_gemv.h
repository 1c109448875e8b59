/*
 * aoship_gemv.h — the decode GEMV's device code (the body of one row block and K split, its
 * LoRA expand, the h shrink's partials and their sum), shared by the GEMV launches
 * (aoship_gemv.hip) and the launch that routes the tokens and runs the gate/up GEMV together
 * (aoship_router.hip). The design notes are at the top of aoship_gemv.hip.
 */
#ifndef AOSHIP_GEMV_H
#define AOSHIP_GEMV_H

#include "aoship_device.h"
#include "aoship_internal.h"
#include "aoship_shrink.h"

namespace aos_gemv {

constexpr int XE = 4; /* x staging: 16-byte loads per thread issued ahead of the weights */

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* Apply one group's scale and bias to the accumulators. Lanes whose token m >= T read a
 * clamped (valid) sum; their accumulators are never stored, so no branch is needed. */
template <int NV>
__device__ __forceinline__ void apply_group(const f32x16 &t, uint32_t sbv, const float *xs, int GR, int gl,
                                            int T, int lane, float (&acc)[NV]) {
  const float s = aos_f16_to_f32(sbv & 0xffffu);
  const float b = aos_f16_to_f32(sbv >> 16);
  const float bp = fmaf(-128.0f, s, b);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    int m = aos_acc_m(v, lane);
    m = m < T ? m : T - 1;
    const float sx = xs[(m * GR + gl) * 2] + xs[(m * GR + gl) * 2 + 1];
    acc[v] = fmaf(s, t[v], fmaf(bp, sx, acc[v]));
  }
  if (NV < 16) aos_mfma_hold(t);
}

/* bf16 pair from two floats, round to nearest even */
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return (uint32_t)aos_f32_to_bf16(lo) | ((uint32_t)aos_f32_to_bf16(hi) << 16);
}

/* One LoRA expand step of a wave: union slot u = 16 q / rpad, rank rows j0 .. j0 + 15. The A
 * operand is coef(t, u) * S[t, col(u) + j0 + 8c ..], the B operand B_list[u][row, j0 + 8c ..]. */
struct ExpandStep {
  float4 s0, s1;
  float cf;
  u32x4 b;
  int a; /* the union slot's adapter */
};

/* coherent: S and the plan were stored by this launch (a fused launch) and are read with
 * device-scope loads, which see other workgroups' device-scope stores. */
__device__ __forceinline__ float load_f(const float *a, bool coherent) {
  return coherent ? __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *a;
}

/* Row pointer of union slot u in a table the plan lists (pk = 1 + its pointer table). */
__device__ __forceinline__ const uint16_t *plan_ptr(const aos_gemv_params &p, int pk, int u, bool coherent) {
  const uint64_t *a = &p.plan->ptr[pk - 1][u];
  return (const uint16_t *)(coherent ? __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *a);
}

/* Row pointer of union slot u in table T: from the plan's pointer table when it lists T (a load
 * beside the list entry's), else through the list entry a (a load after it). */
__device__ __forceinline__ const uint16_t *slot_ptr(const aos_gemv_params &p, const uint16_t *const *T, int pk, int u,
                                                    int a, bool coherent) {
  return pk ? plan_ptr(p, pk, u, coherent) : aos_gld_ptr(&T[a]);
}

/* The plan's part of step q: the adapter of union slot u, the token's coefficient and the B
 * fragment (needs the plan only). pk: the plan's pointer table of tab.B (0: none). */
__device__ __forceinline__ void expand_load_b(const aos_gemv_params &p, const aos_lora_tab &tab, int pk, int q, int row,
                                              int lane, ExpandStep &e, bool coherent) {
  const int i = lane & 31, c = lane >> 5;
  const int ti = i < p.T ? i : 0;
  const int rpad = tab.rpad;
  const int colq = 16 * q, u = colq / rpad, j0 = colq - u * rpad;
  const int a = coherent ? (int)__hip_atomic_load(&p.plan->list[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : (int)p.plan->list[u];
  e.a = a;
  e.cf = i < p.T ? load_f(&p.plan->coef[ti][u], coherent) : 0.0f;
  const uint16_t *B = slot_ptr(p, tab.B, pk, u, a, coherent);
  const uint16_t *bp = B ? B + (size_t)row * rpad + j0 + 8 * c : p.zero_row;
  e.b = aos_gld16(bp);
}

/* The shrink's part of step q: the 8 values of S the lane's half of the A operand scales. */
__device__ __forceinline__ void expand_load_s(const aos_gemv_params &p, const aos_lora_tab &tab, const float *S,
                                              int stride, int q, int lane, ExpandStep &e, bool coherent) {
  const int i = lane & 31, c = lane >> 5;
  const int ti = i < p.T ? i : 0;
  const int rpad = tab.rpad;
  const int colq = 16 * q, u = colq / rpad, j0 = colq - u * rpad;
  const int scol = (p.s_all ? e.a : u) * rpad + j0 + 8 * c;
  const float *sp = S + (size_t)ti * stride + scol;
  if (coherent) {
    e.s0 = make_float4(load_f(sp, true), load_f(sp + 1, true), load_f(sp + 2, true), load_f(sp + 3, true));
    e.s1 = make_float4(load_f(sp + 4, true), load_f(sp + 5, true), load_f(sp + 6, true), load_f(sp + 7, true));
  } else {
    e.s0 = *(const float4 *)sp;
    e.s1 = *(const float4 *)(sp + 4);
  }
}

__device__ __forceinline__ void expand_load(const aos_gemv_params &p, const aos_lora_tab &tab, int pk, const float *S,
                                            int stride, int q, int row, int lane, ExpandStep &e,
                                            bool coherent = false) {
  expand_load_b(p, tab, pk, q, row, lane, e, coherent);
  expand_load_s(p, tab, S, stride, q, lane, e, coherent);
}

/* Step q of a fused launch whose plan lists the B table's row pointers (pk). The table's padded
 * rank rpad is passed by value: a reference to one of two tables of the kernel's arguments would
 * make the compiler copy the arguments to private memory. Three parts, so that loads of one
 * round trip go out together: the plan's part (list entry, coefficient, row pointer; slot clamped
 * into the plan, so it loads before U is known), then the B fragment and S, which read the zero
 * row and S's first column unless the step lies in the union (in = q < nq). */
struct PlanPart {
  const uint16_t *B;
  int u, j0;
};

__device__ __forceinline__ PlanPart expand_plan_part(const aos_gemv_params &p, int rpad, int pk, int q, int lane,
                                                     ExpandStep &e) {
  const int i = lane & 31;
  const int ti = i < p.T ? i : 0;
  const int colq = 16 * q, u0 = colq / rpad;
  PlanPart r;
  r.j0 = colq - u0 * rpad;
  r.u = u0 < AOS_PLAN_MAXU ? u0 : AOS_PLAN_MAXU - 1;
  e.a = (int)__hip_atomic_load(&p.plan->list[r.u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float cf = load_f(&p.plan->coef[ti][r.u], true);
  e.cf = i < p.T ? cf : 0.0f;
  r.B = plan_ptr(p, pk, r.u, true);
  return r;
}

__device__ __forceinline__ void expand_b_of(const aos_gemv_params &p, int rpad, const PlanPart &pp, bool in, int row,
                                            int lane, ExpandStep &e) {
  const int c = lane >> 5;
  e.b = aos_gld16(in && pp.B ? pp.B + (size_t)row * rpad + pp.j0 + 8 * c : p.zero_row);
}

__device__ __forceinline__ void expand_s_of(const aos_gemv_params &p, int rpad, const PlanPart &pp, bool in,
                                            const float *S, int stride, int lane, ExpandStep &e) {
  const int i = lane & 31, c = lane >> 5;
  const int ti = i < p.T ? i : 0;
  const float *sp = S + (in ? (size_t)ti * stride + (p.s_all ? e.a : pp.u) * rpad + pp.j0 + 8 * c : 0);
  e.s0 = make_float4(load_f(sp, true), load_f(sp + 1, true), load_f(sp + 2, true), load_f(sp + 3, true));
  e.s1 = make_float4(load_f(sp + 4, true), load_f(sp + 5, true), load_f(sp + 6, true), load_f(sp + 7, true));
}

__device__ __forceinline__ void expand_apply(const ExpandStep &e, f32x16 &f) {
  u32x4 av;
  av.x = pack_bf16(e.cf * e.s0.x, e.cf * e.s0.y);
  av.y = pack_bf16(e.cf * e.s0.z, e.cf * e.s0.w);
  av.z = pack_bf16(e.cf * e.s1.x, e.cf * e.s1.y);
  av.w = pack_bf16(e.cf * e.s1.z, e.cf * e.s1.w);
  f = aos_mfma32(av, e.b, f);
}

/* Steps q0, q0 + qs, ... (< nq) of one module, up to EB at a time: the loads of a batch go out
 * phase by phase (plan list, then B row pointers, then B fragments, S and coefficients), so a
 * batch costs three memory round trips rather than three per step (two when the plan lists the
 * row pointers). Steps past nq load nothing (the branches are uniform). */
template <int EB>
__device__ __forceinline__ void expand_rest(const aos_gemv_params &p, const aos_lora_tab &tab, int pk, const float *S,
                                            int stride, int q0, int qs, int nq, int row, int lane, bool coherent,
                                            f32x16 &f) {
  const int i = lane & 31, c = lane >> 5;
  const int ti = i < p.T ? i : 0;
  const int rpad = tab.rpad;
  for (int qb = q0; qb < nq; qb += EB * qs) {
    int u[EB], j0[EB], a[EB];
    const uint16_t *bptr[EB];
    ExpandStep e[EB];
#pragma unroll
    for (int k = 0; k < EB; ++k) {
      const int q = qb + k * qs;
      u[k] = 16 * q / rpad;
      j0[k] = 16 * q - u[k] * rpad;
      a[k] = 0;
      if (q < nq)
        a[k] = coherent ? (int)__hip_atomic_load(&p.plan->list[u[k]], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : (int)p.plan->list[u[k]];
    }
#pragma unroll
    for (int k = 0; k < EB; ++k) {
      bptr[k] = nullptr;
      if (qb + k * qs < nq) bptr[k] = slot_ptr(p, tab.B, pk, u[k], a[k], coherent);
    }
#pragma unroll
    for (int k = 0; k < EB; ++k) {
      if (qb + k * qs >= nq) continue;
      e[k].a = a[k];
      e[k].cf = i < p.T ? load_f(&p.plan->coef[ti][u[k]], coherent) : 0.0f;
      e[k].b = aos_gld16(bptr[k] ? bptr[k] + (size_t)row * rpad + j0[k] + 8 * c : p.zero_row);
      const float *sp = S + (size_t)ti * stride + (p.s_all ? a[k] : u[k]) * rpad + j0[k] + 8 * c;
      if (coherent) {
        e[k].s0 = make_float4(load_f(sp, true), load_f(sp + 1, true), load_f(sp + 2, true), load_f(sp + 3, true));
        e[k].s1 = make_float4(load_f(sp + 4, true), load_f(sp + 5, true), load_f(sp + 6, true), load_f(sp + 7, true));
      } else {
        e[k].s0 = *(const float4 *)sp;
        e[k].s1 = *(const float4 *)(sp + 4);
      }
    }
#pragma unroll
    for (int k = 0; k < EB; ++k)
      if (qb + k * qs < nq) expand_apply(e[k], f);
  }
}


/* The rest of both SwiGLU modules' steps in the same batches (EB of each), whose loads go out phase
 * by phase together (plan list and row pointers, then B fragments, S and coefficients): both
 * modules' steps cost the round trips of one module's. Each module's steps are added in its own
 * order, as expand_rest adds them, so the sums are the same. */
template <int EB>
__device__ __forceinline__ void expand_rest2(const aos_gemv_params &p, int qa, int na, int qb, int nb, int qs, int row,
                                             int lane, bool coherent, f32x16 &f0, f32x16 &f1) {
  const int i = lane & 31, c = lane >> 5;
  const int ti = i < p.T ? i : 0;
  while (qa < na || qb < nb) {
    int u[2][EB], j0[2][EB], a[2][EB];
    bool on[2][EB];
    const uint16_t *bptr[2][EB];
    ExpandStep e[2][EB];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int rpad = m ? p.tab1.rpad : p.tab0.rpad;
      const int pk = m ? p.pk1 : p.pk0;
#pragma unroll
      for (int k = 0; k < EB; ++k) {
        const int q = (m ? qb : qa) + k * qs;
        on[m][k] = q < (m ? nb : na);
        u[m][k] = on[m][k] ? 16 * q / rpad : 0;
        j0[m][k] = on[m][k] ? 16 * q - u[m][k] * rpad : 0;
        a[m][k] = 0;
        bptr[m][k] = nullptr;
        if (on[m][k]) {
          a[m][k] = coherent ? (int)__hip_atomic_load(&p.plan->list[u[m][k]], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : (int)p.plan->list[u[m][k]];
          if (pk) bptr[m][k] = plan_ptr(p, pk, u[m][k], coherent);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int pk = m ? p.pk1 : p.pk0;
#pragma unroll
      for (int k = 0; k < EB; ++k)
        if (on[m][k] && !pk) bptr[m][k] = aos_gld_ptr(&(m ? p.tab1.B : p.tab0.B)[a[m][k]]);
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int rpad = m ? p.tab1.rpad : p.tab0.rpad;
      const float *S = m ? p.S1 : p.S0;
      const int stride = m ? p.s_stride1 : p.s_stride0;
#pragma unroll
      for (int k = 0; k < EB; ++k) {
        if (!on[m][k]) continue;
        e[m][k].a = a[m][k];
        e[m][k].cf = i < p.T ? load_f(&p.plan->coef[ti][u[m][k]], coherent) : 0.0f;
        e[m][k].b = aos_gld16(bptr[m][k] ? bptr[m][k] + (size_t)row * rpad + j0[m][k] + 8 * c : p.zero_row);
        const float *sp = S + (size_t)ti * stride + (p.s_all ? a[m][k] : u[m][k]) * rpad + j0[m][k] + 8 * c;
        if (coherent) {
          e[m][k].s0 = make_float4(load_f(sp, true), load_f(sp + 1, true), load_f(sp + 2, true), load_f(sp + 3, true));
          e[m][k].s1 = make_float4(load_f(sp + 4, true), load_f(sp + 5, true), load_f(sp + 6, true), load_f(sp + 7, true));
        } else {
          e[m][k].s0 = *(const float4 *)sp;
          e[m][k].s1 = *(const float4 *)(sp + 4);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < EB; ++k)
      if (on[0][k]) expand_apply(e[0][k], f0);
#pragma unroll
    for (int k = 0; k < EB; ++k)
      if (on[1][k]) expand_apply(e[1][k], f1);
    qa += EB * qs;
    qb += EB * qs;
  }
}

/* Row block rb, K split ksi of one matrix (or of the gate/up pair). */
/* The down projection's LoRA shrink over the 32 rows of h this row block produced (wave 0 only,
 * after the SwiGLU): h goes through LDS as a [token][row] bf16 tile (the MFMA's token operand);
 * the union adapters' A_down rows at these 32 positions are the other operand, 32 union columns
 * per step; the partials land in hpart[rb][t][col]. The plan was produced by this launch, so it
 * is read with device-scope loads. */
/* A_down fragments of union column block cb (32 columns, two 16-row K steps) at this row block */
__device__ __forceinline__ void h_a_load(const aos_gemv_params &p, int rb, int lane, int U, int cb, u32x4 (&b)[2]) {
  const int i = lane & 31, c = lane >> 5;
  const int rpad = p.htab.rpad, in = p.w0.out;
  const int col = cb * 32 + i;
  const int u = col / rpad, j = col - u * rpad;
  const uint16_t *arow = p.zero_row;
  int step = 0;
  if (p.pkh) { /* the row pointer straight from the plan (slot clamped; used only below U) */
    const uint16_t *A = plan_ptr(p, p.pkh, u < AOS_PLAN_MAXU ? u : AOS_PLAN_MAXU - 1, true);
    if (u < U && A) {
      arow = A + (size_t)j * in + (size_t)rb * 32 + 8 * c;
      step = 16;
    }
  } else if (u < U) {
    const int aid = __hip_atomic_load(&p.plan->list[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint16_t *A = p.htab.A[aid];
    if (A) {
      arow = A + (size_t)j * in + (size_t)rb * 32 + 8 * c;
      step = 16;
    }
  }
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) b[k2] = aos_gld16(arow + step * k2);
}

template <int NV>
__device__ __forceinline__ void h_shrink_partial(const aos_gemv_params &p, int rb, int lane, const uint16_t (&hb)[NV],
                                                 unsigned char *smem, int U, const u32x4 (&pre)[2][2]) {
  const int T = p.T, i = lane & 31, c = lane >> 5;
  uint32_t *hw = (uint32_t *)smem; /* [32 tokens][32 rows] bf16 */
#pragma unroll
  for (int e = 0; e < 8; ++e) hw[lane + 64 * e] = 0u;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  uint16_t *hl = (uint16_t *)smem;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int m = aos_acc_m(v, lane);
    if (m < T) hl[m * 32 + i] = hb[v];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  u32x4 a[2];
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) a[k2] = *(const u32x4 *)(hl + i * 32 + 16 * k2 + 8 * c);
  const int cols = U * p.htab.rpad;
  for (int cb = 0; cb * 32 < cols; ++cb) {
    const int col = cb * 32 + i;
    u32x4 b[2];
    if (cb < 2) { /* loaded right after the wait for the plan */
      b[0] = cb == 0 ? pre[0][0] : pre[1][0];
      b[1] = cb == 0 ? pre[0][1] : pre[1][1];
    } else {
      h_a_load(p, rb, lane, U, cb, b);
    }
    f32x16 acc = {};
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) acc = aos_mfma32(a[k2], b[k2], acc);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int m = aos_acc_m(v, lane);
      if (m < T && col < cols) {
        float *dst = p.hpart + ((size_t)rb * T + m) * p.hstride + col;
        if (p.hdone) aos_publish(dst, acc[v]); /* read by this launch's sum workgroups */
        else *dst = acc[v];
      }
    }
    if (NV < 16) aos_mfma_hold(acc);
  }
}

/* S[t][col] = sum over the row blocks of hpart[rb][t][col] in a fixed order: each thread sums
 * row blocks tid, tid + NT, ... in order, then a butterfly within each wave, then the waves in
 * order. */
constexpr int HSUM_V = AOS_HSUM_V;
template <int NT>
__device__ __forceinline__ void hsum_block(const aos_hsum_params &hs, int b, unsigned char *smem) {
  float *red = (float *)smem; /* [HSUM_V][NT] */
  const int tid = threadIdx.x;
  int U = __builtin_amdgcn_readfirstlane(__hip_atomic_load(&hs.plan->U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  U = U < AOS_PLAN_MAXU ? U : AOS_PLAN_MAXU;
  const int cols = U * hs.rpad;
  float sum[HSUM_V];
  int t[HSUM_V], col[HSUM_V];
#pragma unroll
  for (int k = 0; k < HSUM_V; ++k) {
    const int idx = b * HSUM_V + k;
    t[k] = idx / hs.stride;
    col[k] = idx - t[k] * hs.stride;
    sum[k] = 0.0f;
  }
  for (int r0 = 0; r0 < hs.RB; r0 += 4 * NT) {
    float v[4][HSUM_V];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = r0 + q * NT + tid;
#pragma unroll
      for (int k = 0; k < HSUM_V; ++k) {
        const bool ok = r < hs.RB && t[k] < hs.T && col[k] < cols;
        const float *src = hs.hpart + ((size_t)(ok ? r : 0) * hs.T + (ok ? t[k] : 0)) * hs.stride + (ok ? col[k] : 0);
        v[q][k] = ok ? (hs.coherent ? aos_collect(src) : *src) : 0.0f;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int k = 0; k < HSUM_V; ++k) sum[k] += v[q][k];
  }
  /* across each wave by a butterfly, then the NT / 64 wave sums in wave order */
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int k = 0; k < HSUM_V; ++k) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum[k] = sum[k] + aos_shfl_f(sum[k], lane ^ o);
    if (lane == 0) red[k * (NT / 64) + wave] = sum[k];
  }
  __syncthreads();
  if (tid < HSUM_V) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) v += red[tid * (NT / 64) + w];
    red[tid * (NT / 64)] = v;
  }
  if (tid < HSUM_V && t[tid] < hs.T && col[tid] < cols)
    aos_publish(&hs.S[(size_t)t[tid] * hs.stride + col[tid]], red[tid * (NT / 64)]);
}

/* x staging loads: plain, or device-coherent (sc1) when x was written by this launch. */
template <bool XL>
__device__ __forceinline__ u32x4 x_load(const uint16_t *x, size_t elem, __amdgpu_buffer_rsrc_t rs) {
  if (XL) return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(elem * 2), 0, 16));
  return *(const u32x4 *)(x + elem);
}

/* One poll of n producer lines (lane l reads lines l, l + 64, ...): true if every line equals gen.
 * Loads issued after it (and depending on its result) are not moved above it. */
__device__ __forceinline__ bool poll_lines_once(const uint32_t *lines, int n, uint32_t gen, int lane) {
  bool all = true;
  for (int base = 0; base < n; base += 64) {
    const int i = base + lane;
    const uint32_t v = i < n ? __hip_atomic_load(lines + (size_t)i * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : gen;
    all = all && __ballot(v != gen) == 0ull;
  }
  aos_compiler_barrier();
  return all;
}

/* Row-block group rbg, K split ksi of one matrix (or of the gate/up pair): the workgroup's waves
 * cover p.wr row blocks (wave w: row block p.wr * rbg + w % p.wr, K piece w / p.wr of the split),
 * all reading the one x slice staged for the split. Waves of a row block past the matrix (the
 * last group of a matrix whose row blocks wr does not divide) read the last row block and store
 * nothing. XL: x is written by earlier workgroups of this launch; the weight ring is primed
 * first, then the workgroup waits (bounded) for its line of xflag to reach p.gen and stages x
 * with device-coherent loads. DP: the direct expand loads (see (4a)) are allowed; the one-launch
 * MLP turns them off, since in its kernel they cost the compiler's promotion of the kernel
 * arguments to registers (the arguments would be copied to private memory). PP: when the plan
 * arrives after the K loop, poll the other producers with the plan's parts (the launch with the
 * router, whose plan comes last; elsewhere the extra loads measured slower). */
template <int NV, bool SW, int W, int D, bool XL = false, bool DP = true, bool PP = false>
__device__ __forceinline__ void gemv_body(const aos_gemv_params &p, int rbg, int ksi, const uint32_t *xflag = nullptr) {
  constexpr int NA = SW ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); /* uniform: keeps the loop scalar */
  const int G = p.w0.G, in = p.w0.in, T = p.T;
  const int i = lane & 31, c = lane >> 5;
  const int WR = p.wr, WK = W / WR;
  const int wr = wave % WR, wk = wave / WR;
  const bool live = rbg * WR + wr < p.w0.RB;
  const int rb = live ? rbg * WR + wr : p.w0.RB - 1;
  const int row = rb * 32 + i;
  const uint32_t qmask = aos_q4_mask(), qexp = aos_q4_exp();

  float acc0[NV], acc1[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    acc0[v] = 0.0f;
    acc1[v] = 0.0f;
  }

  /* the expand: steps q of each module are dealt round-robin to the row block's ks workgroups
   * and then to the waves of its K pieces (q = ksi + ks * (wk + WK * j)); the SwiGLU kernel loads
   * its first step's operands ahead of the K loop, the single-matrix kernel keeps its registers
   * (and its occupancy) and loads them after the K loop */
  const bool expands = p.has_expand != 0;
  const bool fused = p.sync != nullptr || p.pre_lines != nullptr; /* S (and the plan) are produced by this launch */
  int hU = 0;
  u32x4 hpre[2][2];
  const int q_first = ksi + p.ks * wk, q_step = p.ks * WK;
  int nq0 = 0, nq1 = 0;
  ExpandStep e0, e1;
  if (expands && !fused) {
    const int U = __builtin_amdgcn_readfirstlane(p.plan->U);
    nq0 = p.tab0.rpad ? U * p.tab0.rpad / 16 : 0;
    nq1 = (SW && p.tab1.rpad) ? U * p.tab1.rpad / 16 : 0;
    if (SW && q_first < nq0) expand_load(p, p.tab0, p.pk0, p.S0, p.s_stride0, q_first, row, lane, e0);
    if (SW && q_first < nq1) expand_load(p, p.tab1, p.pk1, p.S1, p.s_stride1, q_first, row, lane, e1);
  }
  /* a fused launch whose plan comes from an earlier launch (only S is produced here): the plan and
   * the first step's B fragments load before the K loop, so that after it only S is waited for.
   * Not with XL: the one-launch MLP's down GEMV reads a plan built earlier in its own launch. */
  const bool plan_early = !XL && expands && fused && p.pre_lines != nullptr && p.plan_line < 0;
  /* direct: the plan lists the row pointers of every table read through it, so wave 0 waits for
   * every producer's line at once, and the first expand step then costs two round trips (the
   * plan's part with U, then the B fragments and S) rather than five. (Measured and not kept:
   * waiting for the plan before the K loop, when the plan is built from rings already in memory,
   * delays the loop by more than it saves after it.) */
  const bool direct = DP && fused && !XL && expands && p.pre_lines != nullptr && p.pk0 != 0 &&
                      (!SW || p.tab1.rpad == 0 || p.pk1 != 0) && (!SW || p.hpart == nullptr || p.pkh != 0);
  /* single-matrix kernels with the direct loads: the wave's next NB steps (q_first + k q_step,
   * k = 1 .. NB) load with its first, so that its first NB + 1 steps cost the round trips of one */
  constexpr int NB = (SW || NV == 1) ? 0 : 3;
  ExpandStep er[NB > 0 ? NB : 1];
  PlanPart pr[NB > 0 ? NB : 1];
  if (plan_early) {
    int U = __builtin_amdgcn_readfirstlane(p.plan->U);
    U = U < AOS_PLAN_MAXU ? U : AOS_PLAN_MAXU;
    nq0 = p.tab0.rpad ? U * p.tab0.rpad / 16 : 0;
    nq1 = (SW && p.tab1.rpad) ? U * p.tab1.rpad / 16 : 0;
    hU = U;
    if (q_first < nq0) expand_load_b(p, p.tab0, p.pk0, q_first, row, lane, e0, false);
    if (SW && q_first < nq1) expand_load_b(p, p.tab1, p.pk1, q_first, row, lane, e1, false);
  }
  {
    const int gw0 = (int)((long)ksi * G / p.ks), gw1 = (int)((long)(ksi + 1) * G / p.ks);
    const int GR = gw1 - gw0;
    const int ga = gw0 + wk * GR / WK, gb = gw0 + (wk + 1) * GR / WK, ng = gb - ga;

    /* (1) first x staging loads, ahead of the weights. Loads are unconditional (addresses
     * clamped into range) so no control flow separates them from their use and the compiler
     * can wait for exactly the load it needs. */
    const int xchunks = GR * 8; /* 16-byte chunks per token row */
    const int nx = T * xchunks;
    const __amdgpu_buffer_rsrc_t xrs = /* unused (and removed) unless XL */
        __builtin_amdgcn_make_buffer_rsrc((void *)p.x, (short)0, T * in * 2, 0x00020000);
    u32x4 xv[XE];
    auto x_first = [&]() {
#pragma unroll
      for (int j = 0; j < XE; ++j) {
        int idx = tid + j * 64 * W;
        idx = idx < nx ? idx : idx % nx; /* surplus lanes re-read chunks spread over x (a single
                                        * clamped chunk would be one cache line hit by every lane) */
        const int t = idx / xchunks, r = idx - t * xchunks;
        xv[j] = x_load<XL>(p.x, (size_t)t * in + (size_t)gw0 * 64 + r * 8, xrs);
      }
    };
    if (!XL) x_first();

    /* (2) the ring: groups ga .. ga+D-1. The host sizes the splits so that every wave has at
     * least one group; a wave without one still loads group ga (in range: ga < gw1 <= G) and
     * never uses it. */
    const u32x4 *q0 = (const u32x4 *)p.w0.qt + ((size_t)rb * G + ga) * 64 + lane;
    const uint32_t *s0 = p.w0.sb + ((size_t)rb * G + ga) * 32 + i;
    const u32x4 *q1 = SW ? (const u32x4 *)p.w1.qt + ((size_t)rb * G + ga) * 64 + lane : nullptr;
    const uint32_t *s1 = SW ? p.w1.sb + ((size_t)rb * G + ga) * 32 + i : nullptr;
    u32x4 wa[D], wb[D];
    uint32_t sa[D], sb[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int jj = d < ng ? d : (ng > 0 ? ng - 1 : 0);
      wa[d] = q0[(size_t)jj * 64];
      sa[d] = s0[(size_t)jj * 32];
      if (SW) {
        wb[d] = q1[(size_t)jj * 64];
        sb[d] = s1[(size_t)jj * 32];
      }
    }

    if (XL) { /* x is being produced by this launch: wait for it with the weights in flight (if
               * the wait gives up, the call is reported as timed out and its output is invalid) */
      if (tid == 0 && !aos_wait_gen(xflag, p.gen) && p.timeout)
        __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      lds_barrier();
      x_first();
    }

    /* (3) x -> LDS (rest of the staging after the ring is in flight), group sums. LDS holds
     * 128 zero bytes (read by lanes without a token), the T x rows, then the group sums. */
    uint16_t *xl = (uint16_t *)(smem + 128);
    float *xs = (float *)(smem + 128 + (size_t)T * GR * 128);
    if (tid < 32) ((uint32_t *)smem)[tid] = 0u;
    const int xstride = GR * 64;
#pragma unroll
    for (int j = 0; j < XE; ++j) {
      const int idx = tid + j * 64 * W;
      if (idx < nx) {
        const int t = idx / xchunks, r = idx - t * xchunks;
        *(u32x4 *)(xl + (size_t)t * xstride + r * 8) = xv[j];
      }
    }
    for (int idx = tid + XE * 64 * W; idx < nx; idx += 64 * W) {
      const int t = idx / xchunks, r = idx - t * xchunks;
      *(u32x4 *)(xl + (size_t)t * xstride + r * 8) = x_load<XL>(p.x, (size_t)t * in + (size_t)gw0 * 64 + r * 8, xrs);
    }
    lds_barrier();
    for (int idx = tid; idx < T * GR * 2; idx += 64 * W) {
      const int t = idx / (GR * 2), rem = idx - t * GR * 2;
      const u32x4 *src = (const u32x4 *)(xl + (size_t)t * xstride + rem * 32);
      const u32x4 v0 = src[0], v1 = src[1], v2 = src[2], v3 = src[3];
      const uint32_t w[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                              v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
      float s = 0.0f; /* the 32 elements in order */
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s += __builtin_bit_cast(float, w[e] << 16);
        s += __builtin_bit_cast(float, w[e] & 0xffff0000u);
      }
      xs[idx] = s;
    }
    lds_barrier();

    /* (4) consume the ring, refilling each slot D groups ahead (refills past the end reload
     * the last group and are never used). x fragment address: lanes with a token step through
     * their row, the others stay on the zero block. */
    const int xbase = i < T ? 128 + i * xstride * 2 + 64 * c : 0;
    const int xmult = i < T ? 128 : 0;
    for (int base = 0; base < ng; base += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int j = base + d;
        if (j < ng) {
          const int gl = ga + j - gw0;
          f32x16 t0 = {}, t1 = {};
          u32x4 a[4];
#pragma unroll
          for (int st = 0; st < 4; ++st)
            a[st] = *(const u32x4 *)(smem + xbase + (size_t)gl * xmult + 16 * st);
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            t0 = aos_mfma32(a[st], aos_q4_magic(wa[d][st], qmask, qexp), t0);
            if (SW) t1 = aos_mfma32(a[st], aos_q4_magic(wb[d][st], qmask, qexp), t1);
          }
          apply_group<NV>(t0, sa[d], xs, GR, gl, T, lane, acc0);
          if (SW) apply_group<NV>(t1, sb[d], xs, GR, gl, T, lane, acc1);
        }
        int jn = j + D;
        jn = jn < ng ? jn : ng - 1;
        wa[d] = q0[(size_t)jn * 64];
        sa[d] = s0[(size_t)jn * 32];
        if (SW) {
          wb[d] = q1[(size_t)jn * 64];
          sb[d] = s1[(size_t)jn * 32];
        }
      }
    }
  }

  /* (4a) fused launch. The producers have the lowest workgroup ids, so they are dispatched before
   * any GEMV workgroup, and none of them waits on a GEMV workgroup. With per-producer lines, wave 0
   * first waits for the plan's line (when the plan is built in this launch), the first expand
   * step's B fragments are loaded, then wave 0 waits for every producer's line before S is read;
   * otherwise it waits for this workgroup's own ready flag, raised once every producer is done.
   * The waits are bounded: past about a second they give up, set p.timeout and the workgroup
   * finishes without the expand or the h shrink; the call's output is then invalid and the layer
   * reports the timeout. */
  if (fused && direct) {
    /* each wave on its own. Plan built by this launch: one poll of every producer line; if all are
     * up, round trip 1 (the plan's parts and U, kept per lane so that nothing waits for it before
     * the other loads go out) and round trip 2 (the B fragments, S, the h shrink's A_down pointers
     * and fragments) follow at once; if not, the wave waits for the plan's line, loads the plan's
     * parts and the B fragments, and only then waits for the other lines and loads S (the B loads
     * then overlap the shrink's tail). Plan from an earlier launch: wait, then S. */
    if (!plan_early) {
      const bool all_up = poll_lines_once(p.pre_lines, p.n_pre_lines, p.gen, lane);
      bool ready = all_up || aos_wait_lines(p.pre_lines + (size_t)p.plan_line * 32, 1, p.gen, lane);
      PlanPart pe0 = {}, pe1 = {};
      int Ue = 0;
      if (ready) {
        /* with the plan's parts, one more poll of the lines (their values are read once the parts
         * have arrived, so it costs no round trip of its own) */
        uint32_t pv = p.gen;
        if (PP && !all_up && p.n_pre_lines <= 64 && lane < p.n_pre_lines)
          pv = __hip_atomic_load(p.pre_lines + (size_t)lane * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (p.tab0.rpad) {
          pe0 = expand_plan_part(p, p.tab0.rpad, p.pk0, q_first, lane, e0);
#pragma unroll
          for (int k = 0; k < NB; ++k)
            pr[k] = expand_plan_part(p, p.tab0.rpad, p.pk0, q_first + (k + 1) * q_step, lane, er[k]);
        }
        if (SW && p.tab1.rpad) pe1 = expand_plan_part(p, p.tab1.rpad, p.pk1, q_first, lane, e1);
        Ue = (int)__hip_atomic_load(&p.plan->U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        Ue = Ue < AOS_PLAN_MAXU ? Ue : AOS_PLAN_MAXU;
        if (SW && p.hpart && wave == 0) {
          h_a_load(p, rb, lane, Ue, 0, hpre[0]);
          h_a_load(p, rb, lane, Ue, 1, hpre[1]);
        }
        if (p.tab0.rpad) {
          const int nq = Ue * p.tab0.rpad / 16;
          expand_b_of(p, p.tab0.rpad, pe0, q_first < nq, row, lane, e0);
#pragma unroll
          for (int k = 0; k < NB; ++k)
            expand_b_of(p, p.tab0.rpad, pr[k], q_first + (k + 1) * q_step < nq, row, lane, er[k]);
        }
        if (SW && p.tab1.rpad) expand_b_of(p, p.tab1.rpad, pe1, q_first < Ue * p.tab1.rpad / 16, row, lane, e1);
        if (!all_up && !(PP && p.n_pre_lines <= 64 && __ballot(pv != p.gen) == 0ull))
          ready = aos_wait_lines(p.pre_lines, p.n_pre_lines, p.gen, lane);
        aos_compiler_barrier();
      }
      if (ready) {
        if (p.tab0.rpad) {
          const int nq = Ue * p.tab0.rpad / 16;
          expand_s_of(p, p.tab0.rpad, pe0, q_first < nq, p.S0, p.s_stride0, lane, e0);
#pragma unroll
          for (int k = 0; k < NB; ++k)
            expand_s_of(p, p.tab0.rpad, pr[k], q_first + (k + 1) * q_step < nq, p.S0, p.s_stride0, lane, er[k]);
        }
        if (SW && p.tab1.rpad)
          expand_s_of(p, p.tab1.rpad, pe1, q_first < Ue * p.tab1.rpad / 16, p.S1, p.s_stride1, lane, e1);
        const int U = __builtin_amdgcn_readfirstlane(Ue);
        nq0 = p.tab0.rpad ? U * p.tab0.rpad / 16 : 0;
        nq1 = (SW && p.tab1.rpad) ? U * p.tab1.rpad / 16 : 0;
        hU = U;
      } else {
        if (lane == 0 && p.timeout) __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        nq0 = 0;
        nq1 = 0;
        hU = 0;
      }
    } else { /* plan and the first step's B fragments loaded before the K loop */
      const bool ready = aos_wait_lines(p.pre_lines, p.n_pre_lines, p.gen, lane);
      if (!ready) {
        if (lane == 0 && p.timeout) __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        nq0 = 0;
        nq1 = 0;
        hU = 0;
      } else {
        if (SW && p.hpart && wave == 0) {
          h_a_load(p, rb, lane, hU, 0, hpre[0]);
          h_a_load(p, rb, lane, hU, 1, hpre[1]);
        }
        if (q_first < nq0) expand_load_s(p, p.tab0, p.S0, p.s_stride0, q_first, lane, e0, true);
        if (SW && q_first < nq1) expand_load_s(p, p.tab1, p.S1, p.s_stride1, q_first, lane, e1, true);
        if (p.tab0.rpad && q_first + q_step < nq0) { /* the next steps: plan parts, then B and S */
#pragma unroll
          for (int k = 0; k < NB; ++k)
            pr[k] = expand_plan_part(p, p.tab0.rpad, p.pk0, q_first + (k + 1) * q_step, lane, er[k]);
#pragma unroll
          for (int k = 0; k < NB; ++k) {
            const bool in = q_first + (k + 1) * q_step < nq0;
            expand_b_of(p, p.tab0.rpad, pr[k], in, row, lane, er[k]);
            expand_s_of(p, p.tab0.rpad, pr[k], in, p.S0, p.s_stride0, lane, er[k]);
          }
        }
      }
    }
  } else if (fused) {
    __shared__ uint32_t ok, ok2;
    const bool lines = p.pre_lines != nullptr;
    if (wave == 0) {
      bool done = true;
      if (lines) {
        if (p.plan_line >= 0) done = aos_wait_lines(p.pre_lines + (size_t)p.plan_line * 32, 1, p.gen, lane);
      } else if (lane == 0) {
        done = aos_wait_gen(p.flags + ((size_t)ksi * p.nrbg + rbg) * 32, p.gen);
      }
      if (lane == 0) {
        ok = done ? 1u : 0u;
        if (!done && p.timeout) __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    }
    lds_barrier();
    if (ok && expands && !plan_early) {
      int U = __builtin_amdgcn_readfirstlane(
          __hip_atomic_load(&p.plan->U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      U = U < AOS_PLAN_MAXU ? U : AOS_PLAN_MAXU;
      nq0 = p.tab0.rpad ? U * p.tab0.rpad / 16 : 0;
      nq1 = (SW && p.tab1.rpad) ? U * p.tab1.rpad / 16 : 0;
      hU = U;
    }
    /* the h shrink's first A_down fragments (wave 0 forms the partials at the end), and the first
     * expand step's plan part */
    if (SW && p.hpart && wave == 0 && ok) {
      h_a_load(p, rb, lane, hU, 0, hpre[0]);
      h_a_load(p, rb, lane, hU, 1, hpre[1]);
    }
    if (!plan_early) {
      if (q_first < nq0) expand_load_b(p, p.tab0, p.pk0, q_first, row, lane, e0, true);
      if (SW && q_first < nq1) expand_load_b(p, p.tab1, p.pk1, q_first, row, lane, e1, true);
    }
    if (lines) {
      if (wave == 0) {
        const bool done = aos_wait_lines(p.pre_lines, p.n_pre_lines, p.gen, lane);
        if (lane == 0) {
          ok2 = done ? 1u : 0u;
          if (!done && p.timeout) __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
      }
      lds_barrier();
      if (!ok2) {
        nq0 = 0;
        nq1 = 0;
        hU = 0;
      }
    }
  }

  /* (4b) the expand, added to the waves' accumulators */
  if (expands) {
    f32x16 f0 = {}, f1 = {};
    if (direct) {
      /* loaded above */
    } else if (fused) {
      if (q_first < nq0) expand_load_s(p, p.tab0, p.S0, p.s_stride0, q_first, lane, e0, true);
      if (SW && q_first < nq1) expand_load_s(p, p.tab1, p.S1, p.s_stride1, q_first, lane, e1, true);
    } else if (!SW && q_first < nq0) {
      expand_load(p, p.tab0, p.pk0, p.S0, p.s_stride0, q_first, row, lane, e0);
    }
    if (q_first < nq0) expand_apply(e0, f0);
    if (SW && q_first < nq1) expand_apply(e1, f1);
    const int nb = direct ? NB : 0; /* steps after the first already loaded */
#pragma unroll
    for (int k = 0; k < NB; ++k)
      if (k < nb && q_first + (k + 1) * q_step < nq0) expand_apply(er[k], f0);
    if (SW && NV > 1) { /* several steps per module per wave (8 tokens and up): both rests together */
      if (q_first + q_step < nq0 || q_first + q_step < nq1)
        expand_rest2<2>(p, q_first + q_step, nq0, q_first + q_step, nq1, q_step, row, lane, fused, f0, f1);
    } else {
      if (q_first + (nb + 1) * q_step < nq0)
        expand_rest<4>(p, p.tab0, p.pk0, p.S0, p.s_stride0, q_first + (nb + 1) * q_step, q_step, nq0, row, lane, fused,
                       f0);
      if (SW && q_first + q_step < nq1)
        expand_rest<4>(p, p.tab1, p.pk1, p.S1, p.s_stride1, q_first + q_step, q_step, nq1, row, lane, fused, f1);
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      acc0[v] += f0[v];
      if (SW) acc1[v] += f1[v];
    }
    if (NV < 16) {
      aos_mfma_hold(f0);
      if (SW) aos_mfma_hold(f1);
    }
  }

  /* (5) fixed-order reduction over the K pieces of each row block (LDS reused once every wave is
   * done with x): wave wr sums the pieces k = 0 .. WK - 1 (waves wr + WR k) in order */
  float *red = (float *)smem;
  lds_barrier();
  if (WK > 1) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      red[(wave * NA * NV + v) * 64 + lane] = acc0[v];
      if (SW) red[(wave * NA * NV + NV + v) * 64 + lane] = acc1[v];
    }
  }
  lds_barrier();
  if (wk != 0) return;
  if (WK > 1) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float a0 = red[(wr * NA * NV + v) * 64 + lane], a1 = SW ? red[(wr * NA * NV + NV + v) * 64 + lane] : 0.0f;
      for (int k = 1; k < WK; ++k) {
        const int w = wr + WR * k;
        a0 += red[(w * NA * NV + v) * 64 + lane];
        if (SW) a1 += red[(w * NA * NV + NV + v) * 64 + lane];
      }
      acc0[v] = a0;
      acc1[v] = a1;
    }
  }
  if (!live) return;

  /* (6) fixed-order reduction over the workgroups of this row block: the last one sums */
  const int nsplit = p.ks;
  if (nsplit > 1) {
    float *part = p.part + ((size_t)rb * nsplit + ksi) * (NA * NV * 64);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      aos_publish(part + v * 64 + lane, acc0[v]);
      if (SW) aos_publish(part + (NV + v) * 64 + lane, acc1[v]);
    }
    uint32_t old = 0;
    if (lane == 0) old = aos_arrive(&p.counters[rb]);
    old = aos_shfl(old, 0);
    if (old != (uint32_t)nsplit - 1u) return;
    if (lane == 0) aos_reset(&p.counters[rb]);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      acc0[v] = 0.0f;
      acc1[v] = 0.0f;
    }
    /* partials are read 4 at a time (all loads in flight together) and summed in order */
    for (int k0 = 0; k0 < nsplit; k0 += 4) {
      float v0[4][NV], v1[4][NV];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int k = k0 + kk < nsplit ? k0 + kk : nsplit - 1;
        const float *pp = p.part + ((size_t)rb * nsplit + k) * (NA * NV * 64);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          v0[kk][v] = aos_collect(pp + v * 64 + lane);
          v1[kk][v] = SW ? aos_collect(pp + (NV + v) * 64 + lane) : 0.0f;
        }
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        if (k0 + kk < nsplit) {
#pragma unroll
          for (int v = 0; v < NV; ++v) {
            acc0[v] += v0[kk][v];
            if (SW) acc1[v] += v1[kk][v];
          }
        }
    }
  }

  /* (7) epilogue */
  const int out = p.w0.out;
  uint16_t hb[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int m = aos_acc_m(v, lane);
    hb[v] = 0;
    if (m >= T) continue;
    if (!SW) {
      if (p.yf) p.yf[(size_t)m * out + row] = acc0[v];
      else p.y[(size_t)m * out + row] = aos_f32_to_bf16(acc0[v]);
    } else {
      const float gt = acc0[v], up = acc1[v];
      const float sg = 1.0f / (1.0f + expf(-gt));
      hb[v] = aos_f32_to_bf16((gt * sg) * up);
      if (p.hdone) /* read by this launch's down workgroups */
        __hip_atomic_store(p.y + (size_t)m * out + row, hb[v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        p.y[(size_t)m * out + row] = hb[v];
    }
  }
  if (SW && p.hpart && hU > 0) h_shrink_partial<NV>(p, rb, lane, hb, smem, hU, hpre);
  /* one-launch decode: this row block of h (and its partials) is out; the last row block raises
   * the lines of every workgroup that reads h */
  if (SW && p.hdone) {
    uint32_t last = 0;
    if (lane == 0) last = aos_arrive_tree(p.hdone, (uint32_t)rb, (uint32_t)p.w0.RB) ? 1u : 0u;
    last = aos_shfl(last, 0);
    if (last) {
      for (uint32_t c2 = lane; c2 < p.n_hflags; c2 += 64)
        __hip_atomic_store(p.hflags + (size_t)c2 * 32, p.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}


/* Producer workgroup b of a fused launch: a shrink workgroup (or, with fp.hsum, a sum of the h
 * shrink's partials). Then, with per-producer lines, the workgroup that completed a row block of
 * the shrink (or the plan, or a sum) raises that producer's line to fp.gen; otherwise every
 * producer counts itself in and the last one raises every GEMV workgroup's ready flag to fp.gen.
 * route_flag (may be NULL): the plan workgroup first waits, bounded, until the launch's routers
 * have raised route_flag to fp.gen and only then reads the rings (with device-scope loads); if
 * that wait gives up it publishes an empty plan instead. start_flag (may be NULL): the producer's
 * inputs are written by earlier workgroups of this launch, which raise start_flag to fp.gen. */
template <int NV, int W>
__device__ __forceinline__ void fused_producer(const aos_gemv_fused_params &fp, int b, unsigned char *smem,
                                               const uint32_t *route_flag, const uint32_t *start_flag = nullptr) {
  __shared__ uint32_t last, routed, started;
  if (start_flag) { /* the inputs come from earlier workgroups of this launch */
    if (threadIdx.x == 0) {
      const bool done = aos_wait_gen(start_flag, fp.gen);
      started = done ? 1u : 0u;
      if (!done && fp.gp[0].timeout)
        __hip_atomic_store(fp.gp[0].timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
  }
  bool done_here = true; /* this workgroup completes its producer (shrink: see shrink_block) */
  if (fp.hsum) {
    if (!start_flag || started) hsum_block<64 * W>(fp.hs, b, smem);
  } else {
    const int lrb = b % fp.pre_rows, ksi = b / fp.pre_rows;
    bool run = true;
    if (route_flag && fp.sp.plan_build.plan && lrb == fp.pre_rows - 1 && ksi == 0) {
      if (threadIdx.x == 0) {
        const bool done = aos_wait_gen(route_flag, fp.gen);
        routed = done ? 1u : 0u;
        if (!done) {
          if (fp.gp[0].timeout) __hip_atomic_store(fp.gp[0].timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
          __hip_atomic_store(&fp.sp.plan_build.plan->U, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      __syncthreads();
      run = routed != 0u;
    }
    done_here = run ? aos_shrink::shrink_block<NV, W, 4>(fp.sp, lrb, ksi, smem) : true;
  }
  /* the partials, S and the plan went out as device-scope stores: wait for them, then count
   * this workgroup in (no cache write-back is needed) */
  aos_mem_wait();
  __syncthreads();
  if (fp.lines) { /* per-producer lines: thread 0 (in wave 0, which decided) raises this one's */
    if (threadIdx.x == 0 && done_here) aos_raise(fp.lines + (size_t)(fp.hsum ? b : b % fp.pre_rows) * 32, fp.gen);
    return;
  }
  if (threadIdx.x == 0) last = aos_arrive_tree(fp.sync, (uint32_t)b, (uint32_t)fp.n_pre) ? 1u : 0u;
  __syncthreads();
  if (last) /* every producer is done: raise the GEMV workgroups' flags */
    for (uint32_t c = threadIdx.x; c < fp.n_cons; c += blockDim.x)
      __hip_atomic_store(fp.flags + (size_t)c * 32, fp.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace aos_gemv

#endif
