/*
 * aoship_router.hip — K-sparse router on gfx950: one wavefront per token.
 *
 * Follows Router::route_with_adapter_info_and_scope_with_ctx in deterministic mode with an
 * empty feature vector (crates/adapteros-lora-router/src/router.rs:1567-1952):
 *   validate priors finite (:611-625, check_numerics numerics/src/noise.rs:308-316)
 *   score = ((prior + 0.0) - 0.0) * routing_bias * 1.0             (:1664-1676, scoring.rs:35-37)
 *   stable sort: score DESC by f32::total_cmp, stable_id ASC, index ASC    (:234-264)
 *   top-K, float64 softmax with Kahan summation in top-K order            (:1340-1411)
 *   entropy floor max(g, eps / K), float32 renormalisation                (:1818-1842)
 *   Q15 = clamp(round_half_away(g * 32767.0f), 0, 32767)                  (quantization.rs:172-175)
 *   canonical re-sort: Q15 DESC, score DESC, stable_id ASC, index ASC     (:1310-1325)
 *
 * Selection is a wavefront bitonic sort over 128-bit composite keys
 * (total-order score key, stable_id, index), which makes every key unique, so the sort yields
 * exactly the order of Rust's stable sort. N > 64 adapters are streamed through the wave 56 at
 * a time while the best 8 stay in lanes 0..7. The softmax uses a correctly rounded float64 exp.
 *
 * Optionally the priors are first computed from router features: one wave per (adapter, token)
 * dot product in float32 with a fixed order (lane l sums elements 256k + 4l + e, then a xor
 * butterfly); the workgroups of one token hand over to the last one to finish, which routes.
 */
#include "aos_exp.h"
#include "aoship_device.h"
#include "aoship_internal.h"
#include <hip/hip_ext.h>

namespace {

__device__ __forceinline__ uint32_t score_key_desc(float x) {
  int32_t b = __builtin_bit_cast(int32_t, x);
  int32_t t = b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
  uint32_t asc = (uint32_t)t ^ 0x80000000u;
  return 0xffffffffu - asc;
}

__device__ __forceinline__ float score_from_key(uint32_t desc) {
  uint32_t asc = 0xffffffffu - desc;
  int32_t t = (int32_t)(asc ^ 0x80000000u);
  int32_t b = t ^ (int32_t)(((uint32_t)(t >> 31)) >> 1);
  return __builtin_bit_cast(float, b);
}

__device__ __forceinline__ bool key_less(uint64_t a0, uint64_t b0, uint64_t a1, uint64_t b1) {
  return a0 < a1 || (a0 == a1 && b0 < b1);
}

/* Ascending bitonic sort of one 128-bit key per lane across the 64-lane wavefront. */
__device__ __forceinline__ void bitonic64(uint64_t &ka, uint64_t &kb, int lane) {
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      int partner = lane ^ j;
      uint64_t oa = aos_shfl64(ka, partner);
      uint64_t ob = aos_shfl64(kb, partner);
      bool up = (lane & k) == 0;
      bool lower = (lane & j) == 0;
      bool take = (lower == up) ? key_less(oa, ob, ka, kb) : key_less(ka, kb, oa, ob);
      if (take) {
        ka = oa;
        kb = ob;
      }
    }
  }
}

__device__ __forceinline__ double rust_f64_max(double a, double b) {
  if (a != a) return b;
  if (b != b) return a;
  return a > b ? a : (b > a ? b : a);
}

__device__ __forceinline__ float rust_f32_max(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  return a > b ? a : (b > a ? b : a);
}

/* f32::round (half away from zero) followed by `as i32` and the Q15 clamp. */
__device__ __forceinline__ int quantize_q15(float g) {
  float v = g * 32767.0f;
  if (v != v) return 0;
  float r = truncf(v);
  if (fabsf(v - r) >= 0.5f) r += copysignf(1.0f, v);
  if (r <= 0.0f) return 0;
  if (r >= 32767.0f) return 32767;
  return (int)r;
}

__device__ void route_one(const aos_route_params &p, const float *priors, int t, int lane) {
  const int n = p.n;
  /* every prior is checked for finiteness, allowed or not (validate_router_inputs); the chunked
   * passes below visit each index exactly once */
  bool bad = false;
  uint64_t ka = ~0ull, kb = ~0ull;
  int m_allowed = 0;
  auto load_key = [&](int i, uint64_t &a, uint64_t &b) -> bool {
    a = ~0ull;
    b = ~0ull;
    if (i >= n) return false;
    const float prior = aos_collect(priors + i);
    if (!__builtin_isfinite(prior)) bad = true;
    if (p.allowed && !p.allowed[i]) return false;
    float sim = (prior + 0.0f) - 0.0f;
    float score = sim * p.bias;
    score = score * 1.0f;
    if (!__builtin_isfinite(score)) bad = true;
    uint64_t sid = p.stable_id ? p.stable_id[i] : 0ull;
    a = ((uint64_t)score_key_desc(score) << 32) | (sid >> 32);
    b = ((sid & 0xffffffffull) << 32) | (uint64_t)(uint32_t)i;
    return true;
  };
  {
    bool v = load_key(lane, ka, kb);
    m_allowed += __popcll(__ballot(v));
    bitonic64(ka, kb, lane);
  }
  for (int base = AOS_WAVE; base < n; base += AOS_WAVE - 8) {
    bool v = false;
    if (lane >= 8) {
      uint64_t a, b;
      v = load_key(base + lane - 8, a, b);
      ka = a;
      kb = b;
    }
    m_allowed += __popcll(__ballot(v));
    bitonic64(ka, kb, lane);
  }

  aoship_ring_t *ring = p.rings + t;
  const bool any_bad = __ballot(bad) != 0ull;
  int kk = p.k < m_allowed ? p.k : m_allowed;
  if (any_bad || kk <= 0) {
    if (lane < 10) ((uint32_t *)ring)[lane] = 0u;
    if (lane == 0) {
      if (!any_bad) ring->current_pos = (uint32_t)t;
      if (p.status) p.status[t] = any_bad ? -1 : 0;
    }
    return;
  }

  /* Gather the top entries into every lane (uniform from here on). */
  float sc[8];
  uint32_t skey[8], sidx[8];
  uint64_t ssid[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    uint64_t a = aos_shfl64(ka, s), b = aos_shfl64(kb, s);
    skey[s] = (uint32_t)(a >> 32);
    sc[s] = score_from_key(skey[s]);
    ssid[s] = ((a & 0xffffffffull) << 32) | (b >> 32);
    sidx[s] = (uint32_t)b;
  }

  /* deterministic_softmax (router.rs:1340-1411); tau > 0 after sanitising. */
  double mx = -__builtin_inf();
#pragma unroll
  for (int s = 0; s < 8; ++s)
    if (s < kk) mx = rust_f64_max(mx, (double)sc[s]);
  /* lane s evaluates exp for top-K entry s (the same value the serial loop would produce), then
   * every lane gathers the K values and runs the Kahan summation in top-K order */
  double my_e;
  {
    const int s = lane & 7;
    float my_sc = sc[0];
#pragma unroll
    for (int q = 1; q < 8; ++q)
      if (s == q) my_sc = sc[q];
    my_e = aos_exp_cr(((double)my_sc - mx) / (double)p.tau);
  }
  double e[8];
  double sum = 0.0, comp = 0.0;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, my_e);
    const double ex = __builtin_bit_cast(double, aos_shfl64(bits, s));
    if (s < kk) {
      double y = ex - comp;
      double tt = sum + y;
      comp = (tt - sum) - y;
      sum = tt;
      e[s] = ex;
    } else {
      e[s] = 0.0;
    }
  }
  float g[8];
  float uni = 1.0f / (float)kk;
#pragma unroll
  for (int s = 0; s < 8; ++s) g[s] = (sum == 0.0) ? uni : (float)(e[s] / sum);
  float min_gate = p.eps / (float)kk;
#pragma unroll
  for (int s = 0; s < 8; ++s)
    if (s < kk) g[s] = rust_f32_max(g[s], min_gate);
  float S = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s)
    if (s < kk) S += g[s];
  if (!(S > 0.0f)) {
    if (lane < 10) ((uint32_t *)ring)[lane] = 0u;
    if (lane == 0) {
      ring->current_pos = (uint32_t)t;
      if (p.status) p.status[t] = 0;
    }
    return;
  }
  int q[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) q[s] = (s < kk) ? quantize_q15(g[s] / S) : 0;

  /* Canonical order (router.rs:1310-1325): rank of each candidate. */
  int rank[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int r = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j == i || j >= kk) continue;
      bool before = q[j] > q[i] ||
                    (q[j] == q[i] &&
                     (skey[j] < skey[i] ||
                      (skey[j] == skey[i] &&
                       (ssid[j] < ssid[i] || (ssid[j] == ssid[i] && sidx[j] < sidx[i])))));
      r += before ? 1 : 0;
    }
    rank[i] = r;
  }
  if (lane < 8) {
    uint32_t oi = 0;
    int oq = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < kk && rank[i] == lane) {
        oi = sidx[i];
        oq = q[i];
      }
    ring->adapter_indices[lane] = (uint16_t)oi;
    ring->gates_q15[lane] = (int16_t)oq;
  }
  if (lane == 0) {
    ring->top_k = (uint32_t)kk;
    ring->current_pos = (uint32_t)t;
    if (p.status) p.status[t] = 0;
  }
}

__global__ void __launch_bounds__(64) aos_route_kernel(aos_route_params p) {
  const int lane = threadIdx.x;
  const int t = blockIdx.y;
  const float *priors;
  if (p.features) {
    /* priors[t, a] for a = blockIdx.x: lane l accumulates elements 256k + 4l + e (k ascending,
     * e = 0..3) with fused multiply-adds, then a xor butterfly over the 64 lanes. */
    const int a = blockIdx.x;
    const float4 *f4 = (const float4 *)(p.features + (size_t)t * p.d);
    const float4 *w4 = (const float4 *)(p.router_w + (size_t)a * p.d);
    const int nk = p.d >> 8;        /* full 256-element chunks */
    const int tail = p.d & 255;     /* multiple of 4 */
    float acc = 0.0f;
    int k = 0;
    for (; k + 4 <= nk; k += 4) {
      float4 fv[4], wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        fv[j] = f4[(k + j) * 64 + lane];
        wv[j] = w4[(k + j) * 64 + lane];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc = fmaf(wv[j].x, fv[j].x, acc);
        acc = fmaf(wv[j].y, fv[j].y, acc);
        acc = fmaf(wv[j].z, fv[j].z, acc);
        acc = fmaf(wv[j].w, fv[j].w, acc);
      }
    }
    for (; k < nk; ++k) {
      const float4 fv = f4[k * 64 + lane], wv = w4[k * 64 + lane];
      acc = fmaf(wv.x, fv.x, acc);
      acc = fmaf(wv.y, fv.y, acc);
      acc = fmaf(wv.z, fv.z, acc);
      acc = fmaf(wv.w, fv.w, acc);
    }
    if (4 * lane < tail) {
      const float4 fv = f4[nk * 64 + lane], wv = w4[nk * 64 + lane];
      acc = fmaf(wv.x, fv.x, acc);
      acc = fmaf(wv.y, fv.y, acc);
      acc = fmaf(wv.z, fv.z, acc);
      acc = fmaf(wv.w, fv.w, acc);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc = acc + aos_shfl_f(acc, lane ^ o);
    if (lane == 0) aos_publish(p.priors_out + (size_t)t * p.n + a, acc);
    if (gridDim.x > 1) {
      uint32_t old = 0;
      if (lane == 0) old = aos_arrive(&p.counters[t]);
      old = aos_shfl(old, 0);
      if (old != gridDim.x - 1) return;
      if (lane == 0) aos_reset(&p.counters[t]);
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    /* the priors are read back with device-coherent loads below */
    priors = p.priors_out + (size_t)t * p.n;
  } else {
    priors = p.priors_in + (size_t)t * p.n;
  }
  route_one(p, priors, t, lane);
}

}  // namespace

extern "C" int aos_launch_route(const aos_route_params *p, const aos_launch_ctx *ctx) {
  dim3 grid(1, p->T);
  if (p->features) grid.x = p->n; /* one wave per (adapter, token) dot product */
  AOS_LAUNCH(ctx, aos_route_kernel, grid, dim3(64), 0, *p);
  return (int)hipGetLastError();
}
