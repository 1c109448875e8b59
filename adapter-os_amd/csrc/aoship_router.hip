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
 * Selection orders 128-bit composite keys (total-order score key, stable_id, index), which makes
 * every key unique, so it yields exactly the order of Rust's stable sort: for N <= 64 by ranking
 * (each lane counts the smaller keys), for larger N by a wavefront bitonic sort, streaming the
 * adapters through the wave 56 at a time while the best 8 stay in lanes 0..7. The softmax uses a correctly rounded float64 exp.
 *
 * Optionally the priors are first computed from router features: one workgroup per token, up to
 * 16 waves, each wave computing whole (adapter, token) dot products in float32 with a fixed order
 * (lane l sums elements 256k + 4l + e with fused multiply-adds, then a xor butterfly), all of a
 * dot product's loads issued before its arithmetic; the priors go through LDS to wave 0, which
 * routes.
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

template <bool LDS>
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
    const float prior = LDS ? priors[i] : priors[i];
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
    if (n <= AOS_WAVE) {
      /* n <= 64: rank selection. Keys are unique (they end in the index), so lane i's rank is
       * the number of smaller keys; the 8 smallest are scattered to lanes 0..7 through LDS. */
      __shared__ uint64_t keys[2 * AOS_WAVE];
      __shared__ uint64_t top[2 * 8];
      keys[2 * lane] = ka;
      keys[2 * lane + 1] = kb;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      int rank = 0;
      for (int j = 0; j < n; ++j) {
        const uint64_t a = keys[2 * j], b = keys[2 * j + 1];
        rank += key_less(a, b, ka, kb) ? 1 : 0;
      }
      if (lane < n && rank < 8) {
        top[2 * rank] = ka;
        top[2 * rank + 1] = kb;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      const int src = lane < 8 && lane < n ? lane : -1;
      ka = src >= 0 ? top[2 * src] : ~0ull;
      kb = src >= 0 ? top[2 * src + 1] : ~0ull;
    } else {
      bitonic64(ka, kb, lane);
    }
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

/* Dot products of router features (staged in LDS) with router weight rows: lane l sums elements
 * 256k + 4l + e (k ascending, e = 0..3) with fused multiply-adds, then a xor butterfly over the
 * 64 lanes. Up to 16 chunks of 256 weights are loaded before any arithmetic. */
__device__ __forceinline__ float router_dot(const float *f_lds, const float *w, int d, int lane) {
  const float4 *f4 = (const float4 *)f_lds;
  const float4 *w4 = (const float4 *)w;
  const int nk = d >> 8;    /* full 256-element chunks */
  const int tail = d & 255; /* multiple of 4 */
  float acc = 0.0f;
  for (int k0 = 0; k0 < nk; k0 += 16) {
    float4 wv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int k = k0 + j < nk ? k0 + j : nk - 1;
      wv[j] = w4[k * 64 + lane];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (k0 + j < nk) {
        const float4 fv = f4[(k0 + j) * 64 + lane];
        acc = fmaf(wv[j].x, fv.x, acc);
        acc = fmaf(wv[j].y, fv.y, acc);
        acc = fmaf(wv[j].z, fv.z, acc);
        acc = fmaf(wv[j].w, fv.w, acc);
      }
    }
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
  return acc;
}

/* Routing from priors already in memory: one wave per token. */
__global__ void __launch_bounds__(64) aos_route_kernel(aos_route_params p) {
  const int t = blockIdx.x;
  route_one<false>(p, p.priors_in + (size_t)t * p.n, t, threadIdx.x);
}

/* Routing from router features: one workgroup per token; wave w computes the priors of
 * adapters w, w + W, ... into LDS (and priors_out), then wave 0 routes. */
__global__ void __launch_bounds__(1024) aos_route_features_kernel(aos_route_params p) {
  extern __shared__ float lds[]; /* features [d], then priors [n] */
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  float *lds_f = lds, *lds_priors = lds + p.d;
  const float4 *f4 = (const float4 *)(p.features + (size_t)t * p.d);
  for (int e = threadIdx.x; e < p.d / 4; e += blockDim.x) ((float4 *)lds_f)[e] = f4[e];
  __syncthreads();
  for (int a = wave; a < p.n; a += nw) {
    const float v = router_dot(lds_f, p.router_w + (size_t)a * p.d, p.d, lane);
    if (lane == 0) {
      lds_priors[a] = v;
      if (p.priors_out) p.priors_out[(size_t)t * p.n + a] = v;
    }
  }
  __syncthreads();
  if (wave == 0) route_one<true>(p, lds_priors, t, lane);
}

}  // namespace

extern "C" int aos_launch_route(const aos_route_params *p, const aos_launch_ctx *ctx) {
  if (p->features) {
    const int waves = p->n < 16 ? p->n : 16;
    AOS_LAUNCH(ctx, aos_route_features_kernel, dim3(p->T), dim3(64 * waves),
               (size_t)(p->d + p->n) * sizeof(float), *p);
  } else {
    AOS_LAUNCH(ctx, aos_route_kernel, dim3(p->T), dim3(64), 0, *p);
  }
  return (int)hipGetLastError();
}
