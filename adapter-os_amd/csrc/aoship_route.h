/*
 * aoship_route.h — the router's device code (selection, float64 softmax, Q15, canonical order,
 * extras, decision hashes, and the router-feature dot products), shared by the routing launches
 * (aoship_router.hip) and the one-token MLP launch that routes its token (aoship_mlp1.hip). The
 * semantics and their reference lines are listed at the top of aoship_router.hip.
 */
#ifndef AOSHIP_ROUTE_H
#define AOSHIP_ROUTE_H

#include "aos_blake3.h"
#include "aos_exp.h"
#include "aoship_device.h"
#include "aoship_internal.h"

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

/* A zero ring; code 0 keeps the token's position (an empty decision), -1 / -2 (errors) do not. */
__device__ __forceinline__ void ring_empty(aoship_ring_t *ring, int32_t *status, int t, int lane, int code) {
  if (lane < 10) ((uint32_t *)ring)[lane] = 0u;
  if (lane == 0) {
    if (code == 0) ring->current_pos = (uint32_t)t;
    if (status) status[t] = code;
  }
}

/* No decision, no hash: 96 zero bytes. */
__device__ __forceinline__ void hash_empty(uint8_t *hashes, int t, int lane) {
  if (hashes && lane < 24) ((uint32_t *)(hashes + (size_t)96 * t))[lane] = 0u;
}

#define AOS_B3_MAX_CHUNKS (AOS_MAX_ADAPTERS * 4 / AOS_B3_CHUNK_LEN + 1)

/* Router::compute_decision_hash (router.rs:1427-1484) with an empty feature vector, for the
 * decision (didx, dq)[0..kk) in canonical order: input = BLAKE3(priors as routed, float32 LE
 * [|| reasoning]), lane c hashing chunk c and lane 0 merging the tree; output = BLAKE3(indices
 * u16 LE || gates i16 LE [|| reasoning]); combined = BLAKE3(input || output [|| reasoning]
 * [|| backend]). Written to hashes[96 t ..]. */
__device__ __noinline__ void decision_hash(uint8_t *hashes, const float *priors, const uint8_t *scope, int n,
                                           const uint32_t *extra, int reasoning, int backend, int t, int lane, int kk,
                                           uint32_t ow0, uint32_t ow1, uint32_t ow2, uint32_t ow3, uint32_t ow4,
                                           uint32_t ow5, uint32_t ow6, uint32_t ow7) {
  __shared__ uint32_t cvs[AOS_B3_MAX_CHUNKS][8];
  const size_t in_len = (size_t)n * 4 + (reasoning ? 32 : 0);
  auto in_word = [&](size_t j) -> uint32_t {
    if (j < (size_t)n) {
      const float v = (scope && !scope[j]) ? -1.0e9f : priors[j];
      return __builtin_bit_cast(uint32_t, v);
    }
    return extra[j - (size_t)n];
  };
  const int C = aos_b3_nchunks(in_len);
  uint32_t h_in[8];
  if (C > 1) {
    if (lane < C) {
      uint32_t cv[8];
      aos_b3_chunk(in_word, in_len, (uint64_t)lane, false, cv);
#pragma unroll
      for (int i = 0; i < 8; ++i) cvs[lane][i] = cv[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  }
  if (lane != 0) return;
  if (C > 1) aos_b3_merge(cvs, C, h_in);
  else aos_b3_chunk(in_word, in_len, 0, true, h_in);

  /* output: the packed words of the kk indices and kk gates, then the reasoning hash */
  const uint32_t ow[8] = {ow0, ow1, ow2, ow3, ow4, ow5, ow6, ow7};
  const size_t out_len = (size_t)kk * 4 + (reasoning ? 32 : 0);
  auto out_word = [&](size_t j) -> uint32_t {
    uint32_t v = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w)
      if ((size_t)w == j) v = ow[w];
    return j < (size_t)kk ? v : extra[j - (size_t)kk];
  };
  uint32_t h_out[8];
  aos_b3_chunk(out_word, out_len, 0, true, h_out);

  const size_t comb_len = 64 + (reasoning ? 32 : 0) + (backend ? 32 : 0);
  auto comb_word = [&](size_t j) -> uint32_t {
    uint32_t v = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      if ((size_t)w == j) v = h_in[w];
      if ((size_t)w + 8 == j) v = h_out[w];
    }
    if (j >= 16) {
      const size_t e = j - 16;
      v = (reasoning && e < 8) ? extra[e] : extra[8 + (reasoning ? e - 8 : e)];
    }
    return v;
  };
  uint32_t h_comb[8];
  aos_b3_chunk(comb_word, comb_len, 0, true, h_comb);
  uint32_t *dst = (uint32_t *)(hashes + (size_t)96 * t);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    dst[i] = h_in[i];
    dst[8 + i] = h_out[i];
    dst[16 + i] = h_comb[i];
  }
}

/* renormalize_gates_q15 (policy_mask.rs:164-213) with gate s in lane s < n: one gate -> 32767;
 * otherwise g = q / 32767 in float64 summed with Kahan in slot order, q' = quantize(float(g / sum)),
 * or the float32 uniform 1/n quantised when the sum is 0. Returns this lane's new gate. */
__device__ __forceinline__ int renormalize_q15_lane(int my_q, int n, int lane) {
  if (n == 1) return lane == 0 ? 32767 : 0;
  double sum = 0.0, c = 0.0;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const double g = (double)(int)aos_shfl((uint32_t)my_q, s) / 32767.0;
    if (s < n) {
      const double y = g - c;
      const double tt = sum + y;
      c = (tt - sum) - y;
      sum = tt;
    }
  }
  if (lane >= n) return 0;
  const double mine = (double)my_q / 32767.0;
  return sum > 0.0 ? quantize_q15((float)(mine / sum)) : quantize_q15(1.0f / (float)n);
}

/* Strength scaling (router_bridge.rs:168-186): round_half_away(q * clamp(strength, 0, 1)) as i16,
 * clamped to +-32767; a NaN strength gives 0 (NaN survives the clamp and casts to 0). */
__device__ __forceinline__ int scale_gate(int q, float strength) {
  if (strength != strength) return 0;
  const float st = strength < 0.0f ? 0.0f : (strength > 1.0f ? 1.0f : strength);
  const float v = (float)q * st;
  float r = truncf(v);
  if (fabsf(v - r) >= 0.5f) r += copysignf(1.0f, v);
  if (r > 32767.0f) r = 32767.0f;
  if (r < -32767.0f) r = -32767.0f;
  return (int)r;
}

/* Per-adapter inputs of the selection besides the prior: the allowed mask, the scope hint and
 * the tie-break key (stable_id, or the adaptive mode's rank). */
struct RouteMeta {
  int allowed, in_scope;
  uint64_t sid;
};

template <bool X>
__device__ __forceinline__ RouteMeta route_meta(const aos_route_params &p, int i) {
  RouteMeta m = {1, 1, 0ull};
  if (i >= p.n) return m;
  if (p.allowed) m.allowed = p.allowed[i];
  if (X && p.scope) m.in_scope = p.scope[i];
  m.sid = (X && p.tie_key) ? p.tie_key[i] : (p.stable_id ? p.stable_id[i] : 0ull);
  return m;
}

/* An empty Decision record (entropy 0, no candidates) for token t. */
__device__ __forceinline__ void decision_empty(aoship_decision_t *decisions, int t, int lane) {
  if (!decisions) return;
  aoship_decision_t *d = decisions + t;
  if (lane < 8) {
    d->adapter_idx[lane] = 0;
    d->gate_q15[lane] = 0;
    d->raw_score[lane] = 0.0f;
  }
  if (lane == 0) {
    d->entropy = 0.0f;
    d->n_candidates = 0u;
  }
}

/* X: the extras (scope, adaptive keys, decision policy, ring mapping, decision hashes) are
 * compiled in; the X = false instance is the plain router, launched when none is set. first: the
 * lane's RouteMeta for adapter `lane`, loaded ahead (NULL: loaded here). */
template <bool LDS, bool X>
__device__ __forceinline__ void route_one(const aos_route_params &p, const float *priors, int t, int lane,
                                          const RouteMeta *first = nullptr) {
  const int n = p.n;
  const uint8_t *scope = X ? p.scope : nullptr;
  const uint64_t *tie_key = X ? p.tie_key : nullptr;
  const uint8_t *post_allowed = X ? p.post_allowed : nullptr;
  const uint16_t *active_ids = X ? p.active_ids : nullptr;
  const float *strengths = X ? p.strengths : nullptr;
  uint8_t *hashes = X ? p.hashes : nullptr;
  aoship_decision_t *decisions = X ? p.decisions : nullptr;
  /* every prior is checked for finiteness, allowed or not (validate_router_inputs); the chunked
   * passes below visit each index exactly once */
  bool bad = false;
  uint64_t ka = ~0ull, kb = ~0ull;
  int m_allowed = 0;
  auto load_key = [&](int i, uint64_t &a, uint64_t &b, const RouteMeta &m) -> bool {
    a = ~0ull;
    b = ~0ull;
    if (i >= n) return false;
    const float raw = priors[i];
    if (!__builtin_isfinite(raw)) bad = true;
    if (!m.allowed) return false;
    /* scope hint (router.rs:1587-1602): adapters outside the scope score from -1e9 */
    const float prior = (scope && !m.in_scope) ? -1.0e9f : raw;
    float sim = (prior + 0.0f) - 0.0f;
    float score = sim * p.bias;
    score = score * 1.0f;
    if (!__builtin_isfinite(score)) bad = true;
    /* adaptive mode (sort_scores_adaptive, router.rs:265-306): the rank of (breaker, stable_id,
     * index) stands in for stable_id, which orders equal scores exactly as those three keys do */
    const uint64_t sid = m.sid;
    a = ((uint64_t)score_key_desc(score) << 32) | (sid >> 32);
    b = ((sid & 0xffffffffull) << 32) | (uint64_t)(uint32_t)i;
    return true;
  };
  {
    bool v = load_key(lane, ka, kb, first ? *first : route_meta<X>(p, lane));
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
      v = load_key(base + lane - 8, a, b, route_meta<X>(p, base + lane - 8));
      ka = a;
      kb = b;
    }
    m_allowed += __popcll(__ballot(v));
    bitonic64(ka, kb, lane);
  }

  aoship_ring_t *ring = p.rings + t;
  const bool any_bad = __ballot(bad) != 0ull;
  const bool policy = post_allowed != nullptr;
  int kk = p.k < m_allowed ? p.k : m_allowed;
  if (any_bad || kk <= 0) {
    /* an empty decision under a decision policy is a PolicyViolation (policy_mask.rs:330-337) */
    ring_empty(ring, p.status, t, lane, any_bad ? -1 : (policy ? -2 : 0));
    hash_empty(hashes, t, lane);
    decision_empty(decisions, t, lane);
    return;
  }

  /* Lane l works on top-K entry e = l % 8 (lanes 8 and up repeat lanes 0..7); what every lane
   * needs of the other entries comes through shuffles. Each entry's arithmetic is the serial
   * loop's, and the sums run over the entries in top-K order, so the results are the serial
   * code's. */
  const int e = lane & 7;
  const uint64_t ea = aos_shfl64(ka, e), eb = aos_shfl64(kb, e);
  const uint32_t e_key = (uint32_t)(ea >> 32), e_idx = (uint32_t)eb;
  const float e_sc = score_from_key(e_key);
  uint64_t e_sid = ((ea & 0xffffffffull) << 32) | (eb >> 32);
  /* the canonical re-sort keeps stable_id in adaptive mode (router.rs:1305-1325) */
  if (tie_key) e_sid = (e < kk && p.stable_id) ? p.stable_id[e_idx] : 0ull;

  /* deterministic_softmax (router.rs:1340-1411); tau > 0 after sanitising. */
  double mx = -__builtin_inf();
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const float v = aos_shfl_f(e_sc, s);
    if (s < kk) mx = rust_f64_max(mx, (double)v);
  }
  const double e_exp = aos_exp_cr(((double)e_sc - mx) / (double)p.tau);
  double sum = 0.0, comp = 0.0;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const double ex = __builtin_bit_cast(double, aos_shfl64(__builtin_bit_cast(uint64_t, e_exp), s));
    if (s < kk) {
      double y = ex - comp;
      double tt = sum + y;
      comp = (tt - sum) - y;
      sum = tt;
    }
  }
  float g = (sum == 0.0) ? 1.0f / (float)kk : (float)(e_exp / sum);
  g = rust_f32_max(g, p.eps / (float)kk);
  float S = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const float gs = aos_shfl_f(g, s);
    if (s < kk) S += gs;
  }
  if (!(S > 0.0f)) {
    ring_empty(ring, p.status, t, lane, policy ? -2 : 0);
    hash_empty(hashes, t, lane);
    decision_empty(decisions, t, lane);
    return;
  }
  const int e_q = e < kk ? quantize_q15(g / S) : 0;
  /* compute_entropy (router.rs:1287-1293) of the renormalised gates g / S: -g log2(g) for g > 0,
   * summed in float32 in top-K order; log2 in double precision, rounded to float */
  float entropy = 0.0f;
  if (decisions) {
    const float gn = g / S;
    const float term = gn > 0.0f ? -gn * (float)log2((double)gn) : 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float ts = aos_shfl_f(term, s), gs = aos_shfl_f(gn, s);
      if (s < kk && gs > 0.0f) entropy += ts;
    }
  }

  /* Canonical order (router.rs:1310-1325): entry e's rank among the kk entries. */
  int rank = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int qj = (int)aos_shfl((uint32_t)e_q, j);
    const uint32_t kj = aos_shfl(e_key, j), ij = aos_shfl(e_idx, j);
    const uint64_t sj = aos_shfl64(e_sid, j);
    const bool before =
        qj > e_q ||
        (qj == e_q && (kj < e_key || (kj == e_key && (sj < e_sid || (sj == e_sid && ij < e_idx)))));
    rank += (j != e && j < kk && before) ? 1 : 0;
  }
  /* lane s < kk holds decision entry s (canonical order) */
  uint32_t my_i = 0;
  int my_q = 0;
  float my_raw = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ri = (int)aos_shfl((uint32_t)rank, i);
    const int qi = (int)aos_shfl((uint32_t)e_q, i);
    const uint32_t ii = aos_shfl(e_idx, i);
    const float ri_sc = aos_shfl_f(e_sc, i);
    if (i < kk && ri == lane) {
      my_i = ii;
      my_q = qi;
      my_raw = ri_sc;
    }
  }
  if (X && hashes) {
    /* the decision hash belongs to the router's decision, before any policy filter: kk indices
     * (u16 LE) then kk gates (i16 LE), packed two halves to a word */
    uint32_t hw[16];
#pragma unroll
    for (int pos = 0; pos < 16; ++pos) hw[pos] = 0;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint32_t is = aos_shfl(my_i, s) & 0xFFFFu;
      const uint32_t qs = (uint32_t)(uint16_t)(int16_t)(int)aos_shfl((uint32_t)my_q, s);
#pragma unroll
      for (int pos = 0; pos < 16; ++pos) {
        if (s < kk && pos == s) hw[pos] = is;
        if (s < kk && pos == kk + s) hw[pos] = qs;
      }
    }
    decision_hash(hashes, priors, scope, p.n, p.hash_extra, p.hash_reasoning, p.hash_backend, t, lane, kk,
                  hw[0] | hw[1] << 16, hw[2] | hw[3] << 16, hw[4] | hw[5] << 16, hw[6] | hw[7] << 16,
                  hw[8] | hw[9] << 16, hw[10] | hw[11] << 16, hw[12] | hw[13] << 16, hw[14] | hw[15] << 16);
  }
  int m = kk;
  int cand_q = my_q; /* a candidate keeps its gate from before a policy's renormalisation */
  if (X && policy) {
    /* filter_decision_by_policy (policy_mask.rs:221-355): passing entries keep decision order,
     * capped at max_adapters_per_token; anything removed renormalises the gates */
    const bool keep = lane < kk && post_allowed[my_i] != 0;
    const uint32_t km = (uint32_t)__ballot(keep) & 0xFFu;
    int kept = __popc(km);
    if (p.post_max >= 0 && kept > p.post_max) kept = p.post_max;
    if (kept == 0) {
      ring_empty(ring, p.status, t, lane, -2);
      decision_empty(decisions, t, lane);
      return;
    }
    /* slot s takes the s-th passing entry */
    int src = 0;
    uint32_t rest = km;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int b = rest ? __ffs(rest) - 1 : 0;
      if (s == lane) src = b;
      rest &= rest - 1u;
    }
    my_i = aos_shfl(my_i, src);
    my_q = (int)aos_shfl((uint32_t)my_q, src);
    my_raw = aos_shfl_f(my_raw, src);
    if (lane >= kept) {
      my_i = 0;
      my_q = 0;
    }
    cand_q = my_q;
    if (kept < kk) my_q = renormalize_q15_lane(my_q, kept, lane);
    m = kept;
  }
  if (decisions) {
    /* the Decision's candidates (types.rs:669-674) in decision order, and its entropy */
    aoship_decision_t *d = decisions + t;
    if (lane < 8) {
      d->adapter_idx[lane] = (uint16_t)(lane < m ? my_i : 0u);
      d->gate_q15[lane] = (int16_t)(lane < m ? cand_q : 0);
      d->raw_score[lane] = lane < m ? my_raw : 0.0f;
    }
    if (lane == 0) {
      d->entropy = entropy;
      d->n_candidates = (uint32_t)m;
    }
  }
  /* decision_to_router_ring_with_active_ids_and_strengths (router_bridge.rs:137-186) */
  uint32_t oi = my_i;
  int oq = my_q;
  if (X && (active_ids || strengths)) {
    if (lane < m && active_ids) oi = active_ids[my_i];
    if (lane < m && strengths) oq = scale_gate(my_q, strengths[my_i]);
    /* set_with_max_adapter(.., u16::MAX): an index of 65535 zero-fills the ring (lib.rs:163-179) */
    if (__ballot(lane < m && oi >= 0xFFFFu) != 0ull) {
      ring_empty(ring, p.status, t, lane, 0);
      return;
    }
  }
  if (lane < 8) {
    ring->adapter_indices[lane] = (uint16_t)(lane < m ? oi : 0u);
    ring->gates_q15[lane] = (int16_t)(lane < m ? oq : 0);
  }
  if (lane == 0) {
    ring->top_k = (uint32_t)m;
    ring->current_pos = (uint32_t)t;
    if (p.status) p.status[t] = 0;
  }
}

/* Dot products of router features (staged in LDS) with router weight rows: lane l sums elements
 * 256k + 4l + e (k ascending, e = 0..3) with fused multiply-adds, then a xor butterfly over the
 * 64 lanes. 16 chunks of 256 weights are loaded (dot_load) before their arithmetic (dot_use). */
__device__ __forceinline__ void dot_load(const float *w, int k0, int nk, int lane, float4 (&wv)[16]) {
  const float4 *w4 = (const float4 *)w;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int k = k0 + j < nk ? k0 + j : nk - 1;
    wv[j] = w4[k * 64 + lane];
  }
}

__device__ __forceinline__ void dot_use(const float *f_lds, const float4 (&wv)[16], int k0, int nk, int lane,
                                        float &acc) {
  const float4 *f4 = (const float4 *)f_lds;
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

/* The rest of a dot product whose first 16 chunks are in wv: the remaining chunks, the tail
 * (d % 256 elements, a multiple of 4), then the butterfly. */
__device__ __forceinline__ float dot_finish(const float *f_lds, const float *w, int d, int lane, float4 (&wv)[16]) {
  const int nk = d >> 8, tail = d & 255;
  float acc = 0.0f;
  if (nk > 0) dot_use(f_lds, wv, 0, nk, lane, acc);
  for (int k0 = 16; k0 < nk; k0 += 16) {
    dot_load(w, k0, nk, lane, wv);
    dot_use(f_lds, wv, k0, nk, lane, acc);
  }
  if (4 * lane < tail) {
    const float4 fv = ((const float4 *)f_lds)[nk * 64 + lane], wt = ((const float4 *)w)[nk * 64 + lane];
    acc = fmaf(wt.x, fv.x, acc);
    acc = fmaf(wt.y, fv.y, acc);
    acc = fmaf(wt.z, fv.z, acc);
    acc = fmaf(wt.w, fv.w, acc);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc = acc + aos_shfl_f(acc, lane ^ o);
  return acc;
}

}  // namespace

#endif
