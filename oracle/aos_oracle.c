/*
 * aos_oracle.c — CPU restatement of adapterOS's router + int4 LoRA layer (test infrastructure).
 *
 * TEST INFRASTRUCTURE ONLY: the oracle the HIP path is tested against, never the product. See aos_oracle.h
 * for the reference file:line each function follows and for how each one is pinned.
 *
 * Built with -O2 -ffp-contract=off and without fast-math, so every float operation below is
 * the single IEEE operation written in the source (the reference forbids fast-math:
 * crates/adapteros-lora-kernel-api/src/attestation.rs:211-219).
 */
#include "aos_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_MAX_K 8                 /* crates/adapteros-core/src/defaults.rs:37 */
#define ORC_DEFAULT_EPS 0.02f       /* crates/adapteros-core/src/defaults.rs:24 */
#define ORC_Q15_DENOM 32767.0f      /* crates/adapteros-lora-router/src/quantization.rs:22 */
#define ORC_Q15_MAX 32767

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* The router's float64 exp: the C library's exp (Rust's f64::exp on the host platform), unless a
 * test installs another implementation to show the outputs do not depend on the choice. */
static double (*g_exp)(double) = exp;
void orc_set_exp(double (*f)(double)) { g_exp = f ? f : exp; }
double orc_exp(double x) { return g_exp(x); }

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ------------------------------------------------------------------------------------------ */
/* Router                                                                                     */
/* ------------------------------------------------------------------------------------------ */

/* f32::total_cmp key (core::f32::total_cmp): bits ^ (((bits as i32) >> 31) as u32 >> 1),
 * compared as i32. Returned here biased to an unsigned key that sorts DESCENDING by score when
 * compared ascending: key = 0x7fffffff - signed_key (as offset u32). */
uint64_t orc_total_cmp_key_desc(float x) {
  int32_t b = (int32_t)f32_bits(x);
  int32_t t = b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
  /* ascending-comparable unsigned form of t, then inverted for descending */
  uint32_t asc = (uint32_t)t ^ 0x80000000u;
  return (uint64_t)(0xffffffffu - asc);
}

/* quantization.rs:172-175: (gate * 32767.0).round() as i32, clamped to [0, 32767].
 * f32::round rounds half away from zero (== C roundf); `as i32` saturates, NaN -> 0. */
int16_t orc_quantize_gate(float gate) {
  float s = gate * ORC_Q15_DENOM;
  float r = roundf(s);
  int32_t v;
  if (r != r) v = 0;
  else if (r >= 2147483647.0f) v = 2147483647;
  else if (r <= -2147483648.0f) v = (int32_t)0x80000000u;
  else v = (int32_t)r;
  if (v < 0) v = 0;
  if (v > ORC_Q15_MAX) v = ORC_Q15_MAX;
  return (int16_t)v;
}

typedef struct {
  int idx;
  float score;
  uint64_t breaker; /* adaptive mode only; 0 for every candidate otherwise */
  uint64_t stable_id;
} orc_cand_t;

/* router.rs:234-264 comparator: score DESC (total_cmp), stable_id ASC; Rust's sort_by is stable,
 * so remaining ties keep index order — made explicit here as the last key. Adaptive mode
 * (sort_scores_adaptive, router.rs:265-306) puts the seeded breaker between score and stable_id. */
static int cmp_scored(const orc_cand_t *a, const orc_cand_t *b) {
  uint64_t ka = orc_total_cmp_key_desc(a->score), kb = orc_total_cmp_key_desc(b->score);
  if (ka != kb) return ka < kb ? -1 : 1;
  if (a->breaker != b->breaker) return a->breaker < b->breaker ? -1 : 1;
  if (a->stable_id != b->stable_id) return a->stable_id < b->stable_id ? -1 : 1;
  if (a->idx != b->idx) return a->idx < b->idx ? -1 : 1;
  return 0;
}

typedef struct {
  int idx;
  float raw;
  int16_t q;
  uint64_t stable_id;
} orc_final_t;

/* router.rs:1310-1325: gate_q15 DESC, raw_score DESC (total_cmp), stable_id ASC, adapter_idx ASC. */
static int cmp_final(const orc_final_t *a, const orc_final_t *b) {
  if (a->q != b->q) return a->q > b->q ? -1 : 1;
  uint64_t ka = orc_total_cmp_key_desc(a->raw), kb = orc_total_cmp_key_desc(b->raw);
  if (ka != kb) return ka < kb ? -1 : 1;
  if (a->stable_id != b->stable_id) return a->stable_id < b->stable_id ? -1 : 1;
  if (a->idx != b->idx) return a->idx < b->idx ? -1 : 1;
  return 0;
}

/* Stable insertion sort (n is small; order is total so stability is moot). */
static void sort_scored(orc_cand_t *c, int n) {
  for (int i = 1; i < n; ++i) {
    orc_cand_t v = c[i];
    int j = i - 1;
    while (j >= 0 && cmp_scored(&c[j], &v) > 0) {
      c[j + 1] = c[j];
      --j;
    }
    c[j + 1] = v;
  }
}

static void sort_final(orc_final_t *c, int n) {
  for (int i = 1; i < n; ++i) {
    orc_final_t v = c[i];
    int j = i - 1;
    while (j >= 0 && cmp_final(&c[j], &v) > 0) {
      c[j + 1] = c[j];
      --j;
    }
    c[j + 1] = v;
  }
}

/* router.rs:146-166 */
static float sanitize_eps(float eps) {
  if (!isfinite(eps)) return ORC_DEFAULT_EPS;
  if (!(eps >= 0.0f && eps <= 1.0f)) return ORC_DEFAULT_EPS;
  return eps;
}

/* router.rs:171-187 */
static float sanitize_tau(float tau) {
  if (!isfinite(tau)) return 1.0f;
  if (tau <= 0.0f) return 1.0f;
  return tau;
}

/* Rust f64::max (IEEE maxNum: a NaN operand yields the other operand). */
static double rust_f64_max(double a, double b) {
  if (a != a) return b;
  if (b != b) return a;
  return a > b ? a : (b > a ? b : a);
}

/* Rust f32::max */
static float rust_f32_max(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  return a > b ? a : (b > a ? b : a);
}

int orc_route_one(const float *priors, int n, const uint64_t *stable_id, const uint8_t *allowed,
                  int k, float tau, float eps, float routing_bias, uint16_t idx_out[8],
                  int16_t q15_out[8]) {
  return orc_route_one_ex(priors, n, stable_id, allowed, NULL, NULL, k, tau, eps, routing_bias, idx_out,
                          q15_out);
}

int orc_route_one_ex(const float *priors, int n, const uint64_t *stable_id, const uint8_t *allowed,
                     const uint8_t *scope, const uint64_t *breakers, int k, float tau, float eps,
                     float routing_bias, uint16_t idx_out[8], int16_t q15_out[8]) {
  return orc_route_one_detail(priors, n, stable_id, allowed, scope, breakers, k, tau, eps, routing_bias, idx_out,
                              q15_out, NULL, NULL);
}

/* orc_route_one_ex that also returns the decision's entropy and its candidates' raw scores (in
 * decision order; the candidates' indices and Q15 gates are idx_out / q15_out). The entropy is
 * Router::compute_entropy (router.rs:1287-1293) of the renormalised f32 gates, applied at
 * router.rs:1844: the sum over gates g > 0, in top-K (score) order, of -g * log2(g) in f32, with
 * the C library's log2f (what Rust's f32::log2 calls on this platform). An empty decision has
 * entropy 0 (router.rs:2070). entropy_out / raw_out may be NULL. */
int orc_route_one_detail(const float *priors, int n, const uint64_t *stable_id, const uint8_t *allowed,
                         const uint8_t *scope, const uint64_t *breakers, int k, float tau, float eps,
                         float routing_bias, uint16_t idx_out[8], int16_t q15_out[8], float *entropy_out,
                         float raw_out[8]) {
  for (int i = 0; i < 8; ++i) {
    idx_out[i] = 0;
    q15_out[i] = 0;
    if (raw_out) raw_out[i] = 0.0f;
  }
  if (entropy_out) *entropy_out = 0.0f;
  /* Router::new rejects k > MAX_K (router.rs:769-777); sanitize_k lifts 0 to 1 (:127-142). */
  if (k > ORC_MAX_K || n < 0) return -1;
  if (k < 1) k = 1;
  tau = sanitize_tau(tau);
  eps = sanitize_eps(eps);
  /* set_routing_bias keeps the default 1.0 for a non-finite or non-positive bias (:556-562). */
  if (!(isfinite(routing_bias) && routing_bias > 0.0f)) routing_bias = 1.0f;

  /* validate_router_inputs (router.rs:611-625): every prior finite, masked or not. */
  for (int i = 0; i < n; ++i)
    if (!isfinite(priors[i])) return -1;

  orc_cand_t *c = (orc_cand_t *)malloc(sizeof(orc_cand_t) * (size_t)(n > 0 ? n : 1));
  int m = 0;
  for (int i = 0; i < n; ++i) {
    if (allowed && !allowed[i]) continue;
    /* router.rs:1664-1676 with empty features (feature score 0.0, :985-988), no orthogonal
     * penalty (0.0, :1490-1501), not MoE, version_weight 1.0 (types.rs:656). A scope hint
     * (router.rs:1587-1602) replaces the priors outside the scope with -1e9 first. */
    const float prior = (scope && !scope[i]) ? -1.0e9f : priors[i];
    float sim = (prior + 0.0f) - 0.0f;
    float score = sim * routing_bias; /* scoring.rs:35-37 */
    score *= 1.0f;                    /* clamp(version_weight, 0, 2) with the default 1.0 */
    if (!isfinite(score)) {
      free(c);
      return -1;
    }
    c[m].idx = i;
    c[m].score = score;
    c[m].breaker = breakers ? breakers[i] : 0;
    c[m].stable_id = stable_id ? stable_id[i] : 0;
    ++m;
  }
  if (m == 0) {
    free(c);
    return 0;
  }
  sort_scored(c, m);
  int kk = k < m ? k : m;

  /* deterministic_softmax (router.rs:1340-1411). tau was sanitized to > 0 at construction, so
   * the tau == 0 one-hot branch is unreachable through the router. */
  double mx = -INFINITY;
  for (int i = 0; i < kk; ++i) mx = rust_f64_max(mx, (double)c[i].score);
  double e[ORC_MAX_K];
  double sum = 0.0, comp = 0.0;
  for (int i = 0; i < kk; ++i) {
    double ex = orc_exp(((double)c[i].score - mx) / (double)tau);
    double y = ex - comp;
    double t = sum + y;
    comp = (t - sum) - y;
    sum = t;
    e[i] = ex;
  }
  float g[ORC_MAX_K];
  if (sum == 0.0) {
    float u = 1.0f / (float)kk;
    for (int i = 0; i < kk; ++i) g[i] = u;
  } else {
    for (int i = 0; i < kk; ++i) g[i] = (float)(e[i] / sum);
  }
  /* entropy floor (router.rs:1820-1827) */
  float min_gate = eps / (float)kk;
  for (int i = 0; i < kk; ++i) g[i] = rust_f32_max(g[i], min_gate);
  /* renormalize (router.rs:1830-1842): f32 sum in order */
  float s = 0.0f;
  for (int i = 0; i < kk; ++i) s += g[i];
  if (s <= 0.0f) {
    free(c);
    return 0;
  }
  for (int i = 0; i < kk; ++i) g[i] /= s;
  if (entropy_out) {
    float h = 0.0f;
    for (int i = 0; i < kk; ++i)
      if (g[i] > 0.0f) h += -g[i] * log2f(g[i]);
    *entropy_out = h;
  }

  orc_final_t f[ORC_MAX_K];
  for (int i = 0; i < kk; ++i) {
    f[i].idx = c[i].idx;
    f[i].raw = c[i].score;
    f[i].q = orc_quantize_gate(g[i]);
    f[i].stable_id = c[i].stable_id;
  }
  free(c);
  sort_final(f, kk);
  for (int i = 0; i < kk; ++i) {
    idx_out[i] = (uint16_t)f[i].idx;
    q15_out[i] = f[i].q;
    if (raw_out) raw_out[i] = f[i].raw;
  }
  return kk;
}

int orc_route_batch(const float *priors, int T, int n, const uint64_t *stable_id,
                    const uint8_t *allowed, int k, float tau, float eps, float routing_bias,
                    orc_ring_t *rings, int *bad_token) {
  int bad = -1;
  for (int t = 0; t < T; ++t) {
    orc_ring_t *r = &rings[t];
    memset(r, 0, sizeof(*r));
    int kk = orc_route_one(priors + (size_t)t * n, n, stable_id, allowed, k, tau, eps,
                           routing_bias, r->adapter_indices, r->gates_q15);
    if (kk < 0) {
      if (bad < 0) bad = t;
      continue;
    }
    r->top_k = (uint32_t)kk;
    r->current_pos = (uint32_t)t;
  }
  if (bad_token) *bad_token = bad;
  return bad < 0 ? 0 : -1;
}

/* renormalize_gates_q15 (crates/adapteros-lora-router/src/policy_mask.rs:164-213). */
void orc_renormalize_q15(const int16_t *q, int n, int16_t *out) {
  if (n <= 0) return;
  if (n == 1) {
    out[0] = orc_quantize_gate(1.0f);
    return;
  }
  const double denom = (double)ORC_Q15_DENOM;
  double sum = 0.0, c = 0.0, g[ORC_MAX_K];
  for (int i = 0; i < n; ++i) {
    g[i] = (double)q[i] / denom;
    double y = g[i] - c;
    double t = sum + y;
    c = (t - sum) - y;
    sum = t;
  }
  if (sum > 0.0) {
    for (int i = 0; i < n; ++i) out[i] = orc_quantize_gate((float)(g[i] / sum));
  } else {
    float u = 1.0f / (float)n;
    for (int i = 0; i < n; ++i) out[i] = orc_quantize_gate(u);
  }
}

/* filter_decision_by_policy (policy_mask.rs:221-355), the id and cluster sets reduced to
 * allowed[n] (nonzero = passes). Returns the new length or -2 (AosError::PolicyViolation). */
int orc_filter_decision(const uint16_t *idx, const int16_t *q, int kk, const uint8_t *allowed,
                        int max_per_token, uint16_t *idx_out, int16_t *q_out) {
  uint16_t fi[ORC_MAX_K];
  int16_t fq[ORC_MAX_K];
  int m = 0;
  for (int i = 0; i < kk; ++i) {
    if (!allowed[idx[i]]) continue;
    fi[m] = idx[i];
    fq[m] = q[i];
    ++m;
  }
  if (max_per_token >= 0) {
    if (max_per_token == 0) return -2; /* :318-322 */
    if (m > max_per_token) m = max_per_token;
  }
  if (m == 0) return -2; /* :330-337 */
  if (m < kk) {
    orc_renormalize_q15(fq, m, q_out); /* :339-345, only when something was removed */
  } else {
    for (int i = 0; i < m; ++i) q_out[i] = fq[i];
  }
  for (int i = 0; i < m; ++i) idx_out[i] = fi[i];
  return m;
}

/* decision_to_router_ring_with_active_ids_and_strengths
 * (crates/adapteros-lora-worker/src/router_bridge.rs:137-186). active_ids (NULL = identity) and
 * strengths (NULL = none) have n_active entries. Returns 0, or -1 for a decision index outside
 * the active set (AosError::Routing). */
int orc_decision_to_ring(const uint16_t *idx, const int16_t *q, int kk, const uint16_t *active_ids,
                         const float *strengths, int n_active, int position, orc_ring_t *ring) {
  uint16_t mapped[ORC_MAX_K];
  for (int i = 0; i < kk; ++i) {
    if (active_ids && idx[i] >= n_active) return -1;
    mapped[i] = active_ids ? active_ids[idx[i]] : idx[i];
  }
  memset(ring, 0, sizeof(*ring));
  ring->current_pos = (uint32_t)position;
  /* RouterRing::set_with_max_adapter(mapped, gates, u16::MAX), release build (lib.rs:122-193) */
  int zero = 0;
  for (int i = 0; i < kk; ++i) zero |= mapped[i] >= 0xFFFFu;
  if (!zero) {
    for (int i = 0; i < kk; ++i) {
      ring->adapter_indices[i] = mapped[i];
      ring->gates_q15[i] = q[i];
    }
    ring->top_k = (uint32_t)kk;
  }
  if (strengths) {
    for (int slot = 0; slot < kk; ++slot) {
      float s = idx[slot] < n_active ? strengths[idx[slot]] : 1.0f; /* unwrap_or(1.0) */
      /* f32::clamp keeps NaN; NaN * q rounds to NaN, and `as i16` maps NaN to 0 */
      if (s == s) s = s < 0.0f ? 0.0f : (s > 1.0f ? 1.0f : s);
      float v = roundf((float)ring->gates_q15[slot] * s);
      int32_t iv;
      if (v != v) iv = 0;
      else if (v >= 32767.0f) iv = 32767;
      else if (v <= -32768.0f) iv = -32768;
      else iv = (int32_t)v;
      if (iv > ORC_Q15_MAX) iv = ORC_Q15_MAX;
      if (iv < -ORC_Q15_MAX) iv = -ORC_Q15_MAX;
      ring->gates_q15[slot] = (int16_t)iv;
    }
  }
  return 0;
}

/* What one device routing call produces per token: route, then (policy) filter, then the ring.
 * status[t]: 0, -1 (DeterminismViolation: ring zero) or -2 (PolicyViolation: ring zero). */
void orc_route_batch_ex(const float *priors, int T, int n, const uint64_t *stable_id,
                        const uint8_t *allowed, const uint8_t *scope, const uint64_t *breakers, int k,
                        float tau, float eps, float routing_bias, const uint8_t *post_allowed,
                        int post_max, const uint16_t *active_ids, const float *strengths,
                        orc_ring_t *rings, int32_t *status) {
  for (int t = 0; t < T; ++t) {
    uint16_t idx[ORC_MAX_K], fi[ORC_MAX_K];
    int16_t q[ORC_MAX_K], fq[ORC_MAX_K];
    orc_ring_t *r = &rings[t];
    memset(r, 0, sizeof(*r));
    int kk = orc_route_one_ex(priors + (size_t)t * n, n, stable_id, allowed, scope, breakers, k, tau,
                              eps, routing_bias, idx, q);
    if (kk < 0) {
      status[t] = -1;
      continue;
    }
    if (post_allowed) {
      kk = orc_filter_decision(idx, q, kk, post_allowed, post_max, fi, fq);
      if (kk < 0) {
        status[t] = -2;
        continue;
      }
      memcpy(idx, fi, sizeof(idx));
      memcpy(q, fq, sizeof(q));
    }
    orc_decision_to_ring(idx, q, kk, active_ids, strengths, n, t, r);
    status[t] = 0;
  }
}

/* ChaCha20 block function, RFC 8439 section 2.3: twenty rounds of quarter rounds over the 16
 * input words (columns then diagonals), the input added to the result. */
void orc_chacha20_block(const uint32_t in[16], uint32_t out[16]) {
#define ORC_ROTL(v, c) (((v) << (c)) | ((v) >> (32 - (c))))
#define ORC_QR(a, b, c, d)                                      \
  x[a] += x[b]; x[d] ^= x[a]; x[d] = ORC_ROTL(x[d], 16);        \
  x[c] += x[d]; x[b] ^= x[c]; x[b] = ORC_ROTL(x[b], 12);        \
  x[a] += x[b]; x[d] ^= x[a]; x[d] = ORC_ROTL(x[d], 8);         \
  x[c] += x[d]; x[b] ^= x[c]; x[b] = ORC_ROTL(x[b], 7);
  uint32_t x[16];
  for (int i = 0; i < 16; ++i) x[i] = in[i];
  for (int round = 0; round < 20; round += 2) {
    ORC_QR(0, 4, 8, 12) ORC_QR(1, 5, 9, 13) ORC_QR(2, 6, 10, 14) ORC_QR(3, 7, 11, 15)
    ORC_QR(0, 5, 10, 15) ORC_QR(1, 6, 11, 12) ORC_QR(2, 7, 8, 13) ORC_QR(3, 4, 9, 14)
  }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + in[i];
#undef ORC_QR
#undef ORC_ROTL
}

/* ChaCha20Rng::from_seed(seed) (rand_chacha 0.3.1) then n x gen::<u64>() (rand 0.8.5): the
 * keystream of key = seed, 64-bit block counter from 0 (words 12-13), stream 0 (words 14-15),
 * serialised little-endian; value a is bytes 8a .. 8a+7 of it, little-endian. */
void orc_tie_breakers(const uint8_t seed[32], int n, uint64_t *out) {
  uint8_t ks[64];
  long have_block = -1;
  for (int a = 0; a < n; ++a) {
    uint64_t v = 0;
    for (int byte = 7; byte >= 0; --byte) {
      long pos = 8L * a + byte;
      long blk = pos / 64;
      if (blk != have_block) {
        uint32_t st[16], o[16];
        st[0] = 0x61707865u; /* "expa" */
        st[1] = 0x3320646eu; /* "nd 3" */
        st[2] = 0x79622d32u; /* "2-by" */
        st[3] = 0x6b206574u; /* "te k" */
        for (int w = 0; w < 8; ++w)
          st[4 + w] = (uint32_t)seed[4 * w] | ((uint32_t)seed[4 * w + 1] << 8) |
                      ((uint32_t)seed[4 * w + 2] << 16) | ((uint32_t)seed[4 * w + 3] << 24);
        st[12] = (uint32_t)blk;
        st[13] = (uint32_t)((uint64_t)blk >> 32);
        st[14] = 0;
        st[15] = 0;
        orc_chacha20_block(st, o);
        for (int w = 0; w < 16; ++w)
          for (int b = 0; b < 4; ++b) ks[4 * w + b] = (uint8_t)(o[w] >> (8 * b));
        have_block = blk;
      }
      v = (v << 8) | ks[pos % 64];
    }
    out[a] = v;
  }
}

/* ---- BLAKE3 (the specification's incremental hasher, byte oriented) ---------------------------- */

static const uint32_t B3_IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                                  0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
static const int B3_PERM[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};

static uint32_t b3_rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

/* compression: 7 rounds; round r reads message word sched[r][i], sched[0] = identity and
 * sched[r+1][i] = sched[r][PERM[i]] */
static void b3_compress(const uint32_t cv[8], const uint8_t block[64], uint32_t block_len, uint64_t counter,
                        uint32_t flags, uint32_t out[16]) {
  uint32_t m[16], v[16];
  int sched[16], next[16];
  for (int i = 0; i < 16; ++i) {
    m[i] = (uint32_t)block[4 * i] | ((uint32_t)block[4 * i + 1] << 8) | ((uint32_t)block[4 * i + 2] << 16) |
           ((uint32_t)block[4 * i + 3] << 24);
    sched[i] = i;
  }
  for (int i = 0; i < 8; ++i) v[i] = cv[i];
  for (int i = 0; i < 4; ++i) v[8 + i] = B3_IV[i];
  v[12] = (uint32_t)(counter & 0xffffffffu);
  v[13] = (uint32_t)(counter >> 32);
  v[14] = block_len;
  v[15] = flags;
  static const int cols[8][4] = {{0, 4, 8, 12}, {1, 5, 9, 13}, {2, 6, 10, 14}, {3, 7, 11, 15},
                                 {0, 5, 10, 15}, {1, 6, 11, 12}, {2, 7, 8, 13}, {3, 4, 9, 14}};
  for (int r = 0; r < 7; ++r) {
    for (int g = 0; g < 8; ++g) {
      int a = cols[g][0], b = cols[g][1], c = cols[g][2], d = cols[g][3];
      uint32_t x = m[sched[2 * g]], y = m[sched[2 * g + 1]];
      v[a] = v[a] + v[b] + x;
      v[d] = b3_rotr(v[d] ^ v[a], 16);
      v[c] = v[c] + v[d];
      v[b] = b3_rotr(v[b] ^ v[c], 12);
      v[a] = v[a] + v[b] + y;
      v[d] = b3_rotr(v[d] ^ v[a], 8);
      v[c] = v[c] + v[d];
      v[b] = b3_rotr(v[b] ^ v[c], 7);
    }
    for (int i = 0; i < 16; ++i) next[i] = sched[B3_PERM[i]];
    for (int i = 0; i < 16; ++i) sched[i] = next[i];
  }
  for (int i = 0; i < 8; ++i) {
    out[i] = v[i] ^ v[i + 8];
    out[i + 8] = v[i + 8] ^ cv[i];
  }
}

typedef struct {
  uint32_t cv[8];
  uint64_t counter;
  uint8_t block[64];
  uint32_t block_len;
  uint32_t blocks_done;
} b3_chunk_t;

static void b3_chunk_init(b3_chunk_t *c, uint64_t counter) {
  memcpy(c->cv, B3_IV, sizeof(B3_IV));
  c->counter = counter;
  memset(c->block, 0, 64);
  c->block_len = 0;
  c->blocks_done = 0;
}

static uint32_t b3_chunk_flags(const b3_chunk_t *c) { return c->blocks_done == 0 ? 1u : 0u; /* CHUNK_START */ }

/* the chunk's final block compressed with CHUNK_END (and extra flags) */
static void b3_chunk_output(const b3_chunk_t *c, uint32_t extra, uint32_t out[16]) {
  b3_compress(c->cv, c->block, c->block_len, c->counter, b3_chunk_flags(c) | 2u | extra, out);
}

static void b3_parent_output(const uint32_t l[8], const uint32_t r[8], uint32_t extra, uint32_t out[16]) {
  uint8_t blk[64];
  for (int i = 0; i < 8; ++i)
    for (int b = 0; b < 4; ++b) {
      blk[4 * i + b] = (uint8_t)(l[i] >> (8 * b));
      blk[32 + 4 * i + b] = (uint8_t)(r[i] >> (8 * b));
    }
  b3_compress(B3_IV, blk, 64, 0, 4u | extra, out);
}

void orc_blake3(const uint8_t *in, size_t len, uint8_t out[32]) {
  uint32_t stack[64][8];
  int depth = 0;
  b3_chunk_t ch;
  b3_chunk_init(&ch, 0);
  size_t pos = 0;
  while (pos < len) {
    /* a full chunk followed by more input: push its chaining value, merging finished subtrees */
    if (ch.blocks_done * 64 + ch.block_len == 1024) {
      uint32_t o[16], cv[8];
      b3_chunk_output(&ch, 0, o);
      memcpy(cv, o, sizeof(cv));
      const uint64_t next_counter = ch.counter + 1;
      uint64_t total = next_counter; /* chunks completed so far */
      while ((total & 1) == 0) {
        b3_parent_output(stack[--depth], cv, 0, o);
        memcpy(cv, o, sizeof(cv));
        total >>= 1;
      }
      memcpy(stack[depth++], cv, sizeof(cv));
      b3_chunk_init(&ch, next_counter);
    }
    /* a full block followed by more input: compress it */
    if (ch.block_len == 64) {
      uint32_t o[16];
      b3_compress(ch.cv, ch.block, 64, ch.counter, b3_chunk_flags(&ch), o);
      memcpy(ch.cv, o, 32);
      ch.blocks_done++;
      memset(ch.block, 0, 64);
      ch.block_len = 0;
    }
    ch.block[ch.block_len++] = in[pos++];
  }
  uint32_t o[16];
  if (depth == 0) {
    b3_chunk_output(&ch, 8u /* ROOT */, o);
  } else {
    uint32_t cv[8];
    b3_chunk_output(&ch, 0, o);
    memcpy(cv, o, sizeof(cv));
    while (depth > 0) {
      --depth;
      b3_parent_output(stack[depth], cv, depth == 0 ? 8u : 0u, o);
      memcpy(cv, o, sizeof(cv));
    }
  }
  for (int i = 0; i < 32; ++i) out[i] = (uint8_t)(o[i / 4] >> (8 * (i % 4)));
}

/* Router::compute_decision_hash (router.rs:1427-1484) with an empty feature vector: out[0..32) =
 * BLAKE3(priors LE [|| reasoning]), out[32..64) = BLAKE3(indices u16 LE || gates i16 LE
 * [|| reasoning]), out[64..96) = BLAKE3(input || output [|| reasoning] [|| backend]). */
void orc_decision_hash(const float *priors, int n, const uint16_t *idx, const int16_t *q, int kk,
                       const uint8_t *reasoning, const uint8_t *backend, uint8_t out[96]) {
  size_t inl = (size_t)n * 4 + (reasoning ? 32 : 0);
  uint8_t *buf = (uint8_t *)malloc(inl > 160 ? inl : 160);
  for (int i = 0; i < n; ++i) {
    uint32_t b = f32_bits(priors[i]);
    for (int j = 0; j < 4; ++j) buf[4 * i + j] = (uint8_t)(b >> (8 * j));
  }
  if (reasoning) memcpy(buf + (size_t)n * 4, reasoning, 32);
  orc_blake3(buf, inl, out);
  size_t ol = 0;
  for (int i = 0; i < kk; ++i) {
    buf[ol++] = (uint8_t)(idx[i] & 0xff);
    buf[ol++] = (uint8_t)(idx[i] >> 8);
  }
  for (int i = 0; i < kk; ++i) {
    uint16_t g = (uint16_t)q[i];
    buf[ol++] = (uint8_t)(g & 0xff);
    buf[ol++] = (uint8_t)(g >> 8);
  }
  if (reasoning) {
    memcpy(buf + ol, reasoning, 32);
    ol += 32;
  }
  orc_blake3(buf, ol, out + 32);
  size_t cl = 0;
  memcpy(buf + cl, out, 32);
  cl += 32;
  memcpy(buf + cl, out + 32, 32);
  cl += 32;
  if (reasoning) {
    memcpy(buf + cl, reasoning, 32);
    cl += 32;
  }
  if (backend) {
    memcpy(buf + cl, backend, 32);
    cl += 32;
  }
  orc_blake3(buf, cl, out + 64);
  free(buf);
}

/* ---- decoder step pieces (mlx_cpp_wrapper_real.cpp, fused forward) ----------------------------- */

/* rms_norm (…real.cpp:3384-3390): y = x * (w / sqrt(mean(x^2) + eps)). mode 0: float32 with the
 * sum of squares in order; mode 1: float64. */
void orc_rmsnorm(const float *x, int T, int H, const float *w, float eps, float *y, int mode) {
  for (int t = 0; t < T; ++t) {
    const float *r = x + (size_t)t * H;
    float *o = y + (size_t)t * H;
    if (mode == 0) {
      float ss = 0.0f;
      for (int e = 0; e < H; ++e) ss += r[e] * r[e];
      float d = sqrtf(ss / (float)H + eps);
      for (int e = 0; e < H; ++e) o[e] = r[e] * (w[e] / d);
    } else {
      double ss = 0.0;
      for (int e = 0; e < H; ++e) ss += (double)r[e] * (double)r[e];
      double d = sqrt(ss / (double)H + (double)eps);
      for (int e = 0; e < H; ++e) o[e] = (float)((double)r[e] * ((double)w[e] / d));
    }
  }
}

/* RoPE of the fused forward (…real.cpp:3249-3279), in place on x[T][heads][hd]: inv_freq_i =
 * 1 / theta^(-2i/hd) (float32 powf), angle = (offset + t) * inv_freq_i, halves x1 = x[:hd/2],
 * x2 = x[hd/2:] -> [x1 cos - x2 sin, x1 sin + x2 cos]. */
void orc_rope(float *x, int T, int heads, int hd, int offset, float theta) {
  int half = hd / 2;
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < heads; ++h) {
      float *r = x + ((size_t)t * heads + h) * hd;
      for (int i = 0; i < half; ++i) {
        float inv = 1.0f / powf(theta, -2.0f * (float)i / (float)hd);
        float ang = (float)(offset + t) * inv;
        float c = cosf(ang), s = sinf(ang);
        float x1 = r[i], x2 = r[i + half];
        r[i] = x1 * c - x2 * s;
        r[i + half] = x1 * s + x2 * c;
      }
    }
}

/* Causal scaled dot-product attention of the fused forward (…real.cpp:3282-3327): q[T][nh][hd]
 * (rotated), k / v[L][nkv][hd] for positions 0 .. L-1 (the cache then the new tokens,
 * L = offset + T); token t attends to positions <= offset + t (the -1e9 mask), head h to kv head
 * h / (nh / nkv); scores (q . k) * (1 / sqrt(hd)), softmax over the row, . v -> out[T][nh][hd].
 * mode 0: float32 (max-subtracted softmax, sums in position order); mode 1: float64. */
void orc_attention(const float *q, const float *k, const float *v, int T, int offset, int nh, int nkv, int hd,
                   float *out, int mode) {
  int L = offset + T, rep = nh / nkv;
  double *sc = (double *)malloc(sizeof(double) * (size_t)(L > 0 ? L : 1));
  float scale = 1.0f / sqrtf((float)hd);
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < nh; ++h) {
      const float *qr = q + ((size_t)t * nh + h) * hd;
      int kvh = h / rep, vis = offset + t + 1;
      double mx = -INFINITY;
      for (int p = 0; p < vis; ++p) {
        const float *kr = k + ((size_t)p * nkv + kvh) * hd;
        if (mode == 0) {
          float dot = 0.0f;
          for (int d = 0; d < hd; ++d) dot += qr[d] * kr[d];
          sc[p] = (double)(dot * scale);
        } else {
          double dot = 0.0;
          for (int d = 0; d < hd; ++d) dot += (double)qr[d] * (double)kr[d];
          sc[p] = dot * (double)scale;
        }
        if (sc[p] > mx) mx = sc[p];
      }
      float *o = out + ((size_t)t * nh + h) * hd;
      if (mode == 0) {
        float sum = 0.0f;
        for (int p = 0; p < vis; ++p) {
          float e = expf((float)sc[p] - (float)mx);
          sc[p] = (double)e;
          sum += e;
        }
        for (int d = 0; d < hd; ++d) {
          float a = 0.0f;
          for (int p = 0; p < vis; ++p) a += ((float)sc[p] / sum) * v[((size_t)p * nkv + kvh) * hd + d];
          o[d] = a;
        }
      } else {
        double sum = 0.0;
        for (int p = 0; p < vis; ++p) {
          sc[p] = exp(sc[p] - mx);
          sum += sc[p];
        }
        for (int d = 0; d < hd; ++d) {
          double a = 0.0;
          for (int p = 0; p < vis; ++p) a += (sc[p] / sum) * (double)v[((size_t)p * nkv + kvh) * hd + d];
          o[d] = (float)a;
        }
      }
    }
  free(sc);
}

void orc_priors(const float *features, const float *router_w, int T, int n, int d, float *priors) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < T; ++t) {
    for (int a = 0; a < n; ++a) {
      const float *w = router_w + (size_t)a * d;
      const float *f = features + (size_t)t * d;
      float p[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int base = 0; base < d; base += 256)
          for (int e = 0; e < 4; ++e) {
            int i = base + 4 * l + e;
            if (i < d) acc = fmaf(w[i], f[i], acc);
          }
        p[l] = acc;
      }
      for (int o = 32; o >= 1; o >>= 1) {
        float q[64];
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ o];
        memcpy(p, q, sizeof(p));
      }
      priors[(size_t)t * n + a] = p[0];
    }
  }
}

/* ------------------------------------------------------------------------------------------ */
/* Number formats                                                                             */
/* ------------------------------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  if (exp == 0) {
    /* zero / subnormal: man * 2^-24 exactly */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
  return bits_f32(sign | ((exp + 112) << 23) | (man << 13));
}

float orc_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (a < 0x38800000u) {                                  /* below 2^-14: subnormal */
    float v = bits_f32(a) * 16777216.0f;                  /* exact scaling to units of 2^-24 */
    uint32_t q = (uint32_t)v;
    float rem = v - (float)q;
    if (rem > 0.5f || (rem == 0.5f && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (a >> 23) - 112;
  uint32_t m = a & 0x7fffffu;
  uint32_t hm = m >> 13;
  uint32_t rest = m & 0x1fffu;
  uint32_t h = (e << 10) | hm;
  if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) ++h;
  return (uint16_t)(sign | h);
}

/* ------------------------------------------------------------------------------------------ */
/* int4 base weights                                                                          */
/* ------------------------------------------------------------------------------------------ */

/* MLX affine dequant: w[o,i] = scale[o, i/64] * q + bias[o, i/64],
 * q = (wp[o, i/8] >> (4 * (i % 8))) & 0xF. Evaluated in float32. */
static inline float dq(const uint32_t *wrow, const uint16_t *srow, const uint16_t *brow, int i) {
  uint32_t q = (wrow[i >> 3] >> (4 * (i & 7))) & 0xFu;
  float s = orc_f16_to_f32(srow[i >> 6]);
  float b = orc_f16_to_f32(brow[i >> 6]);
  return s * (float)q + b;
}

void orc_dequant_q4(const uint32_t *wp, const uint16_t *scales, const uint16_t *biases, int out,
                    int in, float *w) {
  int gpr = in / 64;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < out; ++o) {
    const uint32_t *wr = wp + (size_t)o * (in / 8);
    const uint16_t *sr = scales + (size_t)o * gpr;
    const uint16_t *br = biases + (size_t)o * gpr;
    for (int i = 0; i < in; ++i) w[(size_t)o * in + i] = dq(wr, sr, br, i);
  }
}

static void linear_row(const float *x, const uint32_t *wr, const uint16_t *sr,
                       const uint16_t *br, int in, float *yo, int mode) {
  const int groups = in / 64;
  if (mode == 0) {
    float acc = 0.0f;
    for (int g = 0; g < groups; ++g) {
      const float s = orc_f16_to_f32(sr[g]), b = orc_f16_to_f32(br[g]);
      for (int i = g * 64; i < g * 64 + 64; ++i) {
        uint32_t q = (wr[i >> 3] >> (4 * (i & 7))) & 0xFu;
        acc += x[i] * (s * (float)q + b);
      }
    }
    *yo = acc;
  } else {
    double acc = 0.0;
    for (int g = 0; g < groups; ++g) {
      const double s = orc_f16_to_f32(sr[g]), b = orc_f16_to_f32(br[g]);
      for (int i = g * 64; i < g * 64 + 64; ++i) {
        uint32_t q = (wr[i >> 3] >> (4 * (i & 7))) & 0xFu;
        acc += (double)x[i] * (s * (double)q + b);
      }
    }
    *yo = (float)acc;
  }
}

void orc_linear_q4(const float *x, int T, const uint32_t *wp, const uint16_t *scales,
                   const uint16_t *biases, int out, int in, float *y, int mode) {
  int gpr = in / 64;
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < T; ++t)
    for (int o = 0; o < out; ++o)
      linear_row(x + (size_t)t * in, wp + (size_t)o * (in / 8), scales + (size_t)o * gpr,
                 biases + (size_t)o * gpr, in, y + (size_t)t * out + o, mode);
}

/* ------------------------------------------------------------------------------------------ */
/* LoRA                                                                                       */
/* ------------------------------------------------------------------------------------------ */

/* mlx_cpp_wrapper_real.cpp:3394-3419: lora_out = (x @ A^T) @ B^T, times (scale * blend); the
 * first active adapter initialises delta, later ones are added in ring order. */
void orc_lora_delta(const float *x, const float *A, const float *B, int r, int in, int out,
                    float coef, float *delta, int first, int mode) {
  float xa[256];
  double xad[256];
  for (int j = 0; j < r; ++j) {
    const float *a = A + (size_t)j * in;
    if (mode == 0) {
      float acc = 0.0f;
      for (int i = 0; i < in; ++i) acc += x[i] * a[i];
      xa[j] = acc;
    } else {
      double acc = 0.0;
      for (int i = 0; i < in; ++i) acc += (double)x[i] * (double)a[i];
      xad[j] = acc;
    }
  }
  for (int o = 0; o < out; ++o) {
    const float *b = B + (size_t)o * r;
    float v;
    if (mode == 0) {
      float acc = 0.0f;
      for (int j = 0; j < r; ++j) acc += xa[j] * b[j];
      v = acc * coef;
    } else {
      double acc = 0.0;
      for (int j = 0; j < r; ++j) acc += xad[j] * (double)b[j];
      v = (float)(acc * (double)coef);
    }
    delta[o] = first ? v : delta[o] + v;
  }
}

/* liquid.rs:163-257: output.fill(0); for each adapter with coeff != 0: rank_buf = A x (f32,
 * sequential), output[o] += coeff * (B[o,:] . rank_buf) * (alpha / rank). */
int orc_liquid_blend(int n, const float *const *A, const float *const *B, const int *rank,
                     const float *alpha, const float *coef, const float *x, int in, float *out,
                     int out_len) {
  if (n <= 0 || n > 3) return -1; /* LIQUID_MAX_ADAPTERS = 3 (liquid.rs:12) */
  for (int o = 0; o < out_len; ++o) out[o] = 0.0f;
  for (int a = 0; a < n; ++a) {
    if (coef[a] == 0.0f) continue;
    int r = rank[a];
    float scaling = alpha[a] / (float)r;
    float rb[256];
    for (int j = 0; j < r; ++j) {
      float acc = 0.0f;
      for (int c = 0; c < in; ++c) acc += A[a][(size_t)j * in + c] * x[c];
      rb[j] = acc;
    }
    for (int o = 0; o < out_len; ++o) {
      float acc = 0.0f;
      for (int j = 0; j < r; ++j) acc += B[a][(size_t)o * r + j] * rb[j];
      out[o] += coef[a] * acc * scaling;
    }
  }
  return 0;
}

/* Apply the ring's active adapters to base output y[out] for one token (backend.rs:398-428 then
 * apply_lora). */
static void add_lora_for_ring(const float *x, int in, int out, const orc_lora_mod_t *mods,
                              int n_modules, int m, const float *scale, int n_adapters, int rank,
                              const orc_ring_t *ring, float *y, int mode, float *scratch) {
  int have = 0;
  int kk = ring->top_k > 8 ? 8 : (int)ring->top_k;
  for (int s = 0; s < kk; ++s) {
    int16_t q = ring->gates_q15[s];
    int a = ring->adapter_indices[s];
    if (q <= 0) continue;
    if (a >= n_adapters) continue;
    const orc_lora_mod_t *md = &mods[(size_t)a * n_modules + m];
    if (!md->A || !md->B) continue;
    float blend = (float)q / ORC_Q15_DENOM;
    float coef = scale[a] * blend;
    orc_lora_delta(x, md->A, md->B, rank, in, out, coef, scratch, !have, mode);
    have = 1;
  }
  if (have)
    for (int o = 0; o < out; ++o) y[o] = y[o] + scratch[o];
}

static float silu_mul(float g, float u, int mode) {
  if (mode == 0) {
    float sg = 1.0f / (1.0f + expf(-g));
    return (g * sg) * u;
  }
  double gd = g, sg = 1.0 / (1.0 + exp(-gd));
  return (float)((gd * sg) * (double)u);
}

void orc_proj_forward(const float *x, int T, int in, int out, const orc_q4_t *w,
                      const orc_lora_mod_t *mods, int n_modules, int m, const float *scale,
                      int n_adapters, int rank, const orc_ring_t *rings, float *y, int mode) {
  orc_linear_q4(x, T, w->wp, w->scales, w->biases, out, in, y, mode);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    float *scr = (float *)malloc(sizeof(float) * (size_t)out);
    add_lora_for_ring(x + (size_t)t * in, in, out, mods, n_modules, m, scale, n_adapters, rank,
                      &rings[t], y + (size_t)t * out, mode, scr);
    free(scr);
  }
}

void orc_mlp_forward(const float *x, int T, int H, int I, const orc_q4_t *gate,
                     const orc_q4_t *up, const orc_q4_t *down, const orc_lora_mod_t *mods,
                     const float *scale, int n_adapters, int rank, const orc_ring_t *rings,
                     float *y, int mode, float *h_out) {
  float *g = (float *)malloc(sizeof(float) * (size_t)T * I);
  float *u = (float *)malloc(sizeof(float) * (size_t)T * I);
  float *h = h_out ? h_out : (float *)malloc(sizeof(float) * (size_t)T * I);
  orc_proj_forward(x, T, H, I, gate, mods, 3, 0, scale, n_adapters, rank, rings, g, mode);
  orc_proj_forward(x, T, H, I, up, mods, 3, 1, scale, n_adapters, rank, rings, u, mode);
  for (size_t i = 0; i < (size_t)T * I; ++i) h[i] = silu_mul(g[i], u[i], mode);
  orc_proj_forward(h, T, I, H, down, mods, 3, 2, scale, n_adapters, rank, rings, y, mode);
  free(g);
  free(u);
  if (!h_out) free(h);
}
