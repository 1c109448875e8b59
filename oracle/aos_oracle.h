/*
 * aos_oracle.h — CPU restatement of adapterOS's adapter-augmented inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle the HIP implementation in
 * adapter-os_amd/ is tested against. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only to check or to time the CPU baseline. The product path never calls it.
 *
 * What it restates (reference paths are relative to the adapter-os tree):
 *   - K-sparse router, deterministic mode:
 *       crates/adapteros-lora-router/src/router.rs:127-187   (sanitize_k / eps / tau)
 *       crates/adapteros-lora-router/src/router.rs:234-264   (sort_scores_deterministic)
 *       crates/adapteros-lora-router/src/router.rs:1340-1411 (deterministic_softmax, f64 + Kahan)
 *       crates/adapteros-lora-router/src/router.rs:1567-1952 (route_with_adapter_info_and_scope_with_ctx)
 *       crates/adapteros-lora-router/src/router.rs:1310-1325 (canonical re-sort)
 *       crates/adapteros-lora-router/src/quantization.rs:172-175 (quantize_gate)
 *       crates/adapteros-lora-router/src/scoring.rs:35-37   (compute_score)
 *       crates/adapteros-numerics/src/noise.rs:308-316      (check_numerics)
 *   - RouterRing layout and fill rules: crates/adapteros-lora-kernel-api/src/lib.rs:57-193,
 *       40-byte GPU form crates/adapteros-lora-kernel-mtl/src/ring_buffer.rs:52-58.
 *   - Ring -> blend weights: crates/adapteros-lora-mlx-ffi/src/backend.rs:398-428 (skip q <= 0,
 *       blend = q / 32767.0f), scale = alpha / rank at backend.rs:462.
 *   - MLX affine int4 dequant w = scale * q + bias, group 64, 8 nibbles per u32, low nibble
 *       first: call sites crates/adapteros-lora-mlx-ffi/src/mlx_cpp_wrapper_real.cpp:925-956
 *       (arithmetic lives in the external, un-vendored Apple MLX library).
 *   - linear / apply_lora / SwiGLU / projections in the MLX fused forward:
 *       mlx_cpp_wrapper_real.cpp:3372-3381 (linear), :3394-3419 (apply_lora),
 *       :3445-3455 (q/k/v + LoRA), :3499-3501 (o + LoRA), :3509-3527 (MLP + LoRA).
 *   - CPU multi-LoRA blend: crates/adapteros-lora-kernel-api/src/liquid.rs:163-257.
 *
 * Parity status per function (how each is pinned: tests/test_oracle_router.py, tests/test_oracle_layer.py):
 *   orc_route_*        pinned by the reference's router KATs, Q15 KATs, closed forms and
 *                      brute force over tie permutations.
 *   orc_quantize_gate  pinned by quantization.rs:239-252 known answers.
 *   orc_dequant_q4     pinned by the closed form over every nibble value and lane position.
 *   orc_liquid_blend   pinned by liquid.rs:267-336 (-> [2.0, 4.0]).
 *   orc_lora_delta     pinned by the lora_cpp_tests.rs:57-119 KAT and closed forms.
 *   orc_linear_q4 / orc_mlp_forward / orc_proj_forward
 *                      pinned against an independent float64 evaluation and closed forms
 *                      (identity weights, zero gates, linearity). MLX's own matmul order,
 *                      fp16 dequant rounding and sigmoid are external and absent: covered to
 *                      tolerance only.
 *   orc_priors         defines the router-logit GEMV of the synthetic workloads (the
 *                      reference takes priors as an input); pinned by a float64 evaluation.
 *   orc_route_one_ex / orc_renormalize_q15 / orc_filter_decision / orc_decision_to_ring
 *                      (router extras: scope hint, adaptive tie-breakers, decision policy,
 *                      active ids and strengths) pinned by the reference's policy_mask.rs and
 *                      router_bridge.rs tests, worker_enforcement_tests.rs, exact rational
 *                      arithmetic for renormalisation, and brute force over tie orders.
 *   orc_rmsnorm / orc_rope / orc_attention (decoder step)
 *                      pinned by the reference's RoPE tests (attention.rs:893-980: position 0 is
 *                      the identity, positions 1 and 5 rotate by 1 and 5 radians), closed forms
 *                      (a constant row normalises to the weights, one visible key returns its
 *                      value, equal scores average the values, causality) and float64
 *                      evaluation.
 *   orc_blake3 / orc_decision_hash
 *                      pinned by the BLAKE3 hashes the reference holds (B3Hash of "" and of
 *                      "hello world"; the BLAKE3 checksums of its source files in
 *                      sbom/cargo-sbom.json, multi-chunk inputs) and by the specification's
 *                      known answer for "abc".
 *   orc_chacha20_block / orc_tie_breakers
 *                      pinned by the RFC 8439 block-function test vectors (section 2.3.2 and
 *                      appendix A.1) and by sorting against the breakers on ties.
 */
#ifndef AOS_ORACLE_H
#define AOS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 40-byte ring, identical to MetalRingBufferLayout (ring_buffer.rs:52-58). */
typedef struct {
  uint32_t top_k;
  uint32_t current_pos;
  uint16_t adapter_indices[8];
  int16_t gates_q15[8];
} orc_ring_t;

/* ---- router ---- */
int16_t orc_quantize_gate(float gate);
uint64_t orc_total_cmp_key_desc(float x);

/* Route one token. priors[n], stable_id[n], allowed[n] (NULL = allow all).
 * Returns k_out (0 = empty decision) or -1 for a non-finite prior / score (the reference's
 * AosError::DeterminismViolation) or k > 8 (Router::new's AosError::Routing). */
int orc_route_one(const float *priors, int n, const uint64_t *stable_id, const uint8_t *allowed,
                  int k, float tau, float eps, float routing_bias, uint16_t idx_out[8],
                  int16_t q15_out[8]);

/* orc_route_one with the router extras: scope[n] (NULL = no hint) replaces the priors of
 * adapters outside the scope with -1e9 (router.rs:1587-1602); breakers[n] (NULL = deterministic
 * mode) order equal scores before stable_id (sort_scores_adaptive, router.rs:265-306). */
int orc_route_one_ex(const float *priors, int n, const uint64_t *stable_id, const uint8_t *allowed,
                     const uint8_t *scope, const uint64_t *breakers, int k, float tau, float eps,
                     float routing_bias, uint16_t idx_out[8], int16_t q15_out[8]);
int orc_route_one_detail(const float *priors, int n, const uint64_t *stable_id, const uint8_t *allowed,
                         const uint8_t *scope, const uint64_t *breakers, int k, float tau, float eps,
                         float routing_bias, uint16_t idx_out[8], int16_t q15_out[8], float *entropy_out,
                         float raw_out[8]);

/* renormalize_gates_q15 (policy_mask.rs:164-213): out[n]. */
void orc_renormalize_q15(const int16_t *q, int n, int16_t *out);

/* filter_decision_by_policy (policy_mask.rs:221-355) over a decision of kk entries with the
 * policy's id/cluster sets as allowed[n] and max_per_token (< 0 = no cap). Returns the new length
 * or -2 (PolicyViolation). */
int orc_filter_decision(const uint16_t *idx, const int16_t *q, int kk, const uint8_t *allowed,
                        int max_per_token, uint16_t *idx_out, int16_t *q_out);

/* decision_to_router_ring_with_active_ids_and_strengths (router_bridge.rs:137-186). Returns 0
 * or -1 (AosError::Routing). */
int orc_decision_to_ring(const uint16_t *idx, const int16_t *q, int kk, const uint16_t *active_ids,
                         const float *strengths, int n_active, int position, orc_ring_t *ring);

/* Route + policy filter + ring conversion for T tokens; status[t] = 0, -1 or -2. */
void orc_route_batch_ex(const float *priors, int T, int n, const uint64_t *stable_id,
                        const uint8_t *allowed, const uint8_t *scope, const uint64_t *breakers, int k,
                        float tau, float eps, float routing_bias, const uint8_t *post_allowed,
                        int post_max, const uint16_t *active_ids, const float *strengths,
                        orc_ring_t *rings, int32_t *status);

/* ChaCha20 block function (RFC 8439 section 2.3) and the adaptive tie-breakers
 * ChaCha20Rng::from_seed(seed).gen::<u64>() x n (rand_chacha 0.3.1, rand 0.8.5). */
void orc_chacha20_block(const uint32_t in[16], uint32_t out[16]);
void orc_tie_breakers(const uint8_t seed[32], int n, uint64_t *out);

/* BLAKE3 (B3Hash::hash; crate blake3 1.8.3) of len bytes, and Router::compute_decision_hash
 * (router.rs:1427-1484) for an empty feature vector: out[96] = input, output, combined hashes.
 * reasoning / backend: 32-byte hashes or NULL. */
void orc_blake3(const uint8_t *in, size_t len, uint8_t out[32]);
void orc_decision_hash(const float *priors, int n, const uint16_t *idx, const int16_t *q, int kk,
                       const uint8_t *reasoning, const uint8_t *backend, uint8_t out[96]);

/* Decoder step pieces of the fused forward (mlx_cpp_wrapper_real.cpp:3249-3390): RMSNorm, RoPE
 * (the fused forward's inv_freq = 1 / theta^(-2i/hd) and half rotation), causal GQA attention over
 * k / v[L][nkv][hd]. mode 0 float32, mode 1 float64. */
void orc_rmsnorm(const float *x, int T, int H, const float *w, float eps, float *y, int mode);
void orc_rope(float *x, int T, int heads, int hd, int offset, float theta);
void orc_attention(const float *q, const float *k, const float *v, int T, int offset, int nh, int nkv, int hd,
                   float *out, int mode);

/* Route T tokens (priors[T*n]) into rings[T]. Returns 0 or -1 (first failing token in *bad_token). */
int orc_route_batch(const float *priors, int T, int n, const uint64_t *stable_id,
                    const uint8_t *allowed, int k, float tau, float eps, float routing_bias,
                    orc_ring_t *rings, int *bad_token);

/* Router-logit GEMV of the synthetic workloads: priors[t*n + a] = sum_i Wr[a*d+i] * f[t*d+i],
 * float32, fixed order: partial sum l (of 64) takes elements 256k + 4l + e (k ascending,
 * e = 0..3) with fmaf, then a xor butterfly over the 64 partial sums. d % 4 == 0. */
void orc_priors(const float *features, const float *router_w, int T, int n, int d, float *priors);

/* ---- int4 base weights (MLX layout) ---- */
float orc_f16_to_f32(uint16_t h);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
uint16_t orc_f32_to_f16(float f);
void orc_dequant_q4(const uint32_t *wp, const uint16_t *scales, const uint16_t *biases, int out,
                    int in, float *w);

/* y[T,out] = x[T,in] . dequant(W)^T ; float32 accumulation in index order (mode 0) or float64
 * (mode 1, result rounded to float). */
void orc_linear_q4(const float *x, int T, const uint32_t *wp, const uint16_t *scales,
                   const uint16_t *biases, int out, int in, float *y, int mode);

/* ---- LoRA ---- */
/* One adapter module: A[r,in], B[out,r] float32 (MLX shapes, mlx_cpp_wrapper_real.cpp:1239-1244). */
typedef struct {
  const float *A;
  const float *B;
} orc_lora_mod_t;

/* delta[out] += ((x . A^T) . B^T) * coef for one token (mode 0 float32, 1 float64 truth). */
void orc_lora_delta(const float *x, const float *A, const float *B, int r, int in, int out,
                    float coef, float *delta, int first, int mode);

/* liquid.rs:163-257 for n adapters (A as "down" [r,in], B as "up" [out,r]). */
int orc_liquid_blend(int n, const float *const *A, const float *const *B, const int *rank,
                     const float *alpha, const float *coef, const float *x, int in, float *out,
                     int out_len);

/* ---- layer forwards (per-token rings) ----
 * adapters[a] gives module m of adapter a at mods[a * n_modules + m]; scale[a] = alpha / rank.
 * A ring slot with q <= 0 or an index >= n_adapters is skipped (backend.rs:409-425). */
typedef struct {
  const uint32_t *wp;
  const uint16_t *scales;
  const uint16_t *biases;
} orc_q4_t;

/* SwiGLU MLP (mlx_cpp_wrapper_real.cpp:3509-3527): modules 0=gate, 1=up, 2=down. */
void orc_mlp_forward(const float *x, int T, int H, int I, const orc_q4_t *gate,
                     const orc_q4_t *up, const orc_q4_t *down, const orc_lora_mod_t *mods,
                     const float *scale, int n_adapters, int rank, const orc_ring_t *rings,
                     float *y, int mode, float *h_out);

/* One projection with LoRA (mlx_cpp_wrapper_real.cpp:3445-3455, 3499-3501); module index m of
 * n_modules in mods. */
void orc_proj_forward(const float *x, int T, int in, int out, const orc_q4_t *w,
                      const orc_lora_mod_t *mods, int n_modules, int m, const float *scale,
                      int n_adapters, int rank, const orc_ring_t *rings, float *y, int mode);

/* float64 exp used by the router (libm, as Rust's f64::exp). Exposed for the pinning test;
 * orc_set_exp(NULL) restores libm, a non-NULL pointer substitutes another implementation. */
double orc_exp(double x);
void orc_set_exp(double (*f)(double));

int orc_num_threads(void);
void orc_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
