/*
 * aoship.h — C ABI of the MI355X (gfx950) adapter-augmented inference hot path.
 *
 * One hot path of adapterOS, rebuilt for one MI355X: the K-sparse router's Q15 top-K gating
 * feeding fused int4 (MLX affine, group 64) linear layers — a SwiGLU MLP or the attention
 * projections — that add the selected adapters' low-rank deltas
 *     y = W_q4 . x + sum_k (scale_k * q_k / 32767) * B_k . (A_k . x).
 *
 * The ABI follows the conventions of the reference's MLX FFI
 * (crates/adapteros-lora-mlx-ffi/wrapper.h):
 *   - opaque handles; constructors return NULL on error, other calls return 0 / -1;
 *   - the error text of the last failing call on this thread is read with
 *     aoship_get_last_error() and cleared with aoship_clear_error();
 *   - the caller owns every buffer it passes; weights are copied to device memory by the
 *     set_* calls, so host arrays may be released when those return;
 *   - calls on one handle must be serialised by the caller (the reference serialises every
 *     forward with a mutex: crates/adapteros-lora-mlx-ffi/src/lib.rs:420-425,1250).
 *
 * Pointers documented as "device" are HIP device pointers on the device chosen by
 * aoship_init(); the compute calls are asynchronous on the handle's stream (default: the null
 * stream) and allocate nothing once aoship_layer_reserve() has sized the workspace.
 */
#ifndef AOSHIP_H
#define AOSHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AOSHIP_MAX_K 8           /* crates/adapteros-core/src/defaults.rs:37 (MAX_K) */
#define AOSHIP_Q15_DENOM 32767.0f /* crates/adapteros-core/src/invariants.rs:107 */
#define AOSHIP_GROUP_SIZE 64
#define AOSHIP_BITS 4

/* Router decision handed to the layer kernels: the 40-byte GPU form of RouterRing
 * (crates/adapteros-lora-kernel-api/src/lib.rs:57-71; byte layout of MetalRingBufferLayout,
 * crates/adapteros-lora-kernel-mtl/src/ring_buffer.rs:52-58). Unused slots are zero. */
typedef struct aoship_ring {
  uint32_t top_k;
  uint32_t current_pos;
  uint16_t adapter_indices[8];
  int16_t gates_q15[8];
} aoship_ring_t;

typedef uint16_t aoship_bf16_t; /* bfloat16 bit pattern */

typedef struct aoship_router aoship_router_t;
typedef struct aoship_layer aoship_layer_t;
typedef struct aoship_lora_adapter aoship_lora_adapter_t;

/* ---- errors, version, device -------------------------------------------------------------- */

/* Replaces mlx_get_last_error / mlx_clear_error (wrapper.h:199-200). Thread-local text. */
const char *aoship_get_last_error(void);
void aoship_clear_error(void);

/* Library version string. */
const char *aoship_version(void);

/* Select the HIP device used by later calls on this process (mirrors the MLX backend's device
 * selection, crates/adapteros-lora-kernel-mtl/src/lib.rs:397-399). Returns 0 / -1. */
int aoship_init(int device);

/* Device name, as FusedKernels::device_name (crates/adapteros-lora-kernel-api/src/lib.rs:374).
 * Writes at most len bytes including the terminator. Returns 0 / -1. */
int aoship_device_name(char *buf, int len);

/* Wait for all work on the device (the reference's commit/wait device boundary,
 * crates/adapteros-lora-kernel-mtl/src/fused_mlp.rs:233-234). Returns 0 / -1. */
int aoship_sync(void);

/* Determinism attestation as JSON text, the counterpart of FusedKernels::attest_determinism
 * (crates/adapteros-lora-kernel-api/src/lib.rs:383, DeterminismReport in attestation.rs:130-234).
 * Returns the number of bytes needed (excluding the terminator) or -1. */
int aoship_attest_determinism(char *buf, int len);

/* B3Hash::hash (adapteros-core, crate blake3 1.8.3): the 32-byte BLAKE3 hash of len bytes,
 * computed on the host with the same compression and tree code the router kernel uses for
 * decision hashes. Returns 0 / -1. */
int aoship_blake3(const void *data, size_t len, uint8_t *out);

/* ---- router ---------------------------------------------------------------------------------- */

/* Router::new_with_weights(k, tau, eps) + set_routing_bias (crates/adapteros-lora-router/src/
 * router.rs:397-428, 556-562, 769-785) for n_adapters adapters whose AdapterInfo::stable_id are
 * stable_ids[n] (host; NULL = all zero, the AdapterInfo default, types.rs:645-664).
 * k > 8 fails like Router::new; k == 0 is lifted to 1; tau and eps are sanitised as
 * router.rs:146-187; a non-finite or non-positive routing_bias keeps 1.0. n_adapters <= 4096. */
aoship_router_t *aoship_router_new(int n_adapters, int k, float tau, float eps,
                                   float routing_bias, const uint64_t *stable_ids);

/* PolicyMask::allowed (crates/adapteros-lora-router/src/policy_mask.rs): allowed[n] host bytes,
 * nonzero = allowed; NULL = allow all. Returns 0 / -1. */
int aoship_router_set_policy_mask(aoship_router_t *router, const uint8_t *allowed);

/* Scope hint of Router::route_with_adapter_info_and_scope_with_ctx (router.rs:1587-1602):
 * in_scope[n] host bytes, nonzero where AdapterInfo::scope_path equals the hint; the other
 * adapters score from a prior of -1e9 (the decision hash, when on, sees those priors). The
 * reference ignores a hint that matches no adapter: pass NULL then, as for no hint. */
int aoship_router_set_scope(aoship_router_t *router, const uint8_t *in_scope);

/* Adaptive routing (Router::set_adaptive_routing, router.rs:577; tie-breakers :1705-1724):
 * seed[32] = DeterminismContext::router_tiebreak_seed() (adapteros-core/src/determinism.rs:
 * 172-176). Adapter a gets breaker_a, the a-th ChaCha20Rng::from_seed(seed).gen::<u64>()
 * (rand 0.8.5, rand_chacha 0.3.1), and equal scores are ordered by (breaker, stable_id, index)
 * (sort_scores_adaptive, router.rs:265-306); the canonical re-sort keeps stable_id. NULL = back
 * to deterministic mode. Returns 0 / -1. */
int aoship_router_set_adaptive_seed(aoship_router_t *router, const uint8_t *seed);

/* The breakers of aoship_router_set_adaptive_seed, computed on the host (no device needed):
 * out[a] = the a-th ChaCha20Rng::from_seed(seed).gen::<u64>() for a < n, what the reference
 * reports in its tie-break diagnostics (router.rs:1780-1800). Returns 0 / -1. */
int aoship_adaptive_tie_breakers(const uint8_t *seed, int n, uint64_t *out);

/* filter_decision_by_policy (crates/adapteros-lora-router/src/policy_mask.rs:221-355) on every
 * decision before its ring is written: allowed[n] host bytes, nonzero where the adapter passes the
 * RoutingPolicy's id and cluster allow/deny sets; max_adapters_per_token < 0 = no cap. Entries
 * keep decision order; when any is removed the gates are renormalised (renormalize_gates_q15,
 * :164-213). No entry left (or a cap of 0) is AosError::PolicyViolation: status -2. NULL allowed
 * = no policy. Returns 0 / -1. */
int aoship_router_set_decision_policy(aoship_router_t *router, const uint8_t *allowed,
                                      int max_adapters_per_token);

/* Decision -> ring as decision_to_router_ring_with_active_ids_and_strengths
 * (crates/adapteros-lora-worker/src/router_bridge.rs:137-186): ring index = active_ids[decision
 * index] (NULL = the decision index; 65535 zero-fills the ring as set_with_max_adapter does),
 * gate = round(gate * clamp(strengths[decision index], 0, 1)) (NULL = unscaled). Host arrays of
 * n_adapters entries. Returns 0 / -1. */
int aoship_router_set_ring_mapping(aoship_router_t *router, const uint16_t *active_ids,
                                   const float *strengths);

/* RouterDeterminismConfig::enable_decision_hashing (router.rs:1879-1890): with hashes != NULL,
 * each later route call writes, for token t, 96 bytes at hashes + 96 t: the input, output and
 * combined BLAKE3 hashes of Router::compute_decision_hash (router.rs:1427-1484) for the router's
 * decision (before any decision policy) with an empty feature vector:
 *   input    = BLAKE3(the routed priors, float32 LE [|| reasoning_hash])
 *   output   = BLAKE3(indices u16 LE || gates i16 LE [|| reasoning_hash])
 *   combined = BLAKE3(input || output [|| reasoning_hash] [|| backend_identity_hash])
 * 96 zero bytes for a token without a decision (the reference's decision_hash: None). DecisionHash
 * reports the first 8 bytes of each as hex (B3Hash::to_short_hex). hashes: device buffer of
 * max_tokens * 96 bytes, used until this is called again; reasoning_hash / backend_identity_hash:
 * 32-byte host hashes or NULL. hashes == NULL turns hashing off. Returns 0 / -1. */
int aoship_router_set_decision_hashing(aoship_router_t *router, uint8_t *hashes, int max_tokens,
                                       const uint8_t *reasoning_hash,
                                       const uint8_t *backend_identity_hash);

/* The Decision beyond its ring (types.rs:676-687): the Shannon entropy of the renormalised gates
 * (Router::compute_entropy, router.rs:1287-1293, applied at :1844) and the candidates
 * (DecisionCandidate: adapter index, raw score, Q15 gate), in decision order. After a decision
 * policy the candidates are those that passed, with their gates from before the renormalisation,
 * and the entropy is the router's (filter_decision_by_policy, policy_mask.rs:221-355). A token
 * without a decision has entropy 0 and no candidates. */
typedef struct {
  float entropy;
  uint32_t n_candidates;
  uint16_t adapter_idx[8];
  int16_t gate_q15[8];
  float raw_score[8];
} aoship_decision_t;

/* With decisions != NULL, each later route call writes token t's Decision details to
 * decisions[t] (device buffer of max_tokens entries, used until this is called again). The
 * entropy's log2 is computed in double precision and rounded to float; the products and the sum
 * are float32 in top-K order, as the reference's. decisions == NULL turns this off. Returns 0 / -1. */
int aoship_router_set_decision_output(aoship_router_t *router, aoship_decision_t *decisions, int max_tokens);

/* Stream (hipStream_t) for this router's launches; NULL = null stream. Returns 0 / -1. */
int aoship_router_set_stream(aoship_router_t *router, void *stream);

void aoship_router_free(aoship_router_t *router);

/* Route T tokens with an empty feature vector: the replacement for
 * Router::route_with_adapter_info_and_scope_with_ctx (router.rs:1567-1952) followed by
 * Decision -> RouterRing (types.rs:699-706, kernel-api lib.rs:122-193), with the extras set above.
 *   priors  : device float[T * n_adapters]
 *   rings   : device aoship_ring_t[T] (written)
 *   status  : device int32[T] or NULL; 0 = decision written, -1 = non-finite prior or score
 *             (AosError::DeterminismViolation, router.rs:611-625,1640-1686), -2 = decision
 *             policy left no adapter (AosError::PolicyViolation); ring zero-filled on -1 / -2.
 * Asynchronous. Returns 0 / -1 (argument errors only). */
int aoship_route(aoship_router_t *router, const float *priors, int T, aoship_ring_t *rings,
                 int32_t *status);

/* Route with priors computed on the device from router features: priors[t, a] =
 * sum_i router_w[a, i] * features[t, i] in float32 with a fixed reduction order (64 partial
 * sums, partial l taking elements 256k + 4l + e in order with fused multiply-adds, then a xor
 * butterfly), then as aoship_route. d must be a multiple of 4 and d + n_adapters <= 15360.
 *   features   : device float[T * d];  router_w : device float[n_adapters * d]
 *   priors_out : device float[T * n_adapters] or NULL. */
int aoship_route_features(aoship_router_t *router, const float *features, const float *router_w,
                          int d, int T, aoship_ring_t *rings, float *priors_out,
                          int32_t *status);

/* ---- LoRA adapters (mirrors wrapper.h:375-420) --------------------------------------------- */

/* mlx_lora_adapter_new (mlx_cpp_wrapper_real.cpp:3164-3175): scale = alpha / rank. */
aoship_lora_adapter_t *aoship_lora_adapter_new(int adapter_id, int num_layers, float scale);

/* mlx_lora_adapter_set_module (mlx_cpp_wrapper_real.cpp:3177-3205) with the arrays passed as
 * host float32 data in MLX shapes: lora_a[rank * in_features], lora_b[out_features * rank].
 * module is one of q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj. The weights
 * are stored on the device as bfloat16, rank padded to a multiple of 16 with zeros.
 * rank <= 128. Returns 0 / -1. */
int aoship_lora_adapter_set_module(aoship_lora_adapter_t *adapter, int layer_idx,
                                   const char *module, int rank, int in_features,
                                   int out_features, const float *lora_a, const float *lora_b);

/* mlx_lora_adapter_free (mlx_cpp_wrapper_real.cpp:3207-3211). Device memory is released when
 * no layer still binds the adapter. */
void aoship_lora_adapter_free(aoship_lora_adapter_t *adapter);

/* ---- layers ----------------------------------------------------------------------------------- */

/* A transformer layer's adapter-augmented projections (layer_idx selects the adapters' layer). */
aoship_layer_t *aoship_layer_new(int layer_idx, int group_size, int bits);

/* Upload one base projection in MLX 4-bit layout (get_weight_with_dequant,
 * mlx_cpp_wrapper_real.cpp:925-956): packed[out * in/8] uint32 with 8 nibbles per word, low
 * nibble first; scales_f16 / biases_f16[out * in/64] float16 bit patterns (biases NULL = 0).
 * Requires out % 32 == 0 and in % 64 == 0. Returns 0 / -1. */
int aoship_layer_set_base(aoship_layer_t *layer, const char *module, int out_features,
                          int in_features, const uint32_t *packed, const uint16_t *scales_f16,
                          const uint16_t *biases_f16);

/* Bind the adapter table: ring adapter index a selects table[a] (NULL entries are skipped, as a
 * missing FFI handle is in prepare_lora_for_ring, crates/adapteros-lora-mlx-ffi/src/
 * backend.rs:398-428). All adapters bound for one module must share its rank. Returns 0 / -1. */
int aoship_layer_set_adapters(aoship_layer_t *layer, aoship_lora_adapter_t *const *table, int n);

/* Size the device workspace for calls of up to max_tokens tokens: the MLP when gate, up and down
 * are set, q/k/v together and every projection alone. Forwards within that size allocate
 * nothing. Returns 0 / -1. */
int aoship_layer_reserve(aoship_layer_t *layer, int max_tokens);

/* Stream (hipStream_t) for this layer's launches; NULL = null stream. Returns 0 / -1. */
int aoship_layer_set_stream(aoship_layer_t *layer, void *stream);

/* Per-kernel timing with HIP events on the layer's stream (FusedKernels::get_metrics,
 * crates/adapteros-lora-kernel-api/src/lib.rs:559). enable != 0 turns it on and clears totals. */
int aoship_layer_set_profiling(aoship_layer_t *layer, int enable);

/* Kernel statistics slot idx: name, accumulated milliseconds, launches. Synchronises the
 * stream. Returns the number of slots, or -1. */
int aoship_layer_kernel_stats(aoship_layer_t *layer, int idx, const char **name,
                              double *total_ms, int64_t *launches);

/* Health of the layer's decode launches (part of the metrics surface, FusedKernels::get_metrics,
 * crates/adapteros-lora-kernel-api/src/lib.rs:559): at decode each LoRA shrink runs in the first
 * workgroups of the GEMV launch that reads its result, and the GEMV workgroups wait for it with a
 * bounded wait (about a second). Returns 1 if such a wait gave up since the last call (the
 * outputs of that forward are then invalid), else 0, and clears the flag; -1 on error.
 * Synchronises the device. */
int aoship_layer_wait_timeouts(aoship_layer_t *layer);

void aoship_layer_free(aoship_layer_t *layer);

/* SwiGLU MLP with LoRA on gate/up/down (mlx_cpp_wrapper_real.cpp:3509-3527):
 *   gate = x Wg^T + dg(x); up = x Wu^T + du(x); h = gate * sigmoid(gate) * up;
 *   y = h Wd^T + dd(h)
 * where d(.) sums, over each token's ring slots with q > 0 and a bound adapter,
 * (. A^T) B^T * (scale * q / 32767).
 *   x : device bf16[T * hidden];  rings : device aoship_ring_t[T] (one per token);
 *   y : device bf16[T * hidden]. Asynchronous. Returns 0 / -1. */
int aoship_mlp_forward(aoship_layer_t *layer, const aoship_bf16_t *x, int T,
                       const aoship_ring_t *rings, aoship_bf16_t *y);

/* No counterpart in the reference: the decode MLP forward (aoship_mlp_forward's launches, T <= 32)
 * for callers that cannot allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc). Its workspace, counters and flags live in a static device array
 * of 32 MiB (about 29.75 MiB of workspace) that each GPU holds until the process ends; a layer and
 * token count whose workspace does not fit is rejected with an error (-1), as is T > 32. Makes no
 * hipMalloc, hipFree or other allocating call. The array keeps the last call's contents; calls that
 * overlap on one GPU (on different streams) share it and race: serialise them. Output equals
 * aoship_mlp_forward's bit for bit. Returns 0 / -1. */
int aoship_mlp_forward_noalloc(aoship_layer_t *layer, const aoship_bf16_t *x, int T,
                               const aoship_ring_t *rings, aoship_bf16_t *y);

/* One decode step of a layer's MLP with its tokens routed in the same call: the router's decision
 * from features (aoship_route_features: Router::route_with_adapter_info_and_scope_with_ctx,
 * router.rs:1567-1952, with the plain router settings) feeds the MLP (aoship_mlp_forward: the
 * fused forward's MLP, mlx_cpp_wrapper_real.cpp:3509-3527). rings (and status, may be NULL)
 * receive the decisions as aoship_route_features writes them; y equals aoship_mlp_forward's
 * output for those rings. For T <= 32 with no router extras set, the router runs in the first
 * workgroups of the gate/up launch, beside the LoRA shrink and the weight stream; otherwise the
 * calls run one after the other. Everything runs on the layer's stream. Returns 0 / -1. */
int aoship_route_mlp_forward(aoship_router_t *router, const float *features, const float *router_w, int d,
                             aoship_layer_t *layer, const aoship_bf16_t *x, int T, aoship_ring_t *rings,
                             int32_t *status, aoship_bf16_t *y);

/* One projection with LoRA (mlx_cpp_wrapper_real.cpp:3445-3455 for q/k/v, 3499-3501 for o).
 *   x : device bf16[T * in];  y : device bf16[T * out]. Returns 0 / -1. */
int aoship_proj_forward(aoship_layer_t *layer, const char *module, const aoship_bf16_t *x,
                        int T, const aoship_ring_t *rings, aoship_bf16_t *y);

/* q/k/v projections of one input in one pass (mlx_cpp_wrapper_real.cpp:3445-3455). */
int aoship_qkv_forward(aoship_layer_t *layer, const aoship_bf16_t *x, int T,
                       const aoship_ring_t *rings, aoship_bf16_t *q, aoship_bf16_t *k,
                       aoship_bf16_t *v);

/* ---- decoder model: FusedKernels::run_step's token -> logits path ---------------------------- */

typedef struct aoship_model aoship_model_t;

/* Shape of a decoder-only model (the MLX wrapper's model config). max_seq sizes the KV cache. */
typedef struct {
  int num_layers, hidden, intermediate, num_heads, num_kv_heads, head_dim, vocab, max_seq;
  float rope_theta, rms_eps;
} aoship_model_config_t;

/* A model of num_layers layers with its KV cache (mlx_model_load + mlx_kv_cache_new,
 * wrapper.h). hidden a multiple of 64 up to 16384, intermediate a multiple of 64; num_heads a
 * multiple of num_kv_heads;
 * head_dim a multiple of 8 up to 256; vocab a multiple of 32. Norm weights start at 1, biases
 * absent. NULL on error. */
aoship_model_t *aoship_model_new(const aoship_model_config_t *config);
void aoship_model_free(aoship_model_t *model);

/* Layer i of the model: set its seven projections with aoship_layer_set_base. */
aoship_layer_t *aoship_model_layer(aoship_model_t *model, int layer_idx);

/* model.embed_tokens: MLX 4-bit rows (packed[vocab * hidden/8], float16 scales and biases
 * [vocab * hidden/64], biases NULL = 0) or, with packed NULL, bfloat16 rows[vocab * hidden]
 * (the fused forward's take(embed, ids), mlx_cpp_wrapper_real.cpp:3421-3432). Host arrays. */
int aoship_model_set_embedding(aoship_model_t *model, const uint32_t *packed, const uint16_t *scales_f16,
                               const uint16_t *biases_f16, const uint16_t *rows_bf16);

/* lm_head in MLX 4-bit layout [vocab x hidden] (a model with tied embeddings passes its
 * embedding arrays). Host arrays. */
int aoship_model_set_lm_head(aoship_model_t *model, const uint32_t *packed, const uint16_t *scales_f16,
                             const uint16_t *biases_f16);

/* RMSNorm weights (float32 host [hidden]): layer_idx >= 0 with which 0 = input_layernorm,
 * 1 = post_attention_layernorm; layer_idx = -1 = model.norm. */
int aoship_model_set_norm(aoship_model_t *model, int layer_idx, int which, const float *weight);

/* q_proj / k_proj / v_proj bias of a layer (float32 host [out]; NULL removes it). */
int aoship_model_set_bias(aoship_model_t *model, int layer_idx, const char *module, const float *bias);

/* aoship_layer_set_adapters on every layer. */
int aoship_model_set_adapters(aoship_model_t *model, aoship_lora_adapter_t *const *table, int n);

/* Stream for the model's launches (its layers included); NULL = null stream. */
int aoship_model_set_stream(aoship_model_t *model, void *stream);

/* Sizes every workspace for calls of up to max_tokens tokens, so forwards allocate nothing. */
int aoship_model_reserve(aoship_model_t *model, int max_tokens);

/* The KV cache: emptied, and its length (positions held). */
int aoship_model_reset_cache(aoship_model_t *model);
int aoship_model_cache_len(const aoship_model_t *model);

/* mlx_model_forward_with_cache_and_lora (mlx_cpp_wrapper_real.cpp:3339-3527) for T tokens:
 * embedding, then per layer RMSNorm, q/k/v (+bias, +LoRA), RoPE, K/V appended to the cache,
 * causal GQA attention over the cache, o_proj (+LoRA), residual, RMSNorm, SwiGLU MLP (+LoRA),
 * residual; final RMSNorm; logits[vocab] (device float32) of the last token.
 *   ids   : device int32[T];  rings : device aoship_ring_t[T] (each token's adapters and gates)
 *   position_offset must equal aoship_model_cache_len (tokens extend the cached sequence), and
 *   the cache must hold position_offset + T positions. Asynchronous. Returns 0 / -1. */
int aoship_model_forward(aoship_model_t *model, const int32_t *ids, int T, int position_offset,
                         const aoship_ring_t *rings, float *logits);

/* ---- Liquid blend (crates/adapteros-lora-kernel-api/src/liquid.rs) ------------------------ */

#define AOSHIP_LIQUID_MAX_ADAPTERS 3 /* liquid.rs:12 (LIQUID_MAX_ADAPTERS) */
#define AOSHIP_LIQUID_MAX_RANK 1024  /* per adapter, this backend's limit */

/* LiquidTensor (liquid.rs:66-104): a row-major device matrix of float32 (bf16 == 0) or bfloat16
 * bit patterns (bf16 == 1); len is the buffer's element count, which rows * cols must equal. */
typedef struct {
  const void *data;
  int bf16;
  int rows, cols;
  size_t len;
} aoship_liquid_tensor_t;

/* LiquidAdapterRef (liquid.rs:106-116): down = A [rank x in_features], up = B [out_features x
 * rank], alpha. */
typedef struct {
  uint16_t id;
  aoship_liquid_tensor_t down, up;
  float alpha;
} aoship_liquid_adapter_t;

/* LiquidKernel::blend_and_forward (liquid.rs:147-160) with the result of
 * blend_and_forward_reference (liquid.rs:163-257): output[0 .. out_len) = 0; then for each adapter
 * in order whose coefficient is not 0, rank_buf = down . input and, for o < up.rows,
 * output[o] += coefficient * (up[o, :] . rank_buf) * (alpha / rank), in float32. The checks are
 * the reference's, in its order (at least one and at most AOSHIP_LIQUID_MAX_ADAPTERS adapters, one
 * coefficient per adapter, rows * cols == len for each tensor, down.cols == in_len,
 * up.rows <= out_len, up.cols == down.rows), plus rank <= AOSHIP_LIQUID_MAX_RANK and non-NULL,
 * aligned device pointers. *precision (may be NULL) receives LiquidBlendStats::precision: 0
 * (float32) or 1 (some tensor is bfloat16). Weights, input and output are device memory; adapters
 * and coefficients are host arrays. Runs asynchronously on stream (hipStream_t; NULL = the null
 * stream) and allocates nothing. Returns 0 / -1 (aoship_last_error). */
int aoship_liquid_blend_and_forward(const aoship_liquid_adapter_t *adapters, int n_adapters,
                                    const float *coefficients, int n_coefficients, const float *input,
                                    int in_len, float *output, int out_len, int *precision, void *stream);

#ifdef __cplusplus
}
#endif
#endif
