// aos_kernel_api.hpp — C++ host side of the MI355X hot path, above the C ABI (include/aoship.h).
//
// Mirrors, for the adapter-augmented layer path, the Rust types a backend of adapterOS works with:
//   RouterRing                crates/adapteros-lora-kernel-api/src/lib.rs:57-214
//   AdapterLoadMetadata       crates/adapteros-lora-kernel-api/src/lib.rs:249-257
//   AdapterInfo / Decision    crates/adapteros-lora-router/src/types.rs:645-707
//   PolicyMask (allow/deny)   crates/adapteros-lora-router/src/policy_mask.rs
//   Router                    crates/adapteros-lora-router/src/router.rs:397-428, 556-562,
//                             769-785 (construction), 1567-1952 (routing: scope hint, adaptive
//                             tie-breakers, decision hash), 1427-1484 (compute_decision_hash)
//   RoutingPolicy filter      crates/adapteros-lora-router/src/policy_mask.rs:221-355
//   ring conversion           crates/adapteros-lora-worker/src/router_bridge.rs:137-186
//   FusedKernels (hot-swap, device_name, attest_determinism, layer forwards)
//                             crates/adapteros-lora-kernel-api/src/lib.rs:308-716
//   adapter ingest            crates/adapteros-lora-mlx-ffi/src/backend.rs:891-893, 1017-1210
//                             (safetensors bytes + metadata), 448-522 (every layer, failed modules
//                             skipped); base weights as mlx_cpp_wrapper_real.cpp:683, 925-956 read them
// Errors are thrown as AosError with the reference's error kinds (AosError::Kernel, ::Validation,
// ::Routing, ::DeterminismViolation, ::Parse, ::Io, ::PolicyViolation, ::Config); a Rust Result<T>
// maps to a return value or a throw.
//
// Header-only; link against libaoship.so and the HIP runtime (device buffers for the host-side
// routing convenience call).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <optional>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/aoship.h"
#include "aos_determinism.hpp"
#include "aos_ingest.hpp"

namespace adapteros {

enum class ErrorKind { Kernel, Validation, Routing, DeterminismViolation, Parse, Io, PolicyViolation, Config };

class AosError : public std::runtime_error {
 public:
  AosError(ErrorKind kind, const std::string &msg) : std::runtime_error(msg), kind_(kind) {}
  ErrorKind kind() const { return kind_; }

 private:
  ErrorKind kind_;
};

namespace detail {
inline std::string last_error() {
  const char *e = aoship_get_last_error();
  return e ? std::string(e) : std::string();
}
inline void check(int rc, ErrorKind kind, const char *what) {
  if (rc != 0) throw AosError(kind, std::string(what) + ": " + last_error());
}
inline void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw AosError(ErrorKind::Kernel, std::string(what) + ": " + hipGetErrorString(e));
}
}  // namespace detail

// ---- RouterRing (kernel-api/src/lib.rs:57-214), release-build semantics -----------------------

struct RouterRing {
  std::array<uint16_t, 8> indices{};
  std::array<int16_t, 8> gates_q15{};
  size_t position = 0;
  size_t k = 0;
  uint32_t dropout_seed = 0;
  float dropout_rate = 0.0f;

  // RouterRing::new(k): K above 8 is clamped (the release-build behaviour).
  static RouterRing with_k(size_t k) {
    RouterRing r;
    r.k = k < 8 ? k : 8;
    return r;
  }

  size_t len() const { return k; }
  bool is_empty() const { return k == 0; }

  void set(const std::vector<uint16_t> &idx, const std::vector<int16_t> &gates) {
    set_with_max_adapter(idx, gates, UINT16_MAX);
  }

  // set_with_max_adapter (lib.rs:122-193): mismatched lengths or an index >= max_adapter
  // zero-fill the ring (release builds); K is clamped to 8; unused entries are zeroed.
  void set_with_max_adapter(const std::vector<uint16_t> &idx, const std::vector<int16_t> &gates,
                            uint16_t max_adapter) {
    if (idx.size() != gates.size()) {
      indices.fill(0);
      gates_q15.fill(0);
      k = 0;
      return;
    }
    const size_t kk = idx.size() < 8 ? idx.size() : 8;
    for (size_t i = 0; i < idx.size(); ++i)
      if (idx[i] >= max_adapter) {
        indices.fill(0);
        gates_q15.fill(0);
        k = 0;
        return;
      }
    indices.fill(0);
    gates_q15.fill(0);
    for (size_t i = 0; i < kk; ++i) {
      indices[i] = idx[i];
      gates_q15[i] = gates[i];
    }
    k = kk;
  }

  std::vector<uint16_t> active_indices() const { return {indices.begin(), indices.begin() + k}; }
  std::vector<int16_t> active_gates() const { return {gates_q15.begin(), gates_q15.begin() + k}; }

  // The 40-byte device form (MetalRingBufferLayout, kernel-mtl/src/ring_buffer.rs:52-58).
  aoship_ring_t to_device() const {
    aoship_ring_t r;
    std::memset(&r, 0, sizeof(r));
    r.top_k = (uint32_t)k;
    r.current_pos = (uint32_t)position;
    for (size_t i = 0; i < 8; ++i) {
      r.adapter_indices[i] = indices[i];
      r.gates_q15[i] = gates_q15[i];
    }
    return r;
  }

  static RouterRing from_device(const aoship_ring_t &d) {
    RouterRing r = with_k(d.top_k);
    r.position = d.current_pos;
    for (size_t i = 0; i < 8; ++i) {
      r.indices[i] = d.adapter_indices[i];
      r.gates_q15[i] = d.gates_q15[i];
    }
    return r;
  }
};

// ---- router-side types (router/src/types.rs) ----------------------------------------------------

struct AdapterInfo {
  std::string id;
  uint64_t stable_id = 0;
  std::optional<std::string> scope_path;
};

// DecisionHash (types.rs:386-415): short hex (first 8 bytes) of each BLAKE3 hash.
struct DecisionHash {
  std::string input_hash, output_hash, combined_hash;
  std::optional<std::string> reasoning_hash, backend_identity_hash;
  float tau = 0.0f, eps = 0.0f;
  size_t k = 0;
};

// RouterDeterminismConfig (types.rs:370-384); decision hashing is on by default there too.
struct RouterDeterminismConfig {
  bool ieee754_deterministic = true;
  bool enable_decision_hashing = true;
};

// DecisionCandidate (types.rs:669-674): a routed adapter with its raw score and Q15 gate.
struct DecisionCandidate {
  uint16_t adapter_idx = 0;
  float raw_score = 0.0f;
  int16_t gate_q15 = 0;
};

// Decision (types.rs:676-687): entropy is Router::compute_entropy of the renormalised gates
// (router.rs:1287-1293), candidates are in decision order (after a policy: those that passed).
struct Decision {
  std::vector<uint16_t> indices;
  std::vector<int16_t> gates_q15;
  float entropy = 0.0f;
  std::vector<DecisionCandidate> candidates;
  std::optional<DecisionHash> decision_hash;

  std::vector<float> gates_f32() const {
    std::vector<float> g;
    for (int16_t q : gates_q15) g.push_back((float)q / AOSHIP_Q15_DENOM);
    return g;
  }

  // Decision::to_router_ring (types.rs:699-706).
  RouterRing to_router_ring() const {
    if (indices.size() > 8) throw AosError(ErrorKind::Validation, "Decision has too many adapters (k > 8)");
    RouterRing r = RouterRing::with_k(indices.size());
    r.set(indices, gates_q15);
    return r;
  }
};

// PolicyMask: allowed[i] for adapter i (allow_all, or deny by adapter id).
struct PolicyMask {
  std::vector<uint8_t> allowed;
  static PolicyMask allow_all(size_t n) { return PolicyMask{std::vector<uint8_t>(n, 1)}; }
  static PolicyMask deny(const std::vector<AdapterInfo> &info, const std::vector<std::string> &denied) {
    PolicyMask m = allow_all(info.size());
    for (size_t i = 0; i < info.size(); ++i)
      for (const auto &d : denied)
        if (info[i].id == d) m.allowed[i] = 0;
    return m;
  }
};

// RoutingPolicy (the fields filter_decision_by_policy reads, adapteros-api-types) and the per-adapter
// pass bytes the device filter takes: an adapter passes when it is in allowed_adapter_ids (if set),
// not in denied_adapter_ids, has a cluster in allowed_clusters (if set) and no cluster in
// denied_clusters (policy_mask.rs:246-315).
struct RoutingPolicy {
  std::optional<std::vector<std::string>> allowed_adapter_ids, denied_adapter_ids, allowed_clusters,
      denied_clusters;
  std::optional<size_t> max_adapters_per_token;
};

inline std::vector<uint8_t> routing_policy_pass_bytes(const RoutingPolicy &policy,
                                                     const std::vector<std::string> &adapter_ids,
                                                     const std::vector<std::optional<std::string>> &clusters) {
  if (adapter_ids.size() != clusters.size())
    throw AosError(ErrorKind::PolicyViolation, "RoutingPolicy adapter ids/clusters length mismatch");
  auto as_set = [](const std::optional<std::vector<std::string>> &v) {
    return v ? std::optional<std::set<std::string>>(std::set<std::string>(v->begin(), v->end())) : std::nullopt;
  };
  const auto allowed = as_set(policy.allowed_adapter_ids), denied = as_set(policy.denied_adapter_ids),
             allowed_c = as_set(policy.allowed_clusters), denied_c = as_set(policy.denied_clusters);
  std::vector<uint8_t> pass(adapter_ids.size(), 0);
  for (size_t i = 0; i < adapter_ids.size(); ++i) {
    const std::string &id = adapter_ids[i];
    const std::optional<std::string> &c = clusters[i];
    bool ok = true;
    if (allowed && !allowed->count(id)) ok = false;
    if (denied && denied->count(id)) ok = false;
    if (allowed_c && (!c || !allowed_c->count(*c))) ok = false;
    if (denied_c && c && denied_c->count(*c)) ok = false;
    pass[i] = ok ? 1 : 0;
  }
  return pass;
}

// ---- Router (empty feature vector) ------------------------------------------------------------------

class Router {
 public:
  // Router::new_with_weights(.., k, tau, eps): k > 8 fails with AosError::Routing (router.rs:769-777);
  // tau / eps are sanitised by the device router as router.rs:146-187.
  // The device (default 0) is selected on first use.
  Router(size_t k, float tau, float eps, int device = 0) : k_(k), tau_(tau), eps_(eps), device_(device) {
    if (k > AOSHIP_MAX_K)
      throw AosError(ErrorKind::Routing, "Adapter routing failed: K exceeds maximum allowed value of 8");
  }
  ~Router() { release(); }
  Router(const Router &) = delete;
  Router &operator=(const Router &) = delete;

  void set_routing_bias(float bias) {
    bias_ = bias;
    release();
  }

  // Router::set_routing_determinism_mode (router.rs:577): adaptive tie-breaking on exact ties.
  void set_routing_determinism_mode(bool adaptive) { adaptive_ = adaptive; }
  bool adaptive_routing() const { return adaptive_; }
  void set_determinism_config(const RouterDeterminismConfig &c) { config_ = c; }

  // filter_decision_by_policy on every decision (nullptr = no policy); adapter_ids / clusters
  // describe the adapters routed over, in order.
  void set_decision_policy(const RoutingPolicy *policy, const std::vector<std::string> &adapter_ids = {},
                           const std::vector<std::optional<std::string>> &clusters = {}) {
    if (!policy) {
      policy_pass_.clear();
      policy_max_ = -1;
      has_policy_ = false;
      return;
    }
    policy_pass_ = routing_policy_pass_bytes(*policy, adapter_ids, clusters);
    policy_max_ = policy->max_adapters_per_token ? (int)std::min<size_t>(*policy->max_adapters_per_token, 1u << 30) : -1;
    has_policy_ = true;
  }

  Decision route_with_adapter_info(const std::vector<float> &features, const std::vector<float> &priors,
                                   const std::vector<AdapterInfo> &info, const PolicyMask &mask) {
    return route_with_adapter_info_and_scope_with_ctx(features, priors, info, mask, nullptr, nullptr);
  }
  Decision route_with_adapter_info_with_ctx(const std::vector<float> &features, const std::vector<float> &priors,
                                            const std::vector<AdapterInfo> &info, const PolicyMask &mask,
                                            const det::DeterminismContext *ctx) {
    return route_with_adapter_info_and_scope_with_ctx(features, priors, info, mask, nullptr, ctx);
  }

  // One token, host priors (the reference's per-step router call); runs on the device. A decision
  // policy, when set, is applied to the result (a PolicyViolation throws).
  Decision route_with_adapter_info_and_scope_with_ctx(const std::vector<float> &features,
                                                      const std::vector<float> &priors,
                                                      const std::vector<AdapterInfo> &info, const PolicyMask &mask,
                                                      const std::string *scope_hint,
                                                      const det::DeterminismContext *ctx) {
    if (!features.empty())
      throw AosError(ErrorKind::Validation, "feature scoring is not part of this path: pass empty features");
    if (priors.size() != info.size())
      throw AosError(ErrorKind::Validation, "priors and adapter_info lengths differ");
    if (!mask.allowed.empty() && mask.allowed.size() != info.size())
      throw AosError(ErrorKind::Validation, "policy mask length differs from adapter_info");
    if (info.empty()) return Decision{};
    if (has_policy_ && policy_pass_.size() != info.size())
      throw AosError(ErrorKind::PolicyViolation, "RoutingPolicy adapter ids/clusters length mismatch");
    bind(info);
    detail::check(aoship_router_set_policy_mask(h_, mask.allowed.empty() ? nullptr : mask.allowed.data()),
                  ErrorKind::Validation, "aoship_router_set_policy_mask");
    apply_extras(info, scope_hint, ctx);
    detail::check(aoship_router_set_ring_mapping(h_, nullptr, nullptr), ErrorKind::Validation,
                  "aoship_router_set_ring_mapping");
    detail::check(aoship_router_set_decision_hashing(h_, config_.enable_decision_hashing ? d_hash_ : nullptr, 1,
                                                     nullptr, nullptr),
                  ErrorKind::Validation, "aoship_router_set_decision_hashing");
    detail::check(aoship_router_set_decision_output(h_, d_dec_, 1), ErrorKind::Validation,
                  "aoship_router_set_decision_output");
    const size_t n = info.size();
    detail::hip_check(hipMemcpy(d_priors_, priors.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
    detail::check(aoship_route(h_, d_priors_, 1, d_ring_, d_status_), ErrorKind::Routing, "aoship_route");
    aoship_ring_t ring;
    int32_t status = 0;
    uint8_t hashes[96];
    detail::hip_check(hipMemcpy(&ring, d_ring_, sizeof(ring), hipMemcpyDeviceToHost), "hipMemcpy");
    detail::hip_check(hipMemcpy(&status, d_status_, sizeof(status), hipMemcpyDeviceToHost), "hipMemcpy");
    if (config_.enable_decision_hashing)
      detail::hip_check(hipMemcpy(hashes, d_hash_, 96, hipMemcpyDeviceToHost), "hipMemcpy");
    aoship_decision_t rec;
    detail::hip_check(hipMemcpy(&rec, d_dec_, sizeof(rec), hipMemcpyDeviceToHost), "hipMemcpy");
    if (status == -1) throw AosError(ErrorKind::DeterminismViolation, "non-finite prior or score");
    if (status == -2) throw AosError(ErrorKind::PolicyViolation, "Routing policy denied all adapters for this token");
    Decision d;
    for (uint32_t i = 0; i < ring.top_k; ++i) {
      d.indices.push_back(ring.adapter_indices[i]);
      d.gates_q15.push_back(ring.gates_q15[i]);
    }
    d.entropy = rec.entropy;
    for (uint32_t i = 0; i < rec.n_candidates && i < 8; ++i)
      d.candidates.push_back(DecisionCandidate{rec.adapter_idx[i], rec.raw_score[i], rec.gate_q15[i]});
    if (config_.enable_decision_hashing && ring.top_k > 0) {
      DecisionHash h;
      h.input_hash = det::B3Hash::hex(hashes, 8);
      h.output_hash = det::B3Hash::hex(hashes + 32, 8);
      h.combined_hash = det::B3Hash::hex(hashes + 64, 8);
      h.tau = tau_clean();
      h.eps = eps_clean();
      h.k = k_ < 1 ? 1 : k_;
      d.decision_hash = h;
    }
    return d;
  }

  // decision_to_router_ring_with_active_ids_and_strengths for route_device's rings
  // (active_ids / strengths: one entry per adapter, empty = off).
  void set_ring_mapping(const std::vector<uint16_t> &active_ids, const std::vector<float> &strengths) {
    active_ids_ = active_ids;
    strengths_ = strengths;
  }

  // Batch form on device buffers: priors[T * n] -> rings[T] (status[T] may be null; -1 / -2 as
  // aoship_route), with the scope hint, determinism context, decision policy and ring mapping
  // applied; decision hashes into hashes_dev[T * 96] when it is given.
  void route_device(const std::vector<AdapterInfo> &info, const float *priors_dev, int T, aoship_ring_t *rings_dev,
                    int32_t *status_dev, const std::string *scope_hint = nullptr,
                    const det::DeterminismContext *ctx = nullptr, uint8_t *hashes_dev = nullptr) {
    if (has_policy_ && policy_pass_.size() != info.size())
      throw AosError(ErrorKind::PolicyViolation, "RoutingPolicy adapter ids/clusters length mismatch");
    if ((!active_ids_.empty() && active_ids_.size() != info.size()) ||
        (!strengths_.empty() && strengths_.size() != info.size()))
      throw AosError(ErrorKind::Routing, "Strengths / active ids length does not match active adapters");
    bind(info);
    apply_extras(info, scope_hint, ctx);
    detail::check(aoship_router_set_ring_mapping(h_, active_ids_.empty() ? nullptr : active_ids_.data(),
                                                 strengths_.empty() ? nullptr : strengths_.data()),
                  ErrorKind::Validation, "aoship_router_set_ring_mapping");
    detail::check(aoship_router_set_decision_hashing(h_, hashes_dev, T, nullptr, nullptr), ErrorKind::Validation,
                  "aoship_router_set_decision_hashing");
    detail::check(aoship_route(h_, priors_dev, T, rings_dev, status_dev), ErrorKind::Routing, "aoship_route");
  }

 private:
  void bind(const std::vector<AdapterInfo> &info) {
    std::vector<uint64_t> ids;
    for (const auto &a : info) ids.push_back(a.stable_id);
    if (h_ && ids == ids_) return;
    release();
    detail::check(aoship_init(device_), ErrorKind::Kernel, "aoship_init");
    h_ = aoship_router_new((int)ids.size(), (int)k_, tau_, eps_, bias_, ids.data());
    if (!h_) throw AosError(ErrorKind::Routing, "aoship_router_new: " + detail::last_error());
    ids_ = ids;
    detail::hip_check(hipMalloc(&d_priors_, ids.size() * sizeof(float)), "hipMalloc");
    detail::hip_check(hipMalloc(&d_ring_, sizeof(aoship_ring_t)), "hipMalloc");
    detail::hip_check(hipMalloc(&d_status_, sizeof(int32_t)), "hipMalloc");
    detail::hip_check(hipMalloc(&d_hash_, 96), "hipMalloc");
    detail::hip_check(hipMalloc(&d_dec_, sizeof(aoship_decision_t)), "hipMalloc");
    seed_.reset();
  }
  // Router::new sanitises tau and eps (router.rs:146-187); DecisionHash reports them.
  float tau_clean() const { return (std::isfinite(tau_) && tau_ > 0.0f) ? tau_ : 1.0f; }
  float eps_clean() const { return (std::isfinite(eps_) && eps_ >= 0.0f && eps_ <= 1.0f) ? eps_ : 0.02f; }
  // scope hint (router.rs:1587-1602), adaptive seed (:1606-1612, 1705-1724), decision policy
  void apply_extras(const std::vector<AdapterInfo> &info, const std::string *scope_hint,
                    const det::DeterminismContext *ctx) {
    std::vector<uint8_t> in_scope;
    if (scope_hint) {
      bool matched = false;
      for (const auto &a : info) {
        const bool m = a.scope_path && *a.scope_path == *scope_hint;
        in_scope.push_back(m ? 1 : 0);
        matched = matched || m;
      }
      if (!matched) in_scope.clear();
    }
    detail::check(aoship_router_set_scope(h_, in_scope.empty() ? nullptr : in_scope.data()), ErrorKind::Validation,
                  "aoship_router_set_scope");
    if (adaptive_ && !ctx)
      throw AosError(ErrorKind::Config,
                     "Adaptive routing configuration error: determinism context is required for seeded "
                     "tie-breaking when adaptive routing is enabled. Provide a determinism context in the "
                     "request or disable adaptive routing.");
    std::optional<det::Bytes32> seed;
    if (adaptive_) seed = ctx->router_tiebreak_seed();
    if (seed != seed_) {
      detail::check(aoship_router_set_adaptive_seed(h_, seed ? seed->data() : nullptr), ErrorKind::Validation,
                    "aoship_router_set_adaptive_seed");
      seed_ = seed;
    }
    detail::check(aoship_router_set_decision_policy(h_, has_policy_ ? policy_pass_.data() : nullptr, policy_max_),
                  ErrorKind::Validation, "aoship_router_set_decision_policy");
  }
  void release() {
    if (h_) aoship_router_free(h_);
    h_ = nullptr;
    if (d_priors_) (void)hipFree(d_priors_);
    if (d_ring_) (void)hipFree(d_ring_);
    if (d_status_) (void)hipFree(d_status_);
    if (d_hash_) (void)hipFree(d_hash_);
    d_hash_ = nullptr;
    if (d_dec_) (void)hipFree(d_dec_);
    d_dec_ = nullptr;
    d_priors_ = nullptr;
    d_ring_ = nullptr;
    d_status_ = nullptr;
    ids_.clear();
  }

  size_t k_;
  float tau_, eps_, bias_ = 1.0f;
  int device_;
  aoship_router_t *h_ = nullptr;

 public:
  // The C-ABI router behind this object (for HipKernels::route_mlp_forward).
  aoship_router_t *handle() const { return h_; }

 private:
  std::vector<uint64_t> ids_;
  float *d_priors_ = nullptr;
  aoship_ring_t *d_ring_ = nullptr;
  int32_t *d_status_ = nullptr;
  uint8_t *d_hash_ = nullptr;
  aoship_decision_t *d_dec_ = nullptr;
  bool adaptive_ = false;
  RouterDeterminismConfig config_;
  std::optional<det::Bytes32> seed_;
  bool has_policy_ = false;
  std::vector<uint8_t> policy_pass_;
  int policy_max_ = -1;
  std::vector<uint16_t> active_ids_;
  std::vector<float> strengths_;
};

// ---- FusedKernels surface for the layer path -----------------------------------------------------

struct AdapterLoadMetadata {
  std::string adapter_id;
  uint32_t rank = 0;
  float alpha = 0.0f;
  std::vector<std::string> target_modules;
};

// One module's LoRA weights in MLX shapes: A [rank, in], B [out, rank], float32.
struct LoraModuleWeights {
  int in_features = 0, out_features = 0;
  std::vector<float> A, B;
};

// Per layer: module name -> weights.
using LoraLayerWeights = std::map<std::string, LoraModuleWeights>;

class HipKernels {
 public:
  // device ordinal; num_layers layer handles (layer_idx 0..num_layers-1).
  HipKernels(int device, int num_layers) {
    detail::check(aoship_init(device), ErrorKind::Kernel, "aoship_init");
    for (int i = 0; i < num_layers; ++i) {
      aoship_layer_t *l = aoship_layer_new(i, AOSHIP_GROUP_SIZE, AOSHIP_BITS);
      if (!l) throw AosError(ErrorKind::Kernel, "aoship_layer_new: " + detail::last_error());
      layers_.push_back(l);
    }
    char buf[256];
    detail::check(aoship_device_name(buf, sizeof(buf)), ErrorKind::Kernel, "aoship_device_name");
    device_name_ = buf;
  }
  ~HipKernels() {
    for (auto *l : layers_) aoship_layer_free(l);
    for (auto &kv : adapters_) aoship_lora_adapter_free(kv.second);
  }
  HipKernels(const HipKernels &) = delete;
  HipKernels &operator=(const HipKernels &) = delete;

  // FusedKernels::device_name (lib.rs:374)
  const std::string &device_name() const { return device_name_; }

  // FusedKernels::attest_determinism (lib.rs:383): the report as JSON text.
  std::string attest_determinism() const {
    const int n = aoship_attest_determinism(nullptr, 0);
    std::string s((size_t)n + 1, '\0');
    aoship_attest_determinism(&s[0], n + 1);
    s.resize((size_t)n);
    return s;
  }

  // Base projection of a layer in the MLX 4-bit layout.
  void set_base(int layer, const std::string &module, int out_features, int in_features, const uint32_t *packed,
                const uint16_t *scales_f16, const uint16_t *biases_f16) {
    detail::check(aoship_layer_set_base(layer_at(layer), module.c_str(), out_features, in_features, packed,
                                        scales_f16, biases_f16),
                  ErrorKind::Kernel, "aoship_layer_set_base");
  }

  // FusedKernels::load_adapter_with_metadata (lib.rs:398-405): scale = alpha / rank
  // (backend.rs:462); weights[layer][module]. The adapter is attached to every layer.
  void load_adapter_with_metadata(uint16_t id, const std::vector<LoraLayerWeights> &weights,
                                  const AdapterLoadMetadata &md) {
    if (md.rank == 0) throw AosError(ErrorKind::Validation, "adapter rank must be positive");
    if (adapters_.count(id)) unload_adapter(id);
    const float scale = md.alpha / (float)md.rank;
    aoship_lora_adapter_t *a = aoship_lora_adapter_new(id, (int)weights.size(), scale);
    if (!a) throw AosError(ErrorKind::Kernel, "aoship_lora_adapter_new: " + detail::last_error());
    for (size_t li = 0; li < weights.size(); ++li)
      for (const auto &kv : weights[li]) {
        if (!md.target_modules.empty()) {
          bool wanted = false;
          for (const auto &t : md.target_modules) wanted = wanted || t == kv.first;
          if (!wanted) continue;
        }
        const LoraModuleWeights &w = kv.second;
        if (aoship_lora_adapter_set_module(a, (int)li, kv.first.c_str(), (int)md.rank, w.in_features,
                                           w.out_features, w.A.data(), w.B.data()) != 0) {
          const std::string err = detail::last_error();
          aoship_lora_adapter_free(a);
          throw AosError(ErrorKind::Kernel, "aoship_lora_adapter_set_module: " + err);
        }
      }
    install(id, a);
  }

  // MLXFFIBackend::load_adapter (backend.rs:891-893): safetensors bytes, no metadata.
  void load_adapter(uint16_t id, const uint8_t *bytes, size_t len) {
    load_adapter_with_metadata(id, bytes, len, nullptr);
  }

  // MLXFFIBackend::load_adapter_with_metadata (backend.rs:1017-1110): safetensors bytes and the
  // metadata object as JSON text (null or empty: none). scale = alpha / rank of the resolved
  // config; each module keeps the rank of its A tensor and is set on every layer. A module the
  // device path rejects (a name outside q/k/v/o/gate/up/down_proj, rank > 128, in % 64 or
  // out % 32 not 0, B columns != A rows) is skipped with a warning, as add_adapter_internal skips a failed set_module
  // (backend.rs:496-522); load_warnings() lists them. Returns the resolved config.
  ingest::AdapterSpec load_adapter_with_metadata(uint16_t id, const uint8_t *bytes, size_t len,
                                                 const char *metadata_json) {
    ingest::AdapterSpec spec;
    try {
      const ingest::SafeTensors st = ingest::SafeTensors::parse(bytes, len);
      ingest::Json md;
      const bool has_md = metadata_json && *metadata_json;
      if (has_md) md = ingest::parse_json(metadata_json);
      spec = ingest::read_adapter(st, has_md ? &md : nullptr);
    } catch (const ingest::IngestError &e) {
      throw AosError(kind_of(e), std::string("Failed to parse adapter weights: ") + e.what());
    }
    register_adapter(id, spec);
    return spec;
  }

  // MLXFFIBackend::register_adapter (backend.rs:549-551, 448-522) for an adapter read by
  // ingest::read_adapter or ingest::load_lora (LoRAAdapter::load, lora.rs:154-216): replaces id,
  // attaches it, sets each module on every layer, skipping (with a warning) what the device path
  // rejects.
  void register_adapter(uint16_t id, const ingest::AdapterSpec &spec) {
    if (spec.rank == 0) throw AosError(ErrorKind::Validation, "adapter rank must be positive");
    warnings_.clear();
    if (adapters_.count(id)) unload_adapter(id);
    aoship_lora_adapter_t *a = aoship_lora_adapter_new(id, (int)layers_.size(), spec.scale());
    if (!a) throw AosError(ErrorKind::Kernel, "aoship_lora_adapter_new: " + detail::last_error());
    for (const auto &m : spec.modules) {
      if (!m.problem.empty()) {
        warnings_.push_back("module " + m.name + " skipped: " + m.problem);
        continue;
      }
      for (size_t li = 0; li < layers_.size(); ++li)
        if (aoship_lora_adapter_set_module(a, (int)li, m.name.c_str(), m.rank, m.in_features, m.out_features,
                                           m.A.data(), m.B.data()) != 0) {
          warnings_.push_back("module " + m.name + " skipped: " + detail::last_error());
          break;  // the same weights go to every layer, so every layer would fail alike
        }
    }
    install(id, a);
  }

  // Messages for the modules the last safetensors load skipped.
  const std::vector<std::string> &load_warnings() const { return warnings_; }

  // Base projections from an MLX-community 4-bit safetensors file, or one shard of it: per layer
  // i < num_layers, "model.layers.<i>.self_attn.{q,k,v,o}_proj" and
  // "model.layers.<i>.mlp.{gate,up,down}_proj" (.weight / .scales / .biases, read as
  // get_weight_with_dequant reads them). Keys the file does not hold are left unset, so shards
  // load one after another. Returns the number of projections set.
  int load_base_safetensors(const uint8_t *bytes, size_t len) {
    static const char *const kAttn[] = {"q_proj", "k_proj", "v_proj", "o_proj"};
    static const char *const kMlp[] = {"gate_proj", "up_proj", "down_proj"};
    int n = 0;
    try {
      const ingest::SafeTensors st = ingest::SafeTensors::parse(bytes, len);
      for (size_t li = 0; li < layers_.size(); ++li) {
        const std::string prefix = "model.layers." + std::to_string(li);
        auto one = [&](const std::string &group, const char *module) {
          ingest::BaseProjection bp;
          if (!ingest::read_base(st, prefix + group + module, bp)) return;
          set_base((int)li, module, bp.out_features, bp.in_features, bp.packed.data(), bp.scales_f16.data(),
                   bp.biases_f16.data());
          ++n;
        };
        for (const char *m : kAttn) one(".self_attn.", m);
        for (const char *m : kMlp) one(".mlp.", m);
      }
    } catch (const ingest::IngestError &e) {
      throw AosError(kind_of(e), e.what());
    }
    return n;
  }
  int load_base_safetensors(const std::string &path) {
    try {
      const ingest::MappedFile f(path);
      return load_base_safetensors(f.data(), f.size());
    } catch (const ingest::IngestError &e) {
      throw AosError(kind_of(e), e.what());
    }
  }

  // attach / detach / unload (lib.rs:410-432). A detached adapter stays loaded; its ring index
  // then contributes nothing until it is attached again.
  void attach_adapter(uint16_t id) {
    if (!adapters_.count(id)) throw AosError(ErrorKind::Kernel, "adapter not loaded");
    attached_[id] = true;
    rebind();
  }
  void detach_adapter(uint16_t id) {
    if (!adapters_.count(id)) throw AosError(ErrorKind::Kernel, "adapter not loaded");
    attached_.erase(id);
    rebind();
  }
  void unload_adapter(uint16_t id) {
    auto it = adapters_.find(id);
    if (it == adapters_.end()) throw AosError(ErrorKind::Kernel, "adapter not loaded");
    attached_.erase(id);
    aoship_lora_adapter_t *a = it->second;
    adapters_.erase(it);
    rebind();  // layers drop their reference first
    aoship_lora_adapter_free(a);
  }

  // Ring index a selects adapter id a.
  size_t adapter_table_len() const { return table_len_; }

  void reserve(int max_tokens) {
    for (auto *l : layers_) detail::check(aoship_layer_reserve(l, max_tokens), ErrorKind::Kernel, "aoship_layer_reserve");
  }

  // Layer forwards on device buffers (bf16 activations, one 40-byte ring per token).
  void mlp_forward(int layer, const aoship_bf16_t *x, int T, const aoship_ring_t *rings, aoship_bf16_t *y) {
    detail::check(aoship_mlp_forward(layer_at(layer), x, T, rings, y), ErrorKind::Kernel, "aoship_mlp_forward");
  }
  void proj_forward(int layer, const std::string &module, const aoship_bf16_t *x, int T, const aoship_ring_t *rings,
                    aoship_bf16_t *y) {
    detail::check(aoship_proj_forward(layer_at(layer), module.c_str(), x, T, rings, y), ErrorKind::Kernel,
                  "aoship_proj_forward");
  }
  void qkv_forward(int layer, const aoship_bf16_t *x, int T, const aoship_ring_t *rings, aoship_bf16_t *q,
                   aoship_bf16_t *k, aoship_bf16_t *v) {
    detail::check(aoship_qkv_forward(layer_at(layer), x, T, rings, q, k, v), ErrorKind::Kernel,
                  "aoship_qkv_forward");
  }
  // Route T tokens from device features (float32 [T][d]) and run the layer's MLP on them in one
  // call; rings and status (may be null) receive the decisions (aoship_route_mlp_forward).
  void route_mlp_forward(const Router &router, const float *features, const float *router_w, int d, int layer,
                         const aoship_bf16_t *x, int T, aoship_ring_t *rings, int32_t *status, aoship_bf16_t *y) {
    detail::check(aoship_route_mlp_forward(router.handle(), features, router_w, d, layer_at(layer), x, T, rings,
                                           status, y),
                  ErrorKind::Kernel, "aoship_route_mlp_forward");
  }
  // True if a fused decode launch of the layer gave up a bounded wait since the last call
  // (aoship_layer_wait_timeouts); clears the flag.
  bool wait_timed_out(int layer) {
    const int r = aoship_layer_wait_timeouts(layer_at(layer));
    detail::check(r < 0 ? -1 : 0, ErrorKind::Kernel, "aoship_layer_wait_timeouts");
    return r == 1;
  }

 private:
  aoship_layer_t *layer_at(int i) {
    if (i < 0 || i >= (int)layers_.size()) throw AosError(ErrorKind::Validation, "layer index out of range");
    return layers_[(size_t)i];
  }
  static ErrorKind kind_of(const ingest::IngestError &e) {
    switch (e.kind()) {
      case ingest::IngestError::Kind::Parse: return ErrorKind::Parse;
      case ingest::IngestError::Kind::Io: return ErrorKind::Io;
      default: return ErrorKind::Validation;
    }
  }
  void install(uint16_t id, aoship_lora_adapter_t *a) {
    adapters_[id] = a;
    attached_[id] = true;
    rebind();
  }
  // Table: position = adapter id; detached or unloaded ids are null (skipped like a missing
  // handle in prepare_lora_for_ring, backend.rs:398-428).
  void rebind() {
    size_t n = 0;
    for (const auto &kv : adapters_) n = (size_t)kv.first + 1 > n ? (size_t)kv.first + 1 : n;
    std::vector<aoship_lora_adapter_t *> table(n, nullptr);
    for (const auto &kv : adapters_)
      if (attached_.count(kv.first)) table[kv.first] = kv.second;
    for (auto *l : layers_)
      detail::check(aoship_layer_set_adapters(l, table.data(), (int)table.size()), ErrorKind::Kernel,
                    "aoship_layer_set_adapters");
    table_len_ = n;
  }

  std::vector<aoship_layer_t *> layers_;
  std::map<uint16_t, aoship_lora_adapter_t *> adapters_;
  std::map<uint16_t, bool> attached_;
  size_t table_len_ = 0;
  std::string device_name_;
  std::vector<std::string> warnings_;
};

}  // namespace adapteros
