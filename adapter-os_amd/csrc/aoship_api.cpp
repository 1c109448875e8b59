/*
 * aoship_api.cpp — the C ABI declared in include/aoship.h: handles, weight upload, adapter tables,
 * workspaces and the launch sequence of each forward.
 *
 * Conventions follow the reference's MLX FFI (crates/adapteros-lora-mlx-ffi/wrapper.h,
 * src/mlx_cpp_wrapper_real.cpp): NULL from constructors and -1 from other calls on error, with a
 * thread-local message (mlx_cpp_wrapper_real.cpp:27,1682-1684); weights are copied on upload
 * (mlx_cpp_wrapper_real.cpp:3198-3199).
 */
#include <hip/hip_runtime.h>
#include <hip/hip_version.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "aos_blake3.h"
#include "aos_exp.h"
#include "aoship_internal.h"

/* ------------------------------------------------------------------------------------------ */
/* errors                                                                                     */
/* ------------------------------------------------------------------------------------------ */

static thread_local std::string g_last_error;

static int set_err(const std::string &s) {
  g_last_error = s;
  return -1;
}

#define HIP_OR_FAIL(expr, what)                                                        \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess) return set_err(std::string(what) + ": " + hipGetErrorString(e_)); \
  } while (0)

extern "C" const char *aoship_get_last_error(void) { return g_last_error.c_str(); }
extern "C" void aoship_clear_error(void) { g_last_error.clear(); }
extern "C" const char *aoship_version(void) { return "aoship 0.1.0 gfx950"; }

/* Host build of the router's float64 exp, exported for its pinning test (not part of the ABI). */
extern "C" double aoship_internal_exp_cr(double x) { return aos_exp_cr(x); }

static int g_device = -1;

/* ---- the allocation-free decode forward's scratch ----
 * One static device array (each GPU holds its own copy, at its own address, until the process
 * ends): arrival counters (zero at rest), generation-stamped ready flags (zero at first use),
 * then the workspace. Host code never uses the array's name as an address: at set-up, with the
 * device current, hipGetSymbolAddress gives this device's copy, kept per device. */
#define AOS_SCRATCH_BYTES ((size_t)32 << 20)
#define AOS_SCRATCH_CTR_BYTES ((size_t)256 << 10)
#define AOS_SCRATCH_FLAG_BYTES ((size_t)4 << 20)
#define AOS_SCRATCH_WS_BYTES (AOS_SCRATCH_BYTES - AOS_SCRATCH_CTR_BYTES - AOS_SCRATCH_FLAG_BYTES)
#define AOS_MAX_DEVICES 64
static __device__ __align__(256) unsigned char scratch[AOS_SCRATCH_BYTES];

struct ScratchDev {
  unsigned char *ptr = nullptr; /* this device's copy of scratch */
  uint32_t gen = 0;             /* generation of its flags */
};
static ScratchDev g_scratch[AOS_MAX_DEVICES];
static std::mutex g_scratch_mu;

/* Once per device, with that device current: look up its copy of the array and clear the counter
 * and flag regions (the workspace needs no initial contents). */
static int scratch_setup(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (dev < 0 || dev >= AOS_MAX_DEVICES) return set_err("scratch: device index out of range");
  if (g_scratch[dev].ptr) return 0;
  void *p = nullptr;
  HIP_OR_FAIL(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  HIP_OR_FAIL(hipMemset(p, 0, AOS_SCRATCH_CTR_BYTES + AOS_SCRATCH_FLAG_BYTES), "hipMemset(scratch)");
  HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  g_scratch[dev].ptr = (unsigned char *)p;
  g_scratch[dev].gen = 0;
  return 0;
}

static int ensure_device() {
  if (g_device < 0) return set_err("aoship_init() has not been called");
  HIP_OR_FAIL(hipSetDevice(g_device), "hipSetDevice");
  return 0;
}

extern "C" int aoship_init(int device) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) return set_err("no HIP device available");
  if (device < 0 || device >= count) return set_err("device index out of range");
  HIP_OR_FAIL(hipSetDevice(device), "hipSetDevice");
  g_device = device;
  /* the allocation-free forward's scratch; a failure here is reported again by that forward,
   * which retries the set-up on its first call */
  const std::string keep = g_last_error;
  if (scratch_setup(device)) g_last_error = keep;
  return 0;
}

extern "C" int aoship_device_name(char *buf, int len) {
  if (!buf || len <= 0) return set_err("aoship_device_name: null buffer");
  if (ensure_device()) return -1;
  hipDeviceProp_t prop;
  HIP_OR_FAIL(hipGetDeviceProperties(&prop, g_device), "hipGetDeviceProperties");
  snprintf(buf, (size_t)len, "%s (%s)", prop.name, prop.gcnArchName);
  return 0;
}

extern "C" int aoship_sync(void) {
  if (ensure_device()) return -1;
  HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return 0;
}

/* The report in DeterminismReport's serialized form (attestation.rs:130-160): backend "Hip"
 * (deterministic by design: fixed-order reductions, no floating-point atomics, no random draws on
 * the device; adaptive tie-breaks come from the HKDF-seeded ChaCha20 stream on the host), the
 * flags every kernel is built with, and this library's parity levels as extra fields. */
extern "C" int aoship_attest_determinism(char *buf, int len) {
  char js[1024];
  const int n = snprintf(
      js, sizeof(js),
      "{\"backend_type\":\"Hip\",\"metallib_hash\":null,\"metallib_verified\":false,\"manifest\":null,"
      "\"rng_seed_method\":\"HkdfSeeded\",\"floating_point_mode\":\"Deterministic\","
      "\"determinism_level\":\"bit_exact\","
      "\"compiler_flags\":[\"-O3\",\"--offload-arch=gfx950\",\"-ffp-contract=off\",\"-fno-fast-math\","
      "\"-fno-gpu-flush-denormals-to-zero\",\"-fhip-fp32-correctly-rounded-divide-sqrt\"],"
      "\"deterministic\":true,\"runtime_version\":\"HIP %d.%d.%d\",\"device_id\":\"gfx950\","
      "\"reductions\":\"fixed order; no floating-point atomics\","
      "\"router\":\"bit_exact vs the CPU restatement (float64 softmax with correctly rounded exp)\","
      "\"layer\":\"bit_exact run to run; bounded_tolerance vs the CPU restatement (2e-2 relative, bf16)\"}",
      HIP_VERSION_MAJOR, HIP_VERSION_MINOR, HIP_VERSION_PATCH);
  if (buf && len > 0) snprintf(buf, (size_t)len, "%s", js);
  return n;
}

/* ------------------------------------------------------------------------------------------ */
/* small helpers                                                                              */
/* ------------------------------------------------------------------------------------------ */

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static int module_index(const char *name) {
  static const char *names[AOS_MAX_MODULES] = {"q_proj",    "k_proj",  "v_proj",   "o_proj",
                                               "gate_proj", "up_proj", "down_proj"};
  if (!name) return -1;
  for (int i = 0; i < AOS_MAX_MODULES; ++i)
    if (strcmp(name, names[i]) == 0) return i;
  return -1;
}

struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  DevBuf(DevBuf &&o) noexcept : p(o.p), bytes(o.bytes) {
    o.p = nullptr;
    o.bytes = 0;
  }
  DevBuf &operator=(DevBuf &&o) noexcept {
    if (this != &o) {
      release();
      p = o.p;
      bytes = o.bytes;
      o.p = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  int alloc(size_t n, bool zero) {
    release();
    if (n == 0) n = 256;
    HIP_OR_FAIL(hipMalloc(&p, n), "hipMalloc");
    bytes = n;
    if (zero) HIP_OR_FAIL(hipMemset(p, 0, n), "hipMemset");
    return 0;
  }
  int upload(const void *src, size_t n) {
    if (alloc(n, false)) return -1;
    HIP_OR_FAIL(hipMemcpy(p, src, n, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return 0;
  }
  template <class T>
  T *as() const {
    return (T *)p;
  }
};

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

/* ------------------------------------------------------------------------------------------ */
/* router                                                                                     */
/* ------------------------------------------------------------------------------------------ */

struct aoship_router {
  int n = 0, k = 1;
  float tau = 1.0f, eps = 0.02f, bias = 1.0f;
  DevBuf stable_id, allowed;
  bool has_mask = false;
  std::vector<uint64_t> h_stable_id;
  /* extras: each buffer is released when its feature is off */
  DevBuf scope, tie_key, post_allowed, active_ids, strengths;
  int post_max = -1;
  uint8_t *hashes = nullptr; /* caller's device buffer, [hash_max_tokens][96] */
  int hash_max_tokens = 0;
  DevBuf hash_extra;         /* reasoning hash words 0-7, backend identity hash words 8-15 */
  int hash_reasoning = 0, hash_backend = 0;
  aoship_decision_t *decisions = nullptr; /* caller's device buffer, [dec_max_tokens] */
  int dec_max_tokens = 0;
  hipStream_t stream = nullptr;
};

/* ChaCha20 block (RFC 8439 section 2.3: 20 rounds, output = rounds(state) + state) over the state
 * layout of rand_chacha 0.3: "expand 32-byte k", the 32-byte key, a 64-bit block counter in words
 * 12-13 and a 64-bit stream id in words 14-15. */
static void chacha20_block(const uint32_t key[8], uint64_t counter, uint64_t stream, uint32_t out[16]) {
  uint32_t st[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, key[0], key[1], key[2], key[3],
                     key[4],      key[5],      key[6],      key[7],      (uint32_t)counter,
                     (uint32_t)(counter >> 32), (uint32_t)stream, (uint32_t)(stream >> 32)};
  uint32_t x[16];
  memcpy(x, st, sizeof x);
  auto rotl = [](uint32_t v, int c) { return (v << c) | (v >> (32 - c)); };
  auto qr = [&](int a, int b, int c, int d) {
    x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 16);
    x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 12);
    x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 8);
    x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 7);
  };
  for (int i = 0; i < 10; ++i) {
    qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);
    qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + st[i];
}

/* ChaCha20Rng::from_seed(seed) then n x gen::<u64>(): next_u64 joins consecutive keystream words
 * low word first (rand_core BlockRng), the stream starting at block 0 of stream 0. */
extern "C" int aoship_adaptive_tie_breakers(const uint8_t *seed, int n, uint64_t *out) {
  if (!seed || !out || n < 0) return set_err("aoship_adaptive_tie_breakers: bad arguments");
  uint32_t key[8];
  for (int i = 0; i < 8; ++i)
    key[i] = (uint32_t)seed[4 * i] | ((uint32_t)seed[4 * i + 1] << 8) | ((uint32_t)seed[4 * i + 2] << 16) |
             ((uint32_t)seed[4 * i + 3] << 24);
  uint32_t blk[16];
  for (int a = 0; a < n; ++a) {
    if ((a & 7) == 0) chacha20_block(key, (uint64_t)(a >> 3), 0, blk);
    const int w = 2 * (a & 7);
    out[a] = (uint64_t)blk[w] | ((uint64_t)blk[w + 1] << 32);
  }
  return 0;
}

extern "C" int aoship_blake3(const void *data, size_t len, uint8_t *out) {
  if ((!data && len) || !out) return set_err("aoship_blake3: null argument");
  const uint8_t *bytes = (const uint8_t *)data;
  auto word = [&](size_t j) {
    uint32_t v = 0;
    for (int b = 0; b < 4; ++b)
      if (4 * j + (size_t)b < len) v |= (uint32_t)bytes[4 * j + (size_t)b] << (8 * b);
    return v;
  };
  const int n = aos_b3_nchunks(len);
  uint32_t h[8];
  if (n == 1) {
    aos_b3_chunk(word, len, 0, true, h);
  } else {
    std::vector<uint32_t> cvs((size_t)n * 8);
    uint32_t(*cv)[8] = (uint32_t(*)[8])cvs.data();
    for (int c = 0; c < n; ++c) aos_b3_chunk(word, len, (uint64_t)c, false, cv[c]);
    aos_b3_merge(cv, n, h);
  }
  for (int i = 0; i < 32; ++i) out[i] = (uint8_t)(h[i / 4] >> (8 * (i % 4)));
  return 0;
}

static int upload_or_release(DevBuf &b, const void *src, size_t bytes) {
  if (!src) {
    b.release();
    return 0;
  }
  return b.upload(src, bytes);
}

extern "C" aoship_router_t *aoship_router_new(int n_adapters, int k, float tau, float eps,
                                              float routing_bias, const uint64_t *stable_ids) {
  if (n_adapters < 1 || n_adapters > AOS_MAX_ADAPTERS) {
    set_err("aoship_router_new: n_adapters must be in [1, 4096]");
    return nullptr;
  }
  /* Router::new (router.rs:769-777) rejects k > MAX_K. */
  if (k > AOSHIP_MAX_K) {
    set_err("Adapter routing failed: K exceeds maximum allowed value of 8");
    return nullptr;
  }
  if (ensure_device()) return nullptr;
  auto *r = new aoship_router();
  r->n = n_adapters;
  r->k = k < 1 ? 1 : k; /* sanitize_k (router.rs:127-142) */
  r->tau = (std::isfinite(tau) && tau > 0.0f) ? tau : 1.0f;                 /* :171-187 */
  r->eps = (std::isfinite(eps) && eps >= 0.0f && eps <= 1.0f) ? eps : 0.02f; /* :146-166 */
  r->bias = (std::isfinite(routing_bias) && routing_bias > 0.0f) ? routing_bias : 1.0f;
  std::vector<uint64_t> ids((size_t)n_adapters, 0ull);
  if (stable_ids) memcpy(ids.data(), stable_ids, sizeof(uint64_t) * (size_t)n_adapters);
  if (r->stable_id.upload(ids.data(), ids.size() * sizeof(uint64_t))) {
    delete r;
    return nullptr;
  }
  r->h_stable_id = ids;
  return r;
}

extern "C" int aoship_router_set_scope(aoship_router_t *r, const uint8_t *in_scope) {
  if (!r) return set_err("aoship_router_set_scope: null router");
  if (ensure_device()) return -1;
  return upload_or_release(r->scope, in_scope, (size_t)r->n);
}

extern "C" int aoship_router_set_adaptive_seed(aoship_router_t *r, const uint8_t *seed) {
  if (!r) return set_err("aoship_router_set_adaptive_seed: null router");
  if (ensure_device()) return -1;
  if (!seed) {
    r->tie_key.release();
    return 0;
  }
  /* The rank of each adapter in (breaker, stable_id, index) order: equal scores compare by it
   * exactly as sort_scores_adaptive compares them, and it fits the device's 64-bit key field. */
  const int n = r->n;
  std::vector<uint64_t> brk((size_t)n), rank((size_t)n);
  std::vector<int> order((size_t)n);
  aoship_adaptive_tie_breakers(seed, n, brk.data());
  for (int i = 0; i < n; ++i) order[(size_t)i] = i;
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    if (brk[(size_t)a] != brk[(size_t)b]) return brk[(size_t)a] < brk[(size_t)b];
    if (r->h_stable_id[(size_t)a] != r->h_stable_id[(size_t)b])
      return r->h_stable_id[(size_t)a] < r->h_stable_id[(size_t)b];
    return a < b;
  });
  for (int pos = 0; pos < n; ++pos) rank[(size_t)order[(size_t)pos]] = (uint64_t)pos;
  return r->tie_key.upload(rank.data(), rank.size() * sizeof(uint64_t));
}

extern "C" int aoship_router_set_decision_policy(aoship_router_t *r, const uint8_t *allowed,
                                                 int max_adapters_per_token) {
  if (!r) return set_err("aoship_router_set_decision_policy: null router");
  if (ensure_device()) return -1;
  r->post_max = max_adapters_per_token < 0 ? -1 : max_adapters_per_token;
  return upload_or_release(r->post_allowed, allowed, (size_t)r->n);
}

extern "C" int aoship_router_set_decision_hashing(aoship_router_t *r, uint8_t *hashes, int max_tokens,
                                                  const uint8_t *reasoning_hash,
                                                  const uint8_t *backend_identity_hash) {
  if (!r) return set_err("aoship_router_set_decision_hashing: null router");
  if (hashes && max_tokens < 1) return set_err("aoship_router_set_decision_hashing: max_tokens must be >= 1");
  if (ensure_device()) return -1;
  uint8_t extra[64] = {0};
  if (reasoning_hash) memcpy(extra, reasoning_hash, 32);
  if (backend_identity_hash) memcpy(extra + 32, backend_identity_hash, 32);
  if (hashes && r->hash_extra.upload(extra, sizeof extra)) return -1;
  r->hashes = hashes;
  r->hash_max_tokens = hashes ? max_tokens : 0;
  r->hash_reasoning = reasoning_hash ? 1 : 0;
  r->hash_backend = backend_identity_hash ? 1 : 0;
  return 0;
}

extern "C" int aoship_router_set_decision_output(aoship_router_t *r, aoship_decision_t *decisions, int max_tokens) {
  if (!r) return set_err("aoship_router_set_decision_output: null router");
  if (decisions && max_tokens < 1) return set_err("aoship_router_set_decision_output: max_tokens must be >= 1");
  r->decisions = decisions;
  r->dec_max_tokens = decisions ? max_tokens : 0;
  return 0;
}

extern "C" int aoship_router_set_ring_mapping(aoship_router_t *r, const uint16_t *active_ids,
                                              const float *strengths) {
  if (!r) return set_err("aoship_router_set_ring_mapping: null router");
  if (ensure_device()) return -1;
  if (upload_or_release(r->active_ids, active_ids, (size_t)r->n * sizeof(uint16_t))) return -1;
  return upload_or_release(r->strengths, strengths, (size_t)r->n * sizeof(float));
}

extern "C" int aoship_router_set_policy_mask(aoship_router_t *r, const uint8_t *allowed) {
  if (!r) return set_err("aoship_router_set_policy_mask: null router");
  if (ensure_device()) return -1;
  if (!allowed) {
    r->has_mask = false;
    r->allowed.release();
    return 0;
  }
  if (r->allowed.upload(allowed, (size_t)r->n)) return -1;
  r->has_mask = true;
  return 0;
}

extern "C" int aoship_router_set_stream(aoship_router_t *r, void *stream) {
  if (!r) return set_err("aoship_router_set_stream: null router");
  r->stream = (hipStream_t)stream;
  return 0;
}

extern "C" void aoship_router_free(aoship_router_t *r) { delete r; }

/* The launch parameters of a routing call (T >= 1), validated. */
static int route_fill(aoship_router_t *r, const float *features, const float *router_w, int d,
                      const float *priors_in, int T, aoship_ring_t *rings, float *priors_out, int32_t *status,
                      aos_route_params &p) {
  memset(&p, 0, sizeof(p));
  p.n = r->n;
  p.d = d;
  p.T = T;
  p.k = r->k;
  p.tau = r->tau;
  p.eps = r->eps;
  p.bias = r->bias;
  p.stable_id = r->stable_id.as<uint64_t>();
  p.allowed = r->has_mask ? r->allowed.as<uint8_t>() : nullptr;
  p.rings = rings;
  p.status = status;
  p.priors_in = priors_in;
  p.scope = r->scope.p ? r->scope.as<uint8_t>() : nullptr;
  p.tie_key = r->tie_key.p ? r->tie_key.as<uint64_t>() : nullptr;
  p.post_allowed = r->post_allowed.p ? r->post_allowed.as<uint8_t>() : nullptr;
  p.post_max = r->post_max;
  p.active_ids = r->active_ids.p ? r->active_ids.as<uint16_t>() : nullptr;
  p.strengths = r->strengths.p ? r->strengths.as<float>() : nullptr;
  if (r->hashes) {
    if (T > r->hash_max_tokens)
      return set_err("aoship_route: T exceeds the decision-hash buffer (" + std::to_string(r->hash_max_tokens) +
                     " tokens)");
    p.hashes = r->hashes;
    p.hash_extra = r->hash_extra.as<uint32_t>();
    p.hash_reasoning = r->hash_reasoning;
    p.hash_backend = r->hash_backend;
  }
  if (r->decisions) {
    if (T > r->dec_max_tokens)
      return set_err("aoship_route: T exceeds the decision-output buffer (" + std::to_string(r->dec_max_tokens) +
                     " tokens)");
    p.decisions = r->decisions;
  }
  if (features) {
    if (!router_w || d <= 0 || d % 4 != 0)
      return set_err("aoship_route_features: router weights missing or d not a multiple of 4");
    if ((size_t)(d + r->n) * sizeof(float) > 60 * 1024)
      return set_err("aoship_route_features: d + n_adapters must not exceed 15360");
    if (((uintptr_t)features & 15u) || ((uintptr_t)router_w & 15u))
      return set_err("aoship_route_features: features and router_w must be 16-byte aligned");
    p.features = features;
    p.router_w = router_w;
    p.priors_out = priors_out; /* optional: the kernel hands the priors over in LDS */
  } else if (!priors_in) {
    return set_err("aoship_route: null priors");
  }
  return 0;
}

static int route_common(aoship_router_t *r, const float *features, const float *router_w, int d,
                        const float *priors_in, int T, aoship_ring_t *rings, float *priors_out,
                        int32_t *status, hipStream_t stream) {
  if (!r) return set_err("aoship_route: null router");
  if (T < 0 || T > (1 << 22)) return set_err("aoship_route: T out of range");
  if (T == 0) return 0;
  if (!rings) return set_err("aoship_route: null rings");
  if (ensure_device()) return -1;
  aos_route_params p;
  if (route_fill(r, features, router_w, d, priors_in, T, rings, priors_out, status, p)) return -1;
  aos_launch_ctx ctx = {stream, nullptr, nullptr};
  int e = aos_launch_route(&p, &ctx);
  if (e != 0) return set_err(std::string("route launch: ") + hipGetErrorString((hipError_t)e));
  return 0;
}

extern "C" int aoship_route(aoship_router_t *r, const float *priors, int T, aoship_ring_t *rings,
                            int32_t *status) {
  return route_common(r, nullptr, nullptr, 0, priors, T, rings, nullptr, status, r ? r->stream : nullptr);
}

extern "C" int aoship_route_features(aoship_router_t *r, const float *features,
                                     const float *router_w, int d, int T, aoship_ring_t *rings,
                                     float *priors_out, int32_t *status) {
  if (!features) return set_err("aoship_route_features: null features");
  return route_common(r, features, router_w, d, nullptr, T, rings, priors_out, status, r ? r->stream : nullptr);
}

/* ------------------------------------------------------------------------------------------ */
/* LoRA adapters                                                                              */
/* ------------------------------------------------------------------------------------------ */

struct LoraModule {
  bool valid = false;
  int rank = 0, rpad = 0, in = 0, out = 0;
  DevBuf A, B; /* bf16 [rpad][in], [out][rpad] */
  DevBuf Bf;   /* B in fragment order [out / 32][rpad / 8][32][8] (the prefill GEMMs') */
};

struct aoship_lora_adapter {
  int id = 0;
  float scale = 1.0f;
  std::vector<LoraModule> mods; /* [num_layers * 7] */
  int num_layers = 0;
  int refs = 1; /* the caller's handle + one per binding layer */
};

static void adapter_unref(aoship_lora_adapter *a) {
  if (a && --a->refs == 0) delete a;
}

extern "C" aoship_lora_adapter_t *aoship_lora_adapter_new(int adapter_id, int num_layers,
                                                          float scale) {
  if (num_layers < 1 || num_layers > 4096) {
    set_err("Failed to create LoRA adapter: num_layers out of range");
    return nullptr;
  }
  auto *a = new aoship_lora_adapter();
  a->id = adapter_id;
  a->scale = scale;
  a->num_layers = num_layers;
  a->mods.resize((size_t)num_layers * AOS_MAX_MODULES);
  return a;
}

extern "C" int aoship_lora_adapter_set_module(aoship_lora_adapter_t *a, int layer_idx,
                                              const char *module, int rank, int in_features,
                                              int out_features, const float *lora_a,
                                              const float *lora_b) {
  if (!a || !module || !lora_a || !lora_b)
    return set_err("Null parameter in aoship_lora_adapter_set_module");
  if (layer_idx < 0 || layer_idx >= a->num_layers)
    return set_err("Layer index out of range: " + std::to_string(layer_idx));
  int m = module_index(module);
  if (m < 0) return set_err(std::string("Unknown module name: ") + module);
  if (rank < 1 || rank > 128) return set_err("LoRA rank must be in [1, 128]");
  if (in_features < 64 || in_features % 64 != 0)
    return set_err("LoRA in_features must be a positive multiple of 64");
  if (out_features < 32 || out_features % 32 != 0)
    return set_err("LoRA out_features must be a positive multiple of 32");
  if (ensure_device()) return -1;
  const int rpad = (rank + 15) / 16 * 16;
  std::vector<uint16_t> A((size_t)rpad * in_features, 0), B((size_t)out_features * rpad, 0);
  for (int j = 0; j < rank; ++j)
    for (int i = 0; i < in_features; ++i)
      A[(size_t)j * in_features + i] = f32_to_bf16(lora_a[(size_t)j * in_features + i]);
  for (int o = 0; o < out_features; ++o)
    for (int j = 0; j < rank; ++j)
      B[(size_t)o * rpad + j] = f32_to_bf16(lora_b[(size_t)o * rank + j]);
  std::vector<uint16_t> Bf(B.size(), 0);
  for (int o = 0; o < out_features; ++o)
    for (int j = 0; j < rpad; ++j)
      Bf[((size_t)(o / 32) * (rpad / 8) + j / 8) * 256 + (o % 32) * 8 + j % 8] = B[(size_t)o * rpad + j];
  LoraModule &lm = a->mods[(size_t)layer_idx * AOS_MAX_MODULES + m];
  if (lm.A.upload(A.data(), A.size() * 2)) return -1;
  if (lm.B.upload(B.data(), B.size() * 2)) return -1;
  if (lm.Bf.upload(Bf.data(), Bf.size() * 2)) return -1;
  lm.valid = true;
  lm.rank = rank;
  lm.rpad = rpad;
  lm.in = in_features;
  lm.out = out_features;
  return 0;
}

extern "C" void aoship_lora_adapter_free(aoship_lora_adapter_t *a) { adapter_unref(a); }

/* ------------------------------------------------------------------------------------------ */
/* layers                                                                                     */
/* ------------------------------------------------------------------------------------------ */

struct Q4Mat {
  bool valid = false;
  int out = 0, in = 0, G = 0, RB = 0;
  DevBuf qt, sb;
  aos_q4_dev dev() const {
    aos_q4_dev d;
    d.out = out;
    d.in = in;
    d.G = G;
    d.RB = RB;
    d.qt = qt.as<uint32_t>();
    d.sb = sb.as<uint32_t>();
    return d;
  }
};

struct ModTable {
  int rpad = 0, in = 0, out = 0;
  DevBuf A, B, Bf, scale;
};

struct KStat {
  const char *name;
  double ms = 0.0;
  int64_t launches = 0;
};

struct PendingEvent {
  int slot;
  hipEvent_t a, b;
};

enum {
  KS_ROUTE = 0,
  KS_SHRINK_X,
  KS_GEMV_GU,
  KS_SHRINK_H,
  KS_GEMV_DOWN,
  KS_GEMV_PROJ,
  KS_PPLAN,
  KS_PSHRINK_X,
  KS_GEMM_GU,
  KS_PSHRINK_H,
  KS_GEMM_DOWN,
  KS_GEMM_PROJ,
  KS_DECODE_MLP,
  KS_MLP1,
  KS_PXEXP,
  KS_PAMPLAN,
  KS_PAMX,
  KS_PAMXR,
  KS_PAMH,
  KS_PAMHR,
  KS_PXAML,
  KS_PXAM,
  KS_COUNT
};
static const char *kStatNames[KS_COUNT] = {
    "route",         "lora_shrink_x",   "q4_gemv_gate_up", "lora_shrink_h",
    "q4_gemv_down",  "q4_gemv_proj",    "prefill_group_plan",
    "lora_tile_shrink_x", "q4_gemm_gate_up", "lora_tile_shrink_h", "q4_gemm_down",   "q4_gemm_proj",
    "decode_mlp", "mlp1", "lora_tile_expand_gate_up", "lora_adapter_plan", "lora_adapter_shrink_x",
    "lora_adapter_reduce_x", "lora_adapter_shrink_h", "lora_adapter_reduce_h", "lora_adapter_expand_list",
    "lora_adapter_expand_gate_up"};

struct aoship_layer {
  int layer_idx = 0;
  Q4Mat mats[AOS_MAX_MODULES];
  std::vector<aoship_lora_adapter *> table;
  ModTable tabs[AOS_MAX_MODULES];
  DevBuf bound, scale_all; /* [n] per bound adapter: 1 / alpha-over-rank */
  DevBuf zeros;            /* device zeros read by lanes without an adapter row */
  /* set by a fused launch whose bounded wait gave up: pinned host memory the kernels write
   * through its device mapping, so a forward sees it without synchronising */
  uint32_t *wait_host = nullptr;
  uint32_t *wait_dev = nullptr;
  /* workspace (partials, S, plan, h), arrival counters (zero at rest: each is reset by its last
   * arriver) and generation-stamped ready flags, each grown on demand; counters and flags never
   * share memory, since calls with other token counts lay them out differently */
  DevBuf ws, counters, flags;
  size_t ws_cap = 0, ctr_cap = 0, flag_cap = 0;
  uint32_t gen = 0;        /* generation of the last fused launch (flags are raised to it) */
  const uint16_t *last_perm = nullptr; /* token order of the last grouped prefill chunk (device) */
  int last_perm_T = 0;
  bool separate_shrinks = false; /* each decode shrink in a launch of its own (diagnostic) */
  bool one_launch_mlp = false;   /* 1-2 token MLP in one launch */
  bool producer_lines = true;    /* fused launches hand over through per-producer lines */
  bool plan_ptrs = true;         /* decode plans list the LoRA tables' row pointers */
  bool prefill_fused_shrink = true; /* prefill MLP: the LoRA shrinks run in the GEMM launches */
  int prefill_sk = 3;               /* prefill GEMMs as stream-K: bit 0 gate/up, bit 1 down */
  int last_sk = 0;                  /* the GEMMs the last prefill MLP ran as stream-K (same bits) */
  int prefill_xe_cols = AOS_XE_COLS; /* union columns from which a tile's gate/up expand runs in the
                                        expand launch (0: never) */
  int last_xe = 0;                  /* the last prefill MLP ran the expand launch */
  int prefill_am_tu = AOS_AM_TU;    /* union adapters from which a tile's shrinks run adapter-major
                                       (0: never) */
  int last_am = 0;                  /* the last prefill MLP's adapter-major launches: bit 0 the x shrink,
                                       bit 1 the h shrink, bit 2 the gate/up expand */
  int prefill_xam_tu = AOS_XAM_TU;  /* union adapters from which a tile's gate/up expand runs
                                       adapter-major (0: never) */
  bool mlp1 = false;             /* one token: the MLP (and its routing) in one launch, down in LDS
                                  * (opt-in: slower than the two launches so far) */
  /* decode GEMV geometry forced per launch kind (0 gate/up, 1 down, 2 projections): row blocks per
   * workgroup and K splits, 0 = chosen by the geometry (diagnostic) */
  int geo_wr[3] = {0, 0, 0}, geo_ks[3] = {0, 0, 0};
  hipStream_t stream = nullptr;
  bool profiling = false;
  KStat stats[KS_COUNT];
  std::vector<PendingEvent> pending;
  std::vector<hipEvent_t> event_pool;
};

extern "C" aoship_layer_t *aoship_layer_new(int layer_idx, int group_size, int bits) {
  if (ensure_device()) return nullptr;
  if (group_size != AOSHIP_GROUP_SIZE || bits != AOSHIP_BITS) {
    set_err("aoship_layer_new: only group_size 64 and bits 4 are supported");
    return nullptr;
  }
  if (layer_idx < 0) {
    set_err("aoship_layer_new: negative layer index");
    return nullptr;
  }
  auto *l = new aoship_layer();
  l->layer_idx = layer_idx;
  for (int i = 0; i < KS_COUNT; ++i) l->stats[i].name = kStatNames[i];
  if (l->zeros.alloc(256, true)) {
    delete l;
    return nullptr;
  }
  void *wh = nullptr;
  if (hipHostMalloc(&wh, 256, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) {
    set_err("aoship_layer_new: hipHostMalloc failed");
    delete l;
    return nullptr;
  }
  l->wait_host = (uint32_t *)wh;
  *(volatile uint32_t *)l->wait_host = 0u;
  void *wd = nullptr;
  if (hipHostGetDevicePointer(&wd, wh, 0) != hipSuccess) {
    set_err("aoship_layer_new: hipHostGetDevicePointer failed");
    (void)hipHostFree(wh);
    delete l;
    return nullptr;
  }
  l->wait_dev = (uint32_t *)wd;
  return l;
}

/* The next generation number of a layer's fused launches (never 0: flags start at 0). */
static uint32_t next_gen(uint32_t *g) {
  *g = *g + 1u == 0u ? 1u : *g + 1u;
  return *g;
}

static uint32_t shuffle_nibbles(uint32_t w) {
  uint32_t r = 0;
  for (int p = 0; p < 4; ++p) {
    r |= ((w >> (8 * p)) & 0xFu) << (4 * p);
    r |= ((w >> (8 * p + 4)) & 0xFu) << (4 * (p + 4));
  }
  return r;
}

static int q4_upload(Q4Mat &q, int out_features, int in_features, const uint32_t *packed,
                     const uint16_t *scales_f16, const uint16_t *biases_f16);

extern "C" int aoship_layer_set_base(aoship_layer_t *l, const char *module, int out_features,
                                     int in_features, const uint32_t *packed,
                                     const uint16_t *scales_f16, const uint16_t *biases_f16) {
  if (!l || !packed || !scales_f16) return set_err("aoship_layer_set_base: null argument");
  int m = module_index(module);
  if (m < 0) return set_err(std::string("Unknown module name: ") + (module ? module : "(null)"));
  if (out_features < 32 || out_features % 32 != 0)
    return set_err("aoship_layer_set_base: out_features must be a positive multiple of 32");
  if (in_features < 64 || in_features % 64 != 0)
    return set_err("aoship_layer_set_base: in_features must be a positive multiple of 64");
  if (ensure_device()) return -1;
  return q4_upload(l->mats[m], out_features, in_features, packed, scales_f16, biases_f16);
}

/* MLX 4-bit rows -> the device tile layout: a 1 KiB chunk per (32-row block, group), lane
 * i + 32c holding row i's 32 nibbles of K 32c .. 32c+31 (word s: K 32c+8s .. +7), and one word per
 * (row, group) with the float16 scale (low half) and bias (high half). */
static int q4_upload(Q4Mat &q, int out_features, int in_features, const uint32_t *packed,
                     const uint16_t *scales_f16, const uint16_t *biases_f16) {
  const int G = in_features / 64, RB = out_features / 32, wpr = in_features / 8;
  std::vector<uint32_t> qt((size_t)RB * G * 256), sb((size_t)RB * G * 32);
  for (int rb = 0; rb < RB; ++rb)
    for (int g = 0; g < G; ++g) {
      uint32_t *dst = qt.data() + ((size_t)rb * G + g) * 256;
      for (int l2 = 0; l2 < 64; ++l2) {
        const int n = l2 & 31, c = l2 >> 5;
        const uint32_t *src = packed + (size_t)(rb * 32 + n) * wpr + g * 8 + 4 * c;
        for (int j = 0; j < 4; ++j) dst[l2 * 4 + j] = shuffle_nibbles(src[j]);
      }
      uint32_t *sdst = sb.data() + ((size_t)rb * G + g) * 32;
      for (int n = 0; n < 32; ++n) {
        size_t idx = (size_t)(rb * 32 + n) * G + g;
        uint32_t s = scales_f16[idx], b = biases_f16 ? biases_f16[idx] : 0u;
        sdst[n] = s | (b << 16);
      }
    }
  if (q.qt.upload(qt.data(), qt.size() * 4)) return -1;
  if (q.sb.upload(sb.data(), sb.size() * 4)) return -1;
  q.valid = true;
  q.out = out_features;
  q.in = in_features;
  q.G = G;
  q.RB = RB;
  return 0;
}

static void unbind_all(aoship_layer *l) {
  for (auto *a : l->table) adapter_unref(a);
  l->table.clear();
  for (auto &t : l->tabs) {
    t.A.release();
    t.B.release();
    t.Bf.release();
    t.scale.release();
    t.rpad = 0;
  }
}

extern "C" int aoship_layer_set_adapters(aoship_layer_t *l, aoship_lora_adapter_t *const *table,
                                         int n) {
  if (!l) return set_err("aoship_layer_set_adapters: null layer");
  if (n < 0 || n > AOS_MAX_ADAPTERS) return set_err("aoship_layer_set_adapters: n out of range");
  if (n > 0 && !table) return set_err("aoship_layer_set_adapters: null table");
  if (ensure_device()) return -1;
  /* validate ranks first */
  int rp[AOS_MAX_MODULES] = {0};
  for (int m = 0; m < AOS_MAX_MODULES; ++m)
    for (int a = 0; a < n; ++a) {
      aoship_lora_adapter *ad = table[a];
      if (!ad || l->layer_idx >= ad->num_layers) continue;
      const LoraModule &lm = ad->mods[(size_t)l->layer_idx * AOS_MAX_MODULES + m];
      if (!lm.valid) continue;
      if (rp[m] == 0) rp[m] = lm.rpad;
      if (rp[m] != lm.rpad)
        return set_err("aoship_layer_set_adapters: adapters bound to one module must share a rank");
    }
  HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  unbind_all(l);
  for (int a = 0; a < n; ++a) {
    l->table.push_back(table[a]);
    if (table[a]) table[a]->refs++;
  }
  for (int m = 0; m < AOS_MAX_MODULES; ++m) {
    ModTable &t = l->tabs[m];
    t.rpad = rp[m];
    if (rp[m] == 0 || n == 0) continue;
    std::vector<const void *> A((size_t)n, nullptr), B((size_t)n, nullptr), Bf((size_t)n, nullptr);
    std::vector<float> sc((size_t)n, 0.0f);
    for (int a = 0; a < n; ++a) {
      aoship_lora_adapter *ad = table[a];
      if (!ad || l->layer_idx >= ad->num_layers) continue;
      const LoraModule &lm = ad->mods[(size_t)l->layer_idx * AOS_MAX_MODULES + m];
      if (!lm.valid) continue;
      A[a] = lm.A.p;
      B[a] = lm.B.p;
      Bf[a] = lm.Bf.p;
      sc[a] = ad->scale;
      t.in = lm.in;
      t.out = lm.out;
    }
    if (t.A.upload(A.data(), A.size() * sizeof(void *))) return -1;
    if (t.B.upload(B.data(), B.size() * sizeof(void *))) return -1;
    if (t.Bf.upload(Bf.data(), Bf.size() * sizeof(void *))) return -1;
    if (t.scale.upload(sc.data(), sc.size() * sizeof(float))) return -1;
  }
  std::vector<uint8_t> bd((size_t)(n > 0 ? n : 1), 0);
  std::vector<float> sa((size_t)(n > 0 ? n : 1), 0.0f);
  for (int a = 0; a < n; ++a) {
    aoship_lora_adapter *ad = table[a];
    if (!ad || l->layer_idx >= ad->num_layers) continue;
    for (int m = 0; m < AOS_MAX_MODULES; ++m)
      if (ad->mods[(size_t)l->layer_idx * AOS_MAX_MODULES + m].valid) bd[a] = 1;
    sa[a] = ad->scale;
  }
  if (l->bound.upload(bd.data(), bd.size())) return -1;
  if (l->scale_all.upload(sa.data(), sa.size() * sizeof(float))) return -1;
  return 0;
}

extern "C" int aoship_layer_set_stream(aoship_layer_t *l, void *stream) {
  if (!l) return set_err("aoship_layer_set_stream: null layer");
  l->stream = (hipStream_t)stream;
  return 0;
}

static aos_lora_tab lora_tab(const aoship_layer *l, int m, int in, int out) {
  aos_lora_tab t;
  memset(&t, 0, sizeof(t));
  const ModTable &mt = l->tabs[m];
  if (mt.rpad == 0 || l->table.empty()) return t;
  if (mt.in != in || mt.out != out) return t; /* shapes that do not match this layer are unused */
  t.n = (int)l->table.size();
  t.rpad = mt.rpad;
  t.A = mt.A.as<const uint16_t *const>();
  t.B = mt.B.as<const uint16_t *const>();
  t.Bf = mt.Bf.as<const uint16_t *const>();
  t.scale = mt.scale.as<const float>();
  return t;
}

/* ---- profiling ---- */

static hipEvent_t get_event(aoship_layer *l) {
  if (!l->event_pool.empty()) {
    hipEvent_t e = l->event_pool.back();
    l->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

static void resolve_events(aoship_layer *l) {
  for (auto &pe : l->pending) {
    float ms = 0.0f;
    if (hipEventSynchronize(pe.b) == hipSuccess && hipEventElapsedTime(&ms, pe.a, pe.b) == hipSuccess) {
      l->stats[pe.slot].ms += ms;
      l->stats[pe.slot].launches += 1;
    }
    l->event_pool.push_back(pe.a);
    l->event_pool.push_back(pe.b);
  }
  l->pending.clear();
}

extern "C" int aoship_layer_set_profiling(aoship_layer_t *l, int enable) {
  if (!l) return set_err("aoship_layer_set_profiling: null layer");
  if (ensure_device()) return -1;
  resolve_events(l);
  l->profiling = enable != 0;
  for (auto &s : l->stats) {
    s.ms = 0.0;
    s.launches = 0;
  }
  return 0;
}

/* Reports (1) whether a fused launch of this layer gave up a bounded wait since the last call,
 * and then resets the layer: once the device is idle, every arrival counter and ready flag of its
 * workspace goes back to zero and the generation restarts, so the next forward starts clean. */
extern "C" int aoship_layer_wait_timeouts(aoship_layer_t *l) {
  if (!l) return set_err("aoship_layer_wait_timeouts: null layer");
  if (ensure_device()) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return set_err("aoship_layer_wait_timeouts: device error");
  const uint32_t v = *(volatile uint32_t *)l->wait_host;
  if (!v) return 0;
  if ((l->counters.p && hipMemset(l->counters.p, 0, l->ctr_cap) != hipSuccess) ||
      (l->flags.p && hipMemset(l->flags.p, 0, l->flag_cap) != hipSuccess))
    return set_err("aoship_layer_wait_timeouts: device error");
  /* the allocation-free forward on this device may have been the one that gave up */
  if (g_device >= 0 && g_device < AOS_MAX_DEVICES && g_scratch[g_device].ptr) {
    if (hipMemset(g_scratch[g_device].ptr, 0, AOS_SCRATCH_CTR_BYTES + AOS_SCRATCH_FLAG_BYTES) != hipSuccess)
      return set_err("aoship_layer_wait_timeouts: device error");
    g_scratch[g_device].gen = 0;
  }
  if (hipDeviceSynchronize() != hipSuccess) return set_err("aoship_layer_wait_timeouts: device error");
  l->gen = 0;
  *(volatile uint32_t *)l->wait_host = 0u;
  return 1;
}

/* Diagnostic (no counterpart in the reference): the bound of every in-launch wait of this
 * library's kernels on the current device, in polls (the default, 2^24, is about a second). With
 * 0 every wait gives up before its first poll: each kernel still runs to its end, skips what it
 * waited for and reports the timeout, so tests can drive the give-up paths. Synchronises the
 * device first. */
extern "C" int aoship_internal_set_spin_limit(uint32_t polls) {
  if (ensure_device()) return -1;
  HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  int (*const setters[])(uint32_t) = {aos_spin_setter_router, aos_spin_setter_lora,   aos_spin_setter_gemv,
                                      aos_spin_setter_gemm,   aos_spin_setter_model,  aos_spin_setter_liquid,
                                      aos_spin_setter_mlp1};
  for (auto *f : setters)
    if (f(polls) != (int)hipSuccess) return set_err("aoship_internal_set_spin_limit: hipMemcpyToSymbol failed");
  HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return 0;
}

/* A forward refuses to run while a given-up wait is pending: its counters may be inconsistent. */
static int check_no_timeout(aoship_layer *l) {
  if (*(volatile uint32_t *)l->wait_host)
    return set_err("forward: a fused launch of this layer gave up a bounded wait; "
                   "aoship_layer_wait_timeouts reports and resets it");
  return 0;
}

/* Diagnostic (no counterpart in the reference): the token order (sorted position -> token) of the
 * layer's last grouped MLP prefill chunk, copied to perm[T] on the host after synchronising; valid
 * until the layer's next forward. Returns the chunk's token count, 0 when it was not grouped (no
 * adapters), -1 on error. */
extern "C" int aoship_internal_layer_last_perm(aoship_layer_t *l, uint16_t *perm, int cap) {
  if (!l || !perm) return set_err("aoship_internal_layer_last_perm: null argument");
  if (ensure_device()) return -1;
  if (!l->last_perm) return 0;
  if (cap < l->last_perm_T) return set_err("aoship_internal_layer_last_perm: buffer too small");
  HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  HIP_OR_FAIL(hipMemcpy(perm, l->last_perm, (size_t)l->last_perm_T * 2, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  return l->last_perm_T;
}

/* Diagnostic (no counterpart in the reference): run each decode LoRA shrink in a launch of its
 * own instead of in the first workgroups of the GEMV launch that reads it. Same results within
 * the layer's tolerance; used to test the fused launches against separate ones. */
extern "C" int aoship_internal_layer_set_separate_shrinks(aoship_layer_t *l, int on) {
  if (!l) return set_err("aoship_internal_layer_set_separate_shrinks: null layer");
  l->separate_shrinks = on != 0;
  return 0;
}

/* Diagnostic (no counterpart in the reference): how the decode launches hand over within a
 * launch. one_launch: the 1-2 token MLP runs as one launch instead of two; lines: the producers of
 * a fused launch each raise a line of their own, polled by every consumer, instead of counting in
 * and raising one flag per consumer. Same results either way. */
extern "C" int aoship_internal_layer_set_decode_handoff(aoship_layer_t *l, int one_launch, int lines) {
  if (!l) return set_err("aoship_internal_layer_set_decode_handoff: null layer");
  l->one_launch_mlp = one_launch != 0;
  l->producer_lines = lines != 0;
  return 0;
}

/* Diagnostic (no counterpart in the reference): whether a decode plan also lists the union's
 * row pointers in the LoRA tables its GEMV readers use (default on: a reader then needs one load
 * for a pointer rather than two, and a fused launch's first expand step two round trips after its
 * wait). The loads change, the arithmetic does not: outputs are identical either way. */
/* Diagnostic (no counterpart in the reference): copies bytes [offset, offset + bytes) of the layer's
 * flag memory (where the one-token launch keeps its tagged exchange words) to dst on the host, after
 * synchronising the device. Returns the flag memory's size, or -1. */
extern "C" long aoship_internal_layer_read_flags(aoship_layer_t *l, size_t offset, size_t bytes, void *dst) {
  if (!l) return set_err("aoship_internal_layer_read_flags: null layer");
  if (ensure_device()) return -1;
  HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
  if (bytes) {
    if (!dst || offset + bytes > l->flag_cap) return set_err("aoship_internal_layer_read_flags: out of range");
    HIP_OR_FAIL(hipMemcpy(dst, (char *)l->flags.p + offset, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  }
  return (long)l->flag_cap;
}

/* Diagnostic (no counterpart in the reference): the one-token MLP as one launch with the down
 * matrix in LDS where the layer's shape fits (off by default: the two-launch path is faster). */
extern "C" int aoship_internal_layer_set_mlp1(aoship_layer_t *l, int on) {
  if (!l) return set_err("aoship_internal_layer_set_mlp1: null layer");
  l->mlp1 = on != 0;
  return 0;
}

extern "C" int aoship_internal_layer_set_plan_pointers(aoship_layer_t *l, int on) {
  if (!l) return set_err("aoship_internal_layer_set_plan_pointers: null layer");
  l->plan_ptrs = on != 0;
  return 0;
}

/* Diagnostic (no counterpart in the reference): which prefill GEMMs may run as stream-K over the
 * device's resident workgroups (bit 0 gate/up, bit 1 down; both by default) where the plan finds
 * it pays, instead of one workgroup per (token tile, row block) task. Results agree within
 * float32 summation order; each form is deterministic run to run. */
extern "C" int aoship_internal_layer_set_prefill_sk(aoship_layer_t *l, int mask) {
  if (!l) return set_err("aoship_internal_layer_set_prefill_sk: null layer");
  l->prefill_sk = mask & 3;
  return 0;
}

/* Diagnostic (no counterpart in the reference): the prefill GEMMs that ran as stream-K in the
 * layer's last prefill MLP (bit 0 gate/up, bit 1 down; of its last chunk of tokens). */
extern "C" int aoship_internal_layer_last_stream_k(aoship_layer_t *l) {
  if (!l) return set_err("aoship_internal_layer_last_stream_k: null layer");
  return l->last_sk;
}

/* Diagnostic (no counterpart in the reference): the union width (columns of a tile's wider module,
 * tu * max(rpad_gate, rpad_up)) from which the prefill MLP's gate/up LoRA expand of a tile runs in
 * an expand launch of its own, whose sums the SwiGLU GEMM adds before the activation, instead of in
 * the GEMM (cols 0: never; negative: the default, AOS_XE_COLS). Results agree within float32
 * summation order; each form is deterministic run to run. */
extern "C" int aoship_internal_layer_set_prefill_expand(aoship_layer_t *l, int cols) {
  if (!l) return set_err("aoship_internal_layer_set_prefill_expand: null layer");
  l->prefill_xe_cols = cols < 0 ? AOS_XE_COLS : cols;
  return 0;
}

/* Diagnostic (no counterpart in the reference): 1 when the layer's last prefill MLP (its last
 * chunk of tokens) ran the gate/up expand launch, else 0. */
extern "C" int aoship_internal_layer_last_expand(aoship_layer_t *l) {
  if (!l) return set_err("aoship_internal_layer_last_expand: null layer");
  return l->last_xe;
}

/* Diagnostic (no counterpart in the reference): the union size (adapters) from which a tile's
 * prefill MLP LoRA shrinks run adapter-major (each adapter's users gathered into tiles of their
 * own) instead of over the tile's union (tu 0: never; negative: the default, AOS_AM_TU). Applies to
 * the shrinks that run in launches of their own. Results agree within float32 summation order;
 * each form is deterministic run to run. */
extern "C" int aoship_internal_layer_set_prefill_adapter_major(aoship_layer_t *l, int tu) {
  if (!l) return set_err("aoship_internal_layer_set_prefill_adapter_major: null layer");
  l->prefill_am_tu = tu < 0 ? AOS_AM_TU : tu;
  return 0;
}

/* Diagnostic (no counterpart in the reference): the union size (adapters) from which a tile's
 * prefill MLP gate/up LoRA expand runs adapter-major (each adapter's users gathered into MFMA tiles,
 * their sums added in LDS in adapter order) instead of over the tile's union in the expand launch
 * (tu 0: never; negative: the default, AOS_XAM_TU). Applies with the expand launch and the
 * adapter-major shrinks' user lists, up to AOS_XAM_MAX_N bound adapters and ranks of 64. Results
 * agree within float32 summation order; each form is deterministic run to run. */
extern "C" int aoship_internal_layer_set_prefill_expand_adapter_major(aoship_layer_t *l, int tu) {
  if (!l) return set_err("aoship_internal_layer_set_prefill_expand_adapter_major: null layer");
  l->prefill_xam_tu = tu < 0 ? AOS_XAM_TU : tu;
  return 0;
}

/* Diagnostic (no counterpart in the reference): the adapter-major launches of the layer's last
 * prefill MLP (its last chunk of tokens): bit 0 the x shrink, bit 1 the h shrink, bit 2 the gate/up
 * expand. */
extern "C" int aoship_internal_layer_last_adapter_major(aoship_layer_t *l) {
  if (!l) return set_err("aoship_internal_layer_last_adapter_major: null layer");
  return l->last_am;
}

/* Diagnostic (no counterpart in the reference): whether the prefill MLP's LoRA shrinks run as
 * the first workgroups of the GEMM launches that consume them (fused) or as launches of their
 * own with K split into slices. Results agree within float32 summation order. */
extern "C" int aoship_internal_layer_set_prefill_shrink(aoship_layer_t *l, int fused) {
  if (!l) return set_err("aoship_internal_layer_set_prefill_shrink: null layer");
  l->prefill_fused_shrink = fused != 0;
  return 0;
}

extern "C" int aoship_layer_kernel_stats(aoship_layer_t *l, int idx, const char **name,
                                         double *total_ms, int64_t *launches) {
  if (!l) return set_err("aoship_layer_kernel_stats: null layer");
  if (ensure_device()) return -1;
  resolve_events(l);
  if (idx >= 0 && idx < KS_COUNT) {
    if (name) *name = l->stats[idx].name;
    if (total_ms) *total_ms = l->stats[idx].ms;
    if (launches) *launches = l->stats[idx].launches;
  }
  return KS_COUNT;
}

/* Launch context for one kernel of this layer: with profiling on, the dispatch records a pair
 * of events at kernel start and end, resolved lazily by aoship_layer_kernel_stats. */
static aos_launch_ctx launch_ctx(aoship_layer *l, int slot, bool events = true) {
  aos_launch_ctx c;
  c.stream = l->stream;
  c.ev_start = nullptr;
  c.ev_stop = nullptr;
  if (l->profiling && events) {
    hipEvent_t a = get_event(l), b = get_event(l);
    if (a && b) {
      c.ev_start = a;
      c.ev_stop = b;
      l->pending.push_back({slot, a, b});
    }
  }
  return c;
}

/* ---- workspace ---- */

/* Where a decode forward's scratch memory lives: the layer's own workspace (grown on demand) or
 * the device's static scratch (the allocation-free entry point). gen counts the generations of
 * the flags in that memory; events says whether launches may record profiling events (that
 * creates event objects, which the allocation-free entry point does not do). */
struct Ws {
  void *ws;
  void *ctr;
  void *flg;
  uint32_t *gen;
  bool events;
};

struct Bump {
  char *base;
  size_t off = 0, cap;
  Bump(void *b, size_t c) : base((char *)b), cap(c) {}
  template <class T>
  T *take(size_t n) {
    off = (off + 255) & ~(size_t)255;
    T *p = (T *)(base ? base + off : nullptr);
    off += n * sizeof(T);
    return p;
  }
};

static int ws_reserve(aoship_layer *l, size_t bytes, size_t ctr_words, size_t flag_words = 0) {
  if (bytes > l->ws_cap) {
    HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
    l->last_perm = nullptr;
    l->last_perm_T = 0;
    if (l->ws.alloc(bytes, false)) return -1;
    l->ws_cap = bytes;
  }
  if (ctr_words * 4 > l->ctr_cap) {
    HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (l->counters.alloc(ctr_words * 4, true)) return -1;
    l->ctr_cap = ctr_words * 4;
  }
  if (flag_words * 4 > l->flag_cap) { /* zeroed: no generation is 0 */
    HIP_OR_FAIL(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (l->flags.alloc(flag_words * 4, true)) return -1;
    l->flag_cap = flag_words * 4;
  }
  return 0;
}

static int ceil_div(int a, int b) { return (a + b - 1) / b; }

static int nv_for(int T) {
  if (T <= 1) return 1;
  if (T <= 2) return 2;
  if (T <= 8) return 4;
  if (T <= 16) return 8;
  return 16;
}

/* Decode GEMV geometry: waves per workgroup, K splits across workgroups, dynamic LDS bytes.
 * About 1024 waves stream the matrix (fewer K splits, less reduction); the x slice of a workgroup (T rows) plus its group sums
 * must fit the LDS budget; the K-split-0 workgroup of each row block adds the LoRA expand when
 * any bound adapter has this module. */
#ifndef AOS_GEMV_WAVES
#define AOS_GEMV_WAVES 1024 /* waves streaming one matrix (measured best at decode) */
#define AOS_GEMV_WAVES_DOWN12 1536 /* ... the 1-2 token down GEMV, whose plan and first B fragments load
                                    * before its K loop (measured on two boxes: 4 splits of the 7B
                                    * shape against 3, the launch 0.5-1 us shorter) */
#define AOS_GEMV_WAVES_PROJ12 256 /* ... the 1-2 token projections: one K split from 64 row blocks on
                                   * (the 7B q/k/v and o launches each 3-4 us shorter without the split
                                   * reduction's round trip: model decode 2.65 -> 2.56 ms/token) */
#endif
#ifndef AOS_GEMV_W8_MIN_G
#define AOS_GEMV_W8_MIN_G 128 /* single-matrix GEMVs with at least this many groups use 8 waves */
#endif
static int gemv_splits(int RB, int G, int T, int W, int waves_target) {
  int ks = ceil_div(waves_target, RB * W);
  int cap = G / W;
  if (cap < 1) cap = 1;
  if (ks > cap) ks = cap;
  while (ks < G && (size_t)T * ceil_div(G, ks) * 136 > AOS_GEMV_LDS_MAX) ++ks;
  return ks;
}

/* Staged x (T rows of the split's groups, their group sums and 128 zero bytes) and the wave
 * reduction's LDS. */
static size_t gemv_lds_x(int T, int G, int ks) { return 128 + (size_t)T * ceil_div(G, ks) * 136; }

/* Row-split geometry (3 or more tokens): the waves of a workgroup take different row blocks over
 * one K split, so the x slice staged in LDS serves WR row blocks instead of one (x staged over a
 * whole launch scales with RB / WR). The rules below are the best of sweeps over (WR, ks) on
 * MI355X (the 7B MLP at 4, 8 and 32 tokens, the 3B projections at 32): the fewest K splits that
 * keep x within an LDS budget while each wave streams at most a given number of K groups - fewer
 * splits leave too few workgroups to fill the GPU, more add partial sums and x staging per byte
 * of weights.
 *   gate/up (SwiGLU, 4 waves): 4 row blocks per workgroup, 32 KiB of x, 14 groups of both matrices;
 *   one long matrix (8 waves: K >= 128 groups): 8 row blocks, 64 KiB of x, 40 groups;
 *   one short matrix (4 waves): 4 row blocks, 32 KiB of x, 6 groups.
 * wr_force / ks_force (> 0) pin either choice (diagnostic: up to 64 KiB of x); a pinned shape that
 * does not fit falls back to a row block per wave and the fewest splits that fit 32 KiB. */
#ifndef AOS_GEMV_LDS_MAX_ROWS
#define AOS_GEMV_LDS_MAX_ROWS (64 * 1024) /* staged x of a row-split shape, at most */
#endif
static void gemv_geometry_rows(int RB, int G, int T, bool swiglu, int W, aos_gemv_params &g, int wr_force,
                               int ks_force) {
  const int NA = swiglu ? 2 : 1;
  int wr_auto = 4, gmax = 6;
  size_t budget = AOS_GEMV_LDS_MAX;
  if (swiglu) {
    gmax = 14;
  } else if (W == 8) {
    wr_auto = 8;
    gmax = 40;
    budget = AOS_GEMV_LDS_MAX_ROWS;
  }
  int WR = wr_force > 0 ? wr_force : wr_auto;
  if (WR > W) WR = W;
  const int WK = W / WR;
  auto fits = [&](int ks, size_t b) { return ks <= G && G / ks >= WK && gemv_lds_x(T, G, ks) <= b; };
  int ks = 0;
  if (ks_force > 0) {
    if (fits(ks_force, AOS_GEMV_LDS_MAX_ROWS)) ks = ks_force;
  } else {
    for (int k = 1; k <= G && !ks; ++k)
      if (fits(k, budget) && ceil_div(ceil_div(G, k), WK) <= gmax) ks = k;
    for (int k = 1; k <= G && !ks; ++k) /* no split within the stream limit: the fewest that fit */
      if (fits(k, budget)) ks = k;
  }
  if (ks == 0) { /* nothing fits what was asked: a row block per wave, the fewest splits that fit */
    WR = W;
    ks = 1;
    while (ks < G && gemv_lds_x(T, G, ks) > AOS_GEMV_LDS_MAX) ++ks;
  }
  (void)RB;
  (void)NA;
  g.wr = WR;
  g.ks = ks;
}

/* Every wave of a K split must get at least one group (G / ks >= W): the 8-wave single-matrix
 * kernel falls back to 4 waves when the LDS budget forces more splits (many tokens, long K).
 * From 3 tokens on, the row-split geometry above. */
static void gemv_geometry(int RB, int G, int T, bool swiglu, bool lora, aos_gemv_params &g,
                          int waves_target = AOS_GEMV_WAVES, bool four_waves = false, int wr_force = 0,
                          int ks_force = 0) {
  int W = (swiglu || four_waves) ? 4 : (G >= AOS_GEMV_W8_MIN_G ? 8 : 4);
  int ks = 1;
  g.wr = 1;
  /* at 1-2 tokens the SwiGLU launch forms the h shrink's partials, one row block per workgroup
   * (wave 0 of the workgroup forms them): a pinned shape keeps one row block per workgroup, and
   * a pinned split count that leaves a wave without a K group or exceeds the LDS budget is not
   * applied */
  const bool one_rb = swiglu && T <= 2;
  if (one_rb && ks_force > 0 && (ks_force > G || G / ks_force < W || gemv_lds_x(T, G, ks_force) > AOS_GEMV_LDS_MAX))
    ks_force = 0;
  if (one_rb && ks_force > 0) {
    ks = ks_force;
  } else if (!one_rb && (T > 2 || wr_force > 0 || ks_force > 0)) {
    gemv_geometry_rows(RB, G, T, swiglu, W, g, wr_force, ks_force);
    ks = g.ks;
  } else {
    ks = gemv_splits(RB, G, T, W, waves_target);
    if (G / ks < W && W == 8) {
      W = 4;
      ks = gemv_splits(RB, G, T, W, waves_target);
    }
  }
  const int NA = swiglu ? 2 : 1;
  size_t lds_x = gemv_lds_x(T, G, ks);
  size_t lds_r = (size_t)W * NA * nv_for(T) * 64 * 4;
  g.waves = W;
  g.ks = ks;
  g.nrbg = g.w0.RB > 0 ? ceil_div(g.w0.RB, g.wr) : 0;
  g.has_expand = lora ? 1 : 0;
  g.lds_bytes = (int)(lds_x > lds_r ? lds_x : lds_r);
}

/* Shrink geometry: a target number of workgroups over the row blocks (512 waves for 4-wave
 * workgroups, 2048 for 8-wave ones; measured best at decode with the shrink running beside its
 * GEMV), at least one group per wave, x slice within the LDS budget, at most 16 K splits (their
 * partials are summed by one workgroup). */
#ifndef AOS_SHRINK_WGS
#define AOS_SHRINK_WGS 256
#endif
/* The x shrink's budget for staged x above 16 tokens: those fused launches run two waves per SIMD
 * (their registers), so 64 KB of LDS per workgroup costs them no residency, and fewer K splits
 * keep the launch within one round of resident workgroups (the 32-stream projections: 336 shrink
 * workgroups at 32 KB, 192 at 64 KB). */
#define AOS_XSHRINK_LDS_MAX_T32 (64 * 1024)
static size_t x_shrink_lds_max(int T) { return T > 16 ? AOS_XSHRINK_LDS_MAX_T32 : AOS_GEMV_LDS_MAX; }

static void shrink_geometry(int rb_total, int G, int T, aos_shrink_params &sp, int waves = 4,
                            size_t lds_max = AOS_GEMV_LDS_MAX) {
  const int target = waves == 8 ? AOS_SHRINK_WGS : AOS_SHRINK_WGS / 2;
  int ks = ceil_div(target, rb_total > 0 ? rb_total : 1);
  int cap = G / waves; /* every wave of a workgroup gets at least one group */
  if (cap < 1) cap = 1;
  if (cap > 16) cap = 16;
  if (ks > cap) ks = cap;
  while (ks < G && 128 + (size_t)T * ceil_div(G, ks) * 128 > lds_max) ++ks;
  size_t lds_x = 128 + (size_t)T * ceil_div(G, ks) * 128;
  size_t lds_r = (size_t)waves * nv_for(T) * 64 * 4;
  sp.ks = ks;
  sp.lds_bytes = (int)(lds_x > lds_r ? lds_x : lds_r);
}

/* Diagnostic (no counterpart in the reference): the decode geometry the forwards use, for a
 * CPU-side check that every wave of every launch gets at least one K group. kind 0: the gate/up
 * GEMV (out = intermediate, in = hidden); 1: the down GEMV (out = hidden, in = intermediate);
 * 2: a projection GEMV (out = the row count of the matrices sharing x); 3: a shrink over `out`
 * rank rows launched with 8 waves when in / 64 >= AOS_GEMV_W8_MIN_G, else 4 (the x shrink);
 * 4: the same with 8 waves (the h shrink). Writes the waves, the K splits, the row blocks per
 * workgroup (GEMVs; 1 for a shrink) and the fewest groups any wave gets. */
extern "C" int aoship_internal_decode_geometry_pinned(int kind, int out, int in, int T, int wr_pin, int ks_pin,
                                                      int *waves, int *ks, int *wr, int *min_groups);

extern "C" int aoship_internal_decode_geometry(int kind, int out, int in, int T, int *waves, int *ks, int *wr,
                                               int *min_groups) {
  return aoship_internal_decode_geometry_pinned(kind, out, in, T, 0, 0, waves, ks, wr, min_groups);
}

/* The same with a GEMV shape pinned as aoship_internal_layer_set_gemv_geometry pins it (wr_pin row
 * blocks per workgroup, ks_pin K splits; 0: the geometry's own choice; GEMV kinds only). */
extern "C" int aoship_internal_decode_geometry_pinned(int kind, int out, int in, int T, int wr_pin, int ks_pin,
                                                      int *waves, int *ks, int *wr, int *min_groups) {
  if (out < 32 || in < 64 || in % 64 || T < 1 || T > AOS_DECODE_MAX_T || !waves || !ks || !wr || !min_groups ||
      wr_pin < 0 || wr_pin > 8 || (wr_pin & (wr_pin - 1)) || ks_pin < 0 || ks_pin > 64 ||
      (kind > 2 && (wr_pin || ks_pin)))
    return set_err("aoship_internal_decode_geometry: bad arguments");
  const int G = in / 64, RB = out / 32;
  int W = 4, k = 1, r = 1;
  if (kind <= 2) {
    aos_gemv_params g;
    memset(&g, 0, sizeof(g));
    const int target = kind == 1   ? (T <= 2 ? AOS_GEMV_WAVES_DOWN12 : 2 * AOS_GEMV_WAVES)
                       : kind == 2 ? (T <= 2 ? AOS_GEMV_WAVES_PROJ12 : AOS_GEMV_WAVES)
                                   : AOS_GEMV_WAVES;
    gemv_geometry(RB, G, T, kind == 0, true, g, target, kind == 1 && T <= 2, wr_pin, ks_pin);
    W = g.waves;
    k = g.ks;
    r = g.wr;
  } else if (kind <= 4) {
    aos_shrink_params sp;
    memset(&sp, 0, sizeof(sp));
    W = kind == 4 ? 8 : (G >= AOS_GEMV_W8_MIN_G ? 8 : 4);
    shrink_geometry(RB, G, T, sp, W, kind == 3 ? x_shrink_lds_max(T) : AOS_GEMV_LDS_MAX);
    k = sp.ks;
  } else {
    return set_err("aoship_internal_decode_geometry: unknown kind");
  }
  *waves = W;
  *ks = k;
  *wr = r;
  *min_groups = (G / k) / (W / r);
  return 0;
}

/* Diagnostic (no counterpart in the reference): pin the decode GEMV geometry of one launch kind
 * of this layer (0: gate/up, 1: down, 2: projections) to wr row blocks per workgroup and ks K
 * splits (0: the geometry's own choice), for measurement sweeps. A pinned shape that leaves a
 * wave without a K group or exceeds the LDS budget is rejected at the next forward. */
extern "C" int aoship_internal_layer_set_gemv_geometry(aoship_layer_t *l, int kind, int wr, int ks) {
  if (!l) return set_err("aoship_internal_layer_set_gemv_geometry: null layer");
  if (kind < 0 || kind > 2 || wr < 0 || wr > 8 || (wr & (wr - 1)) || ks < 0 || ks > 64)
    return set_err("aoship_internal_layer_set_gemv_geometry: bad arguments");
  l->geo_wr[kind] = wr;
  l->geo_ks[kind] = ks;
  return 0;
}

/* One decode chunk (T <= 32 tokens) of a forward: the workspace carve-up and every launch's
 * parameters. The same code sizes the workspace (base == nullptr) and fills it. */
struct Carve {
  Bump b;
  uint32_t *cbase, *fbase;
  size_t coff = 0, foff = 0;
  Carve(void *ws, void *ctr, void *flg = nullptr) : b(ws, 0), cbase((uint32_t *)ctr), fbase((uint32_t *)flg) {}
  uint32_t *counters(size_t n) {
    uint32_t *p = cbase ? cbase + coff : nullptr;
    coff += n;
    return p;
  }
  /* counters starting on a 128-byte line (the base is 256-byte aligned) */
  uint32_t *counter_lines(size_t n) {
    coff = (coff + 31) & ~(size_t)31;
    return counters(n);
  }
  /* generation-stamped flags, from a line of their own */
  uint32_t *flag_lines(size_t n) {
    foff = (foff + 31) & ~(size_t)31;
    uint32_t *p = fbase ? fbase + foff : nullptr;
    foff += n;
    return p;
  }
};

static aos_plan_params plan_params(aoship_layer *l, const aoship_ring_t *rings, int T, aos_plan *plan) {
  aos_plan_params pp;
  memset(&pp, 0, sizeof(pp));
  pp.rings = rings;
  pp.T = T;
  pp.n = (int)l->table.size();
  pp.bound = l->bound.as<uint8_t>();
  pp.scale = l->scale_all.as<float>();
  pp.plan = plan;
  return pp;
}

/* Shrink of x for the given modules: every bound adapter ("all" mode, no rings needed) when that
 * is at most twice the rows of the call's possible union, else the union (the plan is then
 * built by a launch of its own first). */
struct XShrink {
  aos_shrink_params sp;
  bool separate_plan = false;
  aos_shrink_params plan_only;
};

static int shrink_wgs(const aos_shrink_params &sp) {
  return (sp.n_rb[0] + (sp.nmod > 1 ? sp.n_rb[1] : 0) + (sp.nmod > 2 ? sp.n_rb[2] : 0) + (sp.plan_build.plan ? 1 : 0)) *
         sp.ks;
}

/* Producer lines of a shrink: its row blocks and the plan workgroup (counted whether or not the
 * shrink builds the plan: a sizing pass has no plan pointer). */
static size_t shrink_lines(const aos_shrink_params &sp) {
  return (size_t)(sp.n_rb[0] + (sp.nmod > 1 ? sp.n_rb[1] : 0) + (sp.nmod > 2 ? sp.n_rb[2] : 0) + 1);
}

/* Arrival counter words for a shrink's workgroups, counting the plan workgroup whether or not
 * the shrink builds the plan (a sizing pass has no plan pointer). */
static size_t shrink_arrive_words(const aos_shrink_params &sp) {
  const int rows = sp.n_rb[0] + (sp.nmod > 1 ? sp.n_rb[1] : 0) + (sp.nmod > 2 ? sp.n_rb[2] : 0) + 1;
  return AOS_ARRIVE_WORDS(rows * sp.ks);
}

/* The hand-off memory of a fused launch: the arrival counter and the consumers' ready flags
 * (counted hand-off), and the producers' lines (per-producer hand-off). */
struct Handoff {
  uint32_t *sync = nullptr, *flags = nullptr, *lines = nullptr;
};

static Handoff carve_handoff(Carve &cv, size_t arrive_words, size_t flag_words, size_t n_lines) {
  Handoff h;
  h.sync = cv.counter_lines(arrive_words);
  h.flags = cv.flag_lines(flag_words);
  h.lines = cv.flag_lines(32 * n_lines);
  return h;
}

/* Flag words of a fused launch: one 128-byte line per GEMV workgroup for its ready flag. */
static size_t fused_flag_words(const aos_gemv_params *gp, int n) {
  size_t c = 0;
  for (int i = 0; i < n; ++i) c += (size_t)gp[i].nrbg * gp[i].ks;
  return 32 * c;
}

static void plan_x_shrink(aoship_layer *l, Carve &cv, const uint16_t *x, int T, int in,
                          const aos_lora_tab *tabs, int nm, aos_plan *plan,
                          const aoship_ring_t *rings, XShrink &xs) {
  const int n = (int)l->table.size();
  int umax = n < 8 * T ? n : 8 * T;
  if (umax < 1) umax = 1;
  const bool all = n <= 2 * umax || n <= 16;
  aos_shrink_params &sp = xs.sp;
  memset(&sp, 0, sizeof(sp));
  sp.x = x;
  sp.T = T;
  sp.in = in;
  sp.nmod = nm;
  sp.all_mode = all ? 1 : 0;
  sp.plan = plan;
  sp.zero_row = l->zeros.as<uint16_t>();
  int rb_total = 0;
  for (int i = 0; i < nm; ++i) {
    sp.tab[i] = tabs[i];
    const int rp = tabs[i].rpad;
    const int slots = all ? n : umax;
    sp.s_stride[i] = slots * (rp ? rp : 16);
    sp.n_rb[i] = rp ? ceil_div(slots * rp, 32) : 0;
    sp.S[i] = cv.b.take<float>((size_t)T * sp.s_stride[i]);
    rb_total += sp.n_rb[i];
  }
  /* sized for the waves of the GEMV it may be fused with (valid for the 4-wave launch too) */
  shrink_geometry(rb_total, in / 64, T, sp, in / 64 >= AOS_GEMV_W8_MIN_G ? 8 : 4, x_shrink_lds_max(T));
  sp.part = cv.b.take<float>((size_t)rb_total * sp.ks * nv_for(T) * 64);
  sp.counters = cv.counters((size_t)rb_total + 1);
  xs.separate_plan = !all;
  if (all) {
    sp.plan_build = plan_params(l, rings, T, plan);
  } else {
    memset(&xs.plan_only, 0, sizeof(xs.plan_only));
    xs.plan_only.T = T;
    xs.plan_only.nmod = 1;
    xs.plan_only.ks = 1;
    xs.plan_only.plan_build = plan_params(l, rings, T, plan);
    xs.plan_only.zero_row = sp.zero_row;
  }
}

/* The plan build of an x shrink (in its launch, or in a launch of its own), and the tables whose
 * row pointers the plan lists for its readers (k: the table's slot; the readers' pk = k + 1). */
static aos_plan_params &plan_build_of(XShrink &xs) {
  return xs.separate_plan ? xs.plan_only.plan_build : xs.sp.plan_build;
}

static int plan_list_table(const aoship_layer *l, XShrink &xs, int k, const uint16_t *const *table) {
  if (!l->plan_ptrs) table = nullptr;
  plan_build_of(xs).ptab[k] = table;
  return table ? k + 1 : 0;
}

/* Plan of one decode chunk of the SwiGLU MLP. */
struct MlpPlan {
  XShrink sx;
  aos_shrink_params sh;
  aos_gemv_params gv1, gv2;
  Handoff ho1, ho2;          /* the fused launches' hand-off memory */
  float *hpart;            /* [RB of gate/up][T][s_stride of the down shrink]: the h shrink's partials
                              (1-2 tokens only, else NULL) */
  uint32_t *hdone;         /* one-launch MLP (1-2 tokens): gate/up row blocks done */
  uint32_t *hflags;        /* ... and the lines raised when h is complete */
  int hsum_wgs = 0;        /* workgroups summing the h shrink's partials */
  uint32_t *route_done;    /* the combined route + gate/up launch's router arrivals */
  uint32_t *route_flag;    /* ... and its routing flag */
  uint32_t *rpart_ctr;     /* ... its per-token counts of prior workgroups */
  float *rpri;             /* ... and the priors they hand over */
  size_t bytes = 0, ctr = 0, flg = 0;
};

static void plan_mlp(aoship_layer *l, int T, const uint16_t *x, const aoship_ring_t *rings,
                     uint16_t *y, void *ws, void *ctr, void *flg, MlpPlan &P) {
  const Q4Mat &Wg = l->mats[MOD_GATE], &Wu = l->mats[MOD_UP], &Wd = l->mats[MOD_DOWN];
  const int H = Wg.in, I = Wg.out;
  aos_lora_tab tabs_gu[2] = {lora_tab(l, MOD_GATE, H, I), lora_tab(l, MOD_UP, H, I)};
  aos_lora_tab td = lora_tab(l, MOD_DOWN, I, H);
  const int n = (int)l->table.size();
  int umax = n < 8 * T ? n : 8 * T;
  if (umax < 1) umax = 1;
  Carve cv(ws, ctr, flg);
  aos_plan *plan = cv.b.take<aos_plan>(1);
  uint16_t *h = cv.b.take<uint16_t>((size_t)T * I);
  plan_x_shrink(l, cv, x, T, H, tabs_gu, 2, plan, rings, P.sx);

  aos_gemv_params &g1 = P.gv1;
  memset(&g1, 0, sizeof(g1));
  g1.w0 = Wg.dev();
  g1.w1 = Wu.dev();
  g1.x = x;
  g1.T = T;
  gemv_geometry(Wg.RB, Wg.G, T, true, tabs_gu[0].rpad > 0 || tabs_gu[1].rpad > 0, g1, AOS_GEMV_WAVES, false,
                l->geo_wr[0], l->geo_ks[0]);
  g1.tab0 = tabs_gu[0];
  g1.tab1 = tabs_gu[1];
  g1.S0 = P.sx.sp.S[0];
  g1.S1 = P.sx.sp.S[1];
  g1.s_stride0 = P.sx.sp.s_stride[0];
  g1.s_stride1 = P.sx.sp.s_stride[1];
  g1.s_all = P.sx.sp.all_mode;
  g1.plan = plan;
  g1.pk0 = plan_list_table(l, P.sx, 0, tabs_gu[0].B);
  g1.pk1 = plan_list_table(l, P.sx, 1, tabs_gu[1].B);
  g1.pkh = plan_list_table(l, P.sx, 2, td.A);
  g1.zero_row = l->zeros.as<uint16_t>();
  g1.y = h;
  g1.part = cv.b.take<float>((size_t)Wg.RB * g1.ks * 2 * nv_for(T) * 64);
  g1.counters = cv.counters((size_t)Wg.RB);

  aos_shrink_params &s2 = P.sh;
  memset(&s2, 0, sizeof(s2));
  s2.x = h;
  s2.T = T;
  s2.in = I;
  s2.nmod = 1;
  s2.tab[0] = td;
  s2.all_mode = 0;
  s2.plan = plan;
  s2.zero_row = l->zeros.as<uint16_t>();
  s2.s_stride[0] = umax * (td.rpad ? td.rpad : 16);
  s2.n_rb[0] = td.rpad ? ceil_div(umax * td.rpad, 32) : 0;
  s2.S[0] = cv.b.take<float>((size_t)T * s2.s_stride[0]);
  shrink_geometry(s2.n_rb[0], I / 64, T, s2, 8); /* valid for the 4-wave launch and the 8-wave fused one */
  s2.part = cv.b.take<float>((size_t)(s2.n_rb[0] + 1) * s2.ks * nv_for(T) * 64);
  s2.counters = cv.counters((size_t)s2.n_rb[0] + 1);

  aos_gemv_params &g2 = P.gv2;
  memset(&g2, 0, sizeof(g2));
  g2.w0 = Wd.dev();
  g2.x = h;
  g2.T = T;
  /* the down GEMV streams beside the h shrink of its launch: more K splits (measured: 3 at the
   * 7B shape) keep its tail short; at 1-2 tokens it runs in the gate/up launch's grid, in
   * 4-wave workgroups like the rest of that grid */
  gemv_geometry(Wd.RB, Wd.G, T, false, td.rpad > 0, g2, T <= 2 ? AOS_GEMV_WAVES_DOWN12 : 2 * AOS_GEMV_WAVES, T <= 2,
                l->geo_wr[1], l->geo_ks[1]);
  g2.tab0 = td;
  g2.S0 = s2.S[0];
  g2.s_stride0 = s2.s_stride[0];
  g2.s_all = 0;
  g2.plan = plan;
  g2.pk0 = plan_list_table(l, P.sx, 3, td.B);
  g2.zero_row = l->zeros.as<uint16_t>();
  g2.y = y;
  g2.part = cv.b.take<float>((size_t)Wd.RB * g2.ks * nv_for(T) * 64);
  g2.counters = cv.counters((size_t)Wd.RB);

  P.hpart = T <= 2 ? cv.b.take<float>((size_t)Wg.RB * T * s2.s_stride[0]) : nullptr;
  P.hsum_wgs = ceil_div(T * s2.s_stride[0], AOS_HSUM_V);
  P.hdone = cv.counter_lines(AOS_ARRIVE_WORDS(Wg.RB));
  P.hflags = cv.flag_lines(((size_t)P.hsum_wgs + (size_t)g2.nrbg * g2.ks) * 32);
  P.route_done = cv.counter_lines(32);
  P.route_flag = cv.flag_lines(32);
  P.rpart_ctr = cv.counter_lines((size_t)32 * T);
  P.rpri = cv.b.take<float>((size_t)T * AOS_ROUTE_PARTS_MAXN);
  P.ho1 = carve_handoff(cv, shrink_arrive_words(P.sx.sp), fused_flag_words(&g1, 1), shrink_lines(P.sx.sp));
  {
    /* the h shrink's or the h sum's workgroups */
    const size_t w_sh = shrink_arrive_words(s2), w_hs = AOS_ARRIVE_WORDS(P.hsum_wgs);
    const size_t l_sh = shrink_lines(s2), l_hs = (size_t)P.hsum_wgs;
    P.ho2 = carve_handoff(cv, w_sh > w_hs ? w_sh : w_hs, fused_flag_words(&g2, 1), l_sh > l_hs ? l_sh : l_hs);
  }
  P.bytes = cv.b.off + 256;
  P.ctr = cv.coff + 64;
  P.flg = cv.foff + 64;
}


/* ---- prefill (T > 32 tokens) ---- */

/* Plan of one prefill chunk: the group plan (token order, tile unions, coefficients, pointer
 * tables), then per module set a tile shrink and the GEMMs that consume it. lora is false when no
 * bound adapter has any of the call's modules: the GEMMs then run in token order with no plan. */
struct PrefillPlan {
  aos_gplan_params gp;
  int mtiles = 0, tu_cap = 1;
  bool lora = false;
};

/* Group plan of one prefill call; tabs are the modules (in the order of the call's GEMMs) whose
 * A and B pointers the plan tabulates. */
static void plan_prefill_common(aoship_layer *l, Carve &cv, const aoship_ring_t *rings, int T,
                                const aos_lora_tab *tabs, int nm, PrefillPlan &P) {
  const int n = (int)l->table.size();
  P.mtiles = ceil_div(T, AOS_GEMM_BM);
  P.tu_cap = n < AOS_TILE_U_MAX ? (n > 0 ? n : 1) : AOS_TILE_U_MAX;
  P.lora = false;
  for (int i = 0; i < nm; ++i) P.lora = P.lora || (tabs[i].rpad > 0 && n > 0);
  aos_gplan_params &gp = P.gp;
  memset(&gp, 0, sizeof(gp));
  if (!P.lora) return;
  gp.rings = rings;
  gp.T = T;
  gp.n = n;
  gp.bound = l->bound.as<uint8_t>();
  gp.scale = l->scale_all.as<float>();
  gp.tu_cap = P.tu_cap;
  gp.perm = cv.b.take<uint16_t>((size_t)T);
  gp.tu = cv.b.take<int>((size_t)P.mtiles);
  gp.list = cv.b.take<uint16_t>((size_t)P.mtiles * P.tu_cap);
  gp.coef = cv.b.take<float>((size_t)T * P.tu_cap);
  gp.nmod = nm;
  for (int i = 0; i < nm; ++i) gp.tab[i] = tabs[i];
  gp.ap = cv.b.take<const uint16_t *>((size_t)nm * P.mtiles * P.tu_cap);
  gp.bp = cv.b.take<const uint16_t *>((size_t)nm * P.mtiles * P.tu_cap);
}

/* Tile shrink over modules [m0, m0 + nm) of the plan (sharing x, whose rows are read through perm,
 * or in sorted order when perm is NULL). K slices: about 512 workgroups over the tiles, at least 8
 * groups a slice, at most 16 slices, and the slices' partial sums within 128 MiB. fused: the
 * shrink runs in the consuming GEMM launch instead (see fuse_shrink): only the SA layout and
 * buffer are planned. */
static void plan_tshrink(aoship_layer *l, Carve &cv, const PrefillPlan &P, const uint16_t *x, const uint16_t *perm,
                         int T, int in, int m0, int nm, aos_tshrink_params &sp, bool fused = false) {
  memset(&sp, 0, sizeof(sp));
  if (!P.lora) return;
  sp.x = x;
  sp.perm = perm;
  sp.T = T;
  sp.in = in;
  sp.nmod = nm;
  int cols = 0;
  for (int i = 0; i < nm; ++i) {
    sp.rpad[i] = P.gp.tab[m0 + i].rpad;
    cols += P.tu_cap * sp.rpad[i];
  }
  if (cols == 0) {
    sp.nmod = 0; /* nothing to shrink: no launch */
    return;
  }
  sp.tu = P.gp.tu;
  sp.coef = P.gp.coef;
  sp.tu_cap = P.tu_cap;
  sp.ap = P.gp.ap ? P.gp.ap + (size_t)m0 * P.mtiles * P.tu_cap : nullptr;
  sp.mtiles = P.mtiles;
  sp.s_stride = ceil_div(cols, 64) * 64;
  sp.csets = ceil_div(cols, 128);
  if (fused) {
    sp.SA = cv.b.take<uint16_t>((size_t)T * sp.s_stride);
    sp.zero_row = l->zeros.as<uint16_t>();
    sp.timeout = l->wait_dev;
    return;
  }
  const int G = in / 64;
  int ks = ceil_div(512, P.mtiles);
  if (ks > 16) ks = 16;
  if (ks > G / 8) ks = G / 8;
  if (ks < 1) ks = 1;
  /* the slices' partial sums (sized for the widest union on every tile) within 512 MB: on the
   * 32B-shaped layer at 4096 tokens (64 rank-64 adapters) the h shrink takes 8 slices (0.94 ms;
   * 2 slices under a 128 MB bound, 1.1 ms; 16 slices, 1.13 ms: the partials' own traffic) and the
   * x shrink 4 (no change against 1; 8 slices, 0.64 against 0.42 ms) */
  while (ks > 1 && (size_t)P.mtiles * ks * AOS_GEMM_BM * sp.s_stride * 4 > ((size_t)512 << 20)) --ks;
  sp.ks = ks;
  sp.part = cv.b.take<float>((size_t)P.mtiles * ks * AOS_GEMM_BM * sp.s_stride);
  sp.counters = cv.counters((size_t)P.mtiles * sp.csets);
  sp.flags = cv.flag_lines((size_t)P.mtiles * sp.csets * 32);
  sp.SA = cv.b.take<uint16_t>((size_t)T * sp.s_stride);
  sp.zero_row = l->zeros.as<uint16_t>();
  sp.timeout = l->wait_dev;
}

/* GEMM of matrix W0 (module mod0 of the plan's tables) or, in SwiGLU mode, W0 and W1 (module
 * mod0 + 1), its expand reading the shrink sp's columns: nbefore modules of sp come before mod0's. */
static void plan_gemm(aoship_layer *l, const PrefillPlan &P, const aos_tshrink_params &sp, const Q4Mat &W0,
                      const Q4Mat *W1, const uint16_t *x, const uint16_t *in_perm, const uint16_t *out_perm, int T,
                      int mod0, int nbefore, uint16_t *y, aos_gemm_params &g) {
  memset(&g, 0, sizeof(g));
  g.w0 = W0.dev();
  if (W1) g.w1 = W1->dev();
  g.x = x;
  g.T = T;
  g.y = y;
  g.zero = l->zeros.as<uint16_t>();
  g.mtiles = P.mtiles;
  g.tu_cap = P.tu_cap;
  if (!P.lora || sp.nmod == 0) return; /* token order, no expand */
  g.in_perm = in_perm;
  g.out_perm = out_perm;
  g.rpad0 = P.gp.tab[mod0].rpad;
  g.rpad1 = W1 ? P.gp.tab[mod0 + 1].rpad : 0;
  g.mod0 = mod0;
  g.tu = P.gp.tu;
  g.bp = P.gp.bp;
  g.SA = sp.SA;
  g.sa_stride = sp.s_stride;
  g.sa_mod_before = nbefore;
  for (int i = 0; i < nbefore && i < 2; ++i) g.rpad_before[i] = sp.rpad[i];
}

/* The shrink sp (planned with fused = true) as the first workgroups of GEMM g, over g's modules
 * (mod0, and mod0 + 1 in SwiGLU mode, the first modules of sp). */
static void fuse_shrink(aoship_layer *l, Carve &cv, const PrefillPlan &P, const aos_tshrink_params &sp,
                        aos_gemm_params &g) {
  if (!P.lora || sp.nmod == 0) return;
  const int c0 = P.tu_cap * g.rpad0, c1 = P.tu_cap * g.rpad1;
  g.s_cols = c0 > c1 ? c0 : c1;
  if (g.s_cols == 0) return;
  g.ap = P.gp.ap;
  g.coef = P.gp.coef;
  g.sa_out = sp.SA;
  g.sa_ctr = cv.counters((size_t)P.mtiles);
  g.sa_lines = cv.flag_lines((size_t)P.mtiles * 32);
  g.timeout = l->wait_dev;
}

/* Stream-K for GEMM g (planned): its partial-sum slots and lines from the workspace, when
 *  - the launch carries no shrink workgroups: those fill the plain grid's last round, and stream-K
 *    over the slots they leave was slower (7B-shaped layer, 2048 tokens: gate/up 643 us against
 *    562 us, down 323 us against 309 us);
 *  - the plain grid's last round leaves at least a tenth of the resident set idle (what stream-K
 *    wins back: 4096 tokens, gate/up 5.53 ms against 5.68 ms, down 1.59 ms against 1.67 ms);
 *  - every workgroup gets at least AOS_SK_MIN_GROUPS K groups. */
#define AOS_SK_MIN_GROUPS 16
static void plan_sk(aoship_layer *l, Carve &cv, aos_gemm_params &g, bool swiglu) {
  g.sk_nwg = 0;
  if (!(l->prefill_sk & (swiglu ? 1 : 2)) || g.s_cols > 0) return;
  const int wv = swiglu ? 4 : 8; /* the kernel shape's waves per workgroup */
  const int slots = aos_gemm_sk_slots(swiglu ? 1 : 0) & ~7; /* one share per XCD */
  if (slots <= 0) return;
  const int mb = (g.T + AOS_GEMM_BM - 1) / AOS_GEMM_BM;
  /* with a multiple of 8 token tiles the SwiGLU GEMM's plain grid gives each XCD its own tiles
   * (interleaved), which balances tiles whose adapter unions differ in size; stream-K's equal shares
   * of K groups do not (a tile's expand steps fall to whichever workgroup ends its tasks). The down
   * GEMM's expand is a small part of its K (rank-64 unions of up to 64 adapters against 27648
   * weight columns on the 32B-shaped layer), and there stream-K wins back its last plain round:
   * 1.575 -> 1.434 ms at 4096 tokens */
  if (mb % 8 == 0 && swiglu) return;
  const uint64_t tasks = (uint64_t)mb * ((g.w0.RB + wv - 1) / wv);
  const uint64_t last = tasks % (uint64_t)slots; /* workgroups of the plain grid's last round */
  if (last == 0 || last * 10 >= (uint64_t)slots * 9) return;
  const uint64_t total = tasks * (uint64_t)g.w0.G;
  if (total / (uint64_t)slots < AOS_SK_MIN_GROUPS || total * (uint64_t)slots >= (1ull << 32)) return;
  g.sk_nwg = slots;
  g.sk_part = cv.b.take<float>((size_t)slots * aos_gemm_sk_slot_floats(swiglu ? 1 : 0));
  g.sk_lines = cv.flag_lines((size_t)slots * 32);
  g.timeout = l->wait_dev;
}

/* The adapter-major shrink of sp (modules m0 .. of the plan's tables) over the users that plan A
 * lists: K slices for about 1024 workgroups, at least 8 groups a slice, at most 16 slices, and
 * the slices' partial sums within 256 MB. */
static void plan_amshrink(Carve &cv, const PrefillPlan &P, const aos_tshrink_params &sp, int m0,
                          const aos_amplan_params &A, aos_amshrink_params &q) {
  memset(&q, 0, sizeof(q));
  q.x = sp.x;
  q.perm = sp.perm;
  q.T = sp.T;
  q.in = sp.in;
  q.nmod = sp.nmod;
  q.tu_cap = sp.tu_cap;
  int cw = 0;
  for (int i = 0; i < sp.nmod; ++i) {
    q.rpad[i] = sp.rpad[i];
    q.A[i] = P.gp.tab[m0 + i].A;
    cw += sp.rpad[i];
  }
  q.tu = sp.tu;
  q.coef = sp.coef;
  q.ctab = A.ctab;
  q.users = A.users;
  q.SA = sp.SA;
  q.s_stride = sp.s_stride;
  q.zero_row = sp.zero_row;
  q.cb = A.cb;
  q.setw = cw <= 64 ? 64 : 128; /* 2-wave workgroups for adapters of 64 columns or fewer */
  q.csets = ceil_div(cw, q.setw);
  const int G = sp.in / 64;
  int ks = ceil_div(1024, q.cb * q.csets);
  if (ks > 16) ks = 16;
  if (ks > G / 8) ks = G / 8;
  if (ks < 1) ks = 1;
  while (ks > 1 && (size_t)ks * q.cb * q.csets * AOS_GEMM_BM * 128 * 4 > ((size_t)256 << 20)) --ks;
  q.ks = ks;
  q.part = ks > 1 ? cv.b.take<float>((size_t)ks * q.cb * q.csets * AOS_GEMM_BM * 128) : nullptr;
}

/* A shrink that can run adapter-major: a launch of its own, every module present. */
static bool am_fits(const aos_tshrink_params &sp, bool fused) {
  if (fused || sp.nmod == 0) return false;
  for (int i = 0; i < sp.nmod; ++i)
    if (sp.rpad[i] < 16) return false;
  return true;
}

struct MlpPrefill {
  PrefillPlan P;
  aos_tshrink_params sx, sh;
  aos_amplan_params amp;
  aos_amshrink_params amx, amh;
  aos_amx_params ame;
  bool use_am_x = false, use_am_h = false; /* the x / h shrink's wide-union tiles run adapter-major */
  bool use_xam = false;                    /* ... and the gate/up expand of the widest */
  aos_gemm_params g1, g2;
  aos_xexp_params xe;
  bool fused_x = false, fused_h = false; /* the x / h shrink runs in the GEMM launch */
  bool use_xe = false;                   /* the gate/up expand launch runs (wide unions) */
  size_t bytes = 0, ctr = 0, flg = 0;
};

static void plan_mlp_prefill(aoship_layer *l, int T, const uint16_t *x, const aoship_ring_t *rings, uint16_t *y,
                             void *ws, void *ctr, void *flg, MlpPrefill &M) {
  const Q4Mat &Wg = l->mats[MOD_GATE], &Wu = l->mats[MOD_UP], &Wd = l->mats[MOD_DOWN];
  const int H = Wg.in, I = Wg.out;
  Carve cv(ws, ctr, flg);
  const aos_lora_tab tall[3] = {lora_tab(l, MOD_GATE, H, I), lora_tab(l, MOD_UP, H, I), lora_tab(l, MOD_DOWN, I, H)};
  plan_prefill_common(l, cv, rings, T, tall, 3, M.P);
  uint16_t *h = cv.b.take<uint16_t>((size_t)T * I); /* sorted rows when grouped */
  const uint16_t *perm = M.P.lora ? M.P.gp.perm : nullptr;
  /* each shrink in its GEMM's launch when its workgroups fit in the idle slots of that grid's
   * last round, else a launch of its own (K split into slices) */
  M.fused_x = M.fused_h = false;
  if (M.P.lora && l->prefill_fused_shrink) {
    const int tc = M.P.tu_cap, rg = tall[0].rpad, ru = tall[1].rpad, rd = tall[2].rpad;
    M.fused_x = aos_gemm_shrink_fits(T, Wg.RB, tc * (rg > ru ? rg : ru), 1) != 0;
    M.fused_h = aos_gemm_shrink_fits(T, Wd.RB, tc * rd, 0) != 0;
  }
  plan_tshrink(l, cv, M.P, x, perm, T, H, 0, 2, M.sx, M.fused_x);
  plan_gemm(l, M.P, M.sx, Wg, &Wu, x, perm, nullptr, T, 0, 0, h, M.g1);
  plan_tshrink(l, cv, M.P, h, nullptr, T, I, 2, 1, M.sh, M.fused_h);
  plan_gemm(l, M.P, M.sh, Wd, nullptr, h, nullptr, perm, T, 2, 0, y, M.g2);
  if (M.fused_x) fuse_shrink(l, cv, M.P, M.sx, M.g1);
  if (M.fused_h) fuse_shrink(l, cv, M.P, M.sh, M.g2);
  plan_sk(l, cv, M.g1, true);
  plan_sk(l, cv, M.g2, false);
  /* the tiles whose union holds at least prefill_am_tu adapters: their shrinks adapter-major */
  const int n = (int)l->table.size();
  M.use_am_x = M.use_am_h = false;
  if (M.P.lora && l->prefill_am_tu > 0 && n <= AOS_AM_MAX_N && M.P.tu_cap >= l->prefill_am_tu) {
    M.use_am_x = am_fits(M.sx, M.fused_x);
    M.use_am_h = am_fits(M.sh, M.fused_h);
  }
  if (M.use_am_x || M.use_am_h) {
    aos_amplan_params &A = M.amp;
    memset(&A, 0, sizeof(A));
    A.T = T;
    A.n = n;
    A.tu_cap = M.P.tu_cap;
    A.cb = ceil_div(8 * T, AOS_GEMM_BM) + n;
    A.am_tu = l->prefill_am_tu;
    A.tu = M.P.gp.tu;
    A.list = M.P.gp.list;
    A.coef = M.P.gp.coef;
    A.count = cv.counters((size_t)n);
    A.done = cv.counters(1);
    A.ctab = cv.b.take<uint32_t>((size_t)A.cb);
    A.users = cv.b.take<uint32_t>((size_t)n * T);
    aos_tshrink_params *sps[2] = {&M.sx, &M.sh};
    const bool on[2] = {M.use_am_x, M.use_am_h};
    for (int k = 0; k < 2; ++k) {
      if (!on[k]) continue;
      aos_tshrink_params &sp = *sps[k];
      aos_am_zero &z = A.zb[A.nz++];
      z.SA = sp.SA;
      z.s_stride = sp.s_stride;
      z.nmod = sp.nmod;
      for (int i = 0; i < sp.nmod; ++i) z.rpad[i] = sp.rpad[i];
      sp.am_tu = A.am_tu;
      plan_amshrink(cv, M.P, sp, k == 0 ? 0 : 2, A, k == 0 ? M.amx : M.amh);
    }
  }
  if (M.P.lora && M.sh.nmod == 0) M.g2.out_perm = perm; /* h is in sorted order even without a down expand */
  if (M.P.lora && M.sx.nmod == 0) M.g1.in_perm = perm;
  /* the gate/up expand of wide tile unions in a launch of its own (the SwiGLU GEMM holds both
   * modules' accumulators, which leaves no registers to pipeline an expand step's B fragments; the
   * expand launch, one module per wave, runs the pipelined expand), when some tile could reach
   * the width and the x shrink is a launch of its own (the expand reads its SA) */
  M.use_xe = false;
  const int rxe = M.g1.rpad0 > M.g1.rpad1 ? M.g1.rpad0 : M.g1.rpad1;
  if (M.P.lora && !M.fused_x && M.sx.nmod && rxe > 0 && l->prefill_xe_cols > 0 &&
      M.P.tu_cap * rxe >= l->prefill_xe_cols) {
    float *xd = cv.b.take<float>((size_t)2 * M.P.mtiles * Wg.RB * AOS_GEMM_BM * 32);
    M.g1.xd = xd;
    M.g1.xe_cols = l->prefill_xe_cols;
    aos_xexp_params &X = M.xe;
    memset(&X, 0, sizeof(X));
    X.g[0] = M.g1;
    X.g[0].rpad1 = 0;
    X.g[1] = M.g1;
    X.g[1].mod0 = M.g1.mod0 + 1;
    X.g[1].rpad0 = M.g1.rpad1;
    X.g[1].rpad1 = 0;
    X.g[1].sa_mod_before = M.g1.sa_mod_before + 1;
    if (M.g1.sa_mod_before < 2) X.g[1].rpad_before[M.g1.sa_mod_before] = M.g1.rpad0;
    X.xd = xd;
    X.xe_cols = l->prefill_xe_cols;
    X.rmax = rxe;
    M.use_xe = true;
  }
  /* the tiles whose union holds at least prefill_xam_tu adapters (a subset of the expand launch's
   * and of the adapter-major shrinks' tiles): their gate/up expand adapter-major */
  M.use_xam = false;
  const int xt = l->prefill_xam_tu;
  if (M.use_xe && M.use_am_x && n <= AOS_XAM_MAX_N && xt > 0 && xt >= l->prefill_am_tu &&
      xt * rxe >= l->prefill_xe_cols && M.P.tu_cap >= xt && M.g1.rpad0 >= 16 && M.g1.rpad0 <= 64 &&
      M.g1.rpad1 == M.g1.rpad0) {
    aos_amplan_params &A = M.amp;
    A.tinfo = cv.b.take<uint32_t>((size_t)M.P.mtiles * M.P.tu_cap);
    A.inv = cv.b.take<uint16_t>((size_t)M.P.mtiles * n);
    A.xl = cv.b.take<uint32_t>((size_t)M.P.mtiles + 1);
    A.xam_tu = xt;
    aos_amx_params &Q = M.ame;
    memset(&Q, 0, sizeof(Q));
    Q.T = T;
    Q.n = n;
    Q.tu_cap = M.P.tu_cap;
    Q.mtiles = M.P.mtiles;
    Q.RB = Wg.RB;
    Q.tu = M.P.gp.tu;
    Q.tinfo = A.tinfo;
    Q.inv = A.inv;
    Q.xl = A.xl;
    Q.users = A.users;
    const int ranges = ceil_div(M.P.mtiles, AOS_XAM_RT);
    Q.rlp = cv.b.take<uint16_t>((size_t)ranges * AOS_XAM_CT * AOS_GEMM_BM);
    Q.ct = cv.b.take<uint32_t>((size_t)ranges * AOS_XAM_CT);
    Q.nch = cv.b.take<uint32_t>((size_t)ranges);
    Q.cidx = cv.b.take<uint32_t>((size_t)n * T);
    Q.SAc = cv.b.take<uint16_t>((size_t)ranges * AOS_XAM_RT * AOS_GEMM_BM * 8 * (M.g1.rpad0 + M.g1.rpad1));
    M.amx.cidx = Q.cidx;
    M.amx.SAc = (uint16_t *)Q.SAc;
    M.amx.xam_tu = xt;
    Q.rpad[0] = M.g1.rpad0;
    Q.rpad[1] = M.g1.rpad1;
    Q.Bf[0] = M.P.gp.tab[0].Bf;
    Q.Bf[1] = M.P.gp.tab[1].Bf;
    Q.zero = l->zeros.as<uint16_t>();
    Q.xd = M.xe.xd;
    M.xe.xam_tu = xt;
    M.use_xam = true;
  }
  M.bytes = cv.b.off + 256;
  M.ctr = cv.coff + 64;
  M.flg = cv.foff + 64;
}

static int launch_err(int e, const char *what);

/* Launch the group plan (nothing without adapters). */
static int launch_gplan(aoship_layer *l, const PrefillPlan &P) {
  if (!P.lora) return 0;
  aos_launch_ctx c0 = launch_ctx(l, KS_PPLAN);
  return launch_err(aos_launch_gplan(&P.gp, &c0), "prefill group plan");
}

/* Launch a tile shrink (nothing when no bound adapter has its modules) with a new generation for
 * its meeting flags. */
static int launch_tshrink(aoship_layer *l, const aos_tshrink_params &sp, int slot) {
  if (sp.nmod == 0) return 0;
  aos_launch_ctx c0 = launch_ctx(l, slot);
  aos_tshrink_params q = sp;
  q.gen = next_gen(&l->gen);
  return launch_err(aos_launch_tshrink(&q, &c0), "lora shrink (prefill)");
}

/* Launch an adapter-major shrink and, with its K split, the sum of its slices (slot + 1). */
static int launch_amshrink(aoship_layer *l, const aos_amshrink_params &q, int slot) {
  aos_launch_ctx c0 = launch_ctx(l, slot);
  if (launch_err(aos_launch_amshrink(&q, &c0), "lora adapter-major shrink (prefill)")) return -1;
  if (q.ks < 2) return 0;
  aos_amshrink_params r = q;
  r.reduce = 1;
  aos_launch_ctx c1 = launch_ctx(l, slot + 1);
  return launch_err(aos_launch_amshrink(&r, &c1), "lora adapter-major shrink sum (prefill)");
}

static int chunk_prefill_t(int T) { return T < AOS_PREFILL_MAX_T ? T : AOS_PREFILL_MAX_T; }

static void size_proj(aoship_layer *l, const int *mods, int nm, int max_tokens, size_t &bytes, size_t &ctr,
                      size_t &flg);

static size_t mlp1_flag_words(aoship_layer *l);

extern "C" int aoship_layer_reserve(aoship_layer_t *l, int max_tokens) {
  if (!l) return set_err("aoship_layer_reserve: null layer");
  if (max_tokens < 1) return set_err("aoship_layer_reserve: max_tokens must be >= 1");
  if (ensure_device()) return -1;
  size_t bytes = 0, ctr = 0, flg = 0;
  const bool mlp = l->mats[MOD_GATE].valid && l->mats[MOD_UP].valid && l->mats[MOD_DOWN].valid;
  for (int T = 1; T <= AOS_DECODE_MAX_T && T <= max_tokens; ++T) {
    if (mlp) {
      MlpPlan P;
      plan_mlp(l, T, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, P);
      if (P.bytes > bytes) bytes = P.bytes;
      if (P.ctr > ctr) ctr = P.ctr;
      if (P.flg > flg) flg = P.flg;
    }
  }
  if (mlp) { /* the one-token launch's tagged words */
    const size_t fw = mlp1_flag_words(l);
    if (fw > flg) flg = fw;
  }
  if (mlp && max_tokens > AOS_DECODE_MAX_T) {
    MlpPrefill M;
    plan_mlp_prefill(l, chunk_prefill_t(max_tokens), nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, M);
    if (M.bytes > bytes) bytes = M.bytes;
    if (M.ctr > ctr) ctr = M.ctr;
    if (M.flg > flg) flg = M.flg;
  }
  /* the projections: q, k and v together (aoship_qkv_forward) and each one alone */
  const int qkv[3] = {MOD_Q, MOD_K, MOD_V};
  if (l->mats[MOD_Q].valid && l->mats[MOD_K].valid && l->mats[MOD_V].valid && l->mats[MOD_K].in == l->mats[MOD_Q].in &&
      l->mats[MOD_V].in == l->mats[MOD_Q].in)
    size_proj(l, qkv, 3, max_tokens, bytes, ctr, flg);
  for (int m = MOD_Q; m <= MOD_O; ++m)
    if (l->mats[m].valid) size_proj(l, &m, 1, max_tokens, bytes, ctr, flg);
  return ws_reserve(l, bytes, ctr, flg);
}

static int check_common(aoship_layer *l, const void *x, int T, const aoship_ring_t *rings,
                        const void *y) {
  if (!l) return set_err("forward: null layer");
  if (!x || !y || !rings) return set_err("forward: null device pointer");
  if (!aligned16(x) || !aligned16(y)) return set_err("forward: x and y must be 16-byte aligned");
  if (T < 0) return set_err("forward: negative token count");
  if (check_no_timeout(l)) return -1;
  return ensure_device();
}

static int launch_err(int e, const char *what) {
  if (e == 0) return 0;
  return set_err(std::string(what) + ": " + hipGetErrorString((hipError_t)e));
}

static int launch_x_shrink(aoship_layer *l, XShrink &xs, bool events = true) {
  if (xs.separate_plan) {
    aos_launch_ctx c0 = launch_ctx(l, KS_SHRINK_X, events);
    if (launch_err(aos_launch_shrink(&xs.plan_only, &c0), "adapter plan")) return -1;
  }
  aos_launch_ctx c1 = launch_ctx(l, KS_SHRINK_X, events);
  return launch_err(aos_launch_shrink(&xs.sp, &c1), "lora shrink");
}

/* A decode shrink and the GEMV that reads its S fused into one launch (the shrink's workgroups
 * first), unless the layer is set to separate launches of the same device code (same results
 * within tolerance). */
static bool fuse_shrinks(const aoship_layer *l) { return !l->separate_shrinks; }


/* Producers of a fused launch hand over through a line each (polled by every consumer) up to this
 * many lines, else through an arrival count and one ready flag per consumer. */
#define AOS_LINES_MAX 512

static void make_fused(aoship_layer *l, uint32_t *genc, const aos_shrink_params &sp, const aos_gemv_params *gp, int n,
                       const Handoff &ho, const aos_hsum_params *hs, aos_gemv_fused_params &f) {
  uint32_t *sync = ho.sync, *flags = ho.flags;
  memset(&f, 0, sizeof(f));
  if (hs) { /* the first workgroups sum the h shrink's partials instead of running a shrink */
    f.hsum = 1;
    f.hs = *hs;
    f.n_pre = ceil_div(hs->T * hs->stride, AOS_HSUM_V);
    f.pre_rows = f.n_pre;
  } else {
    f.sp = sp;
    f.pre_rows = sp.n_rb[0] + (sp.nmod > 1 ? sp.n_rb[1] : 0) + (sp.nmod > 2 ? sp.n_rb[2] : 0) +
                 (sp.plan_build.plan ? 1 : 0);
    f.n_pre = f.pre_rows * sp.ks;
  }
  f.n = n;
  f.sync = sync;          /* AOS_ARRIVE_WORDS(n_pre) words from a line of their own */
  f.flags = flags;
  f.gen = next_gen(genc);
  int end = 0;
  for (int i = 0; i < 3; ++i) {
    if (i < n) {
      f.gp[i] = gp[i];
      f.gp[i].sync = f.sync;
      f.gp[i].flags = f.flags + (size_t)end * 32;
      f.gp[i].sync_target = (uint32_t)f.n_pre;
      f.gp[i].gen = f.gen;
      f.gp[i].timeout = l->wait_dev;
      end += gp[i].nrbg * gp[i].ks;
    }
    f.wg_end[i] = end;
  }
  f.n_cons = (uint32_t)end;
  const int n_lines = hs ? f.n_pre : f.pre_rows;
  if (ho.lines && l->producer_lines && n_lines <= AOS_LINES_MAX) { /* per-producer lines instead of the count */
    f.lines = ho.lines;
    f.n_lines = n_lines;
    f.sync = nullptr;
    f.flags = nullptr;
    if (hs) {
      f.hs.lines = ho.lines;
      f.hs.gen = f.gen;
    } else {
      f.sp.lines = ho.lines;
      f.sp.gen = f.gen;
    }
    const int plan_line = (!hs && sp.plan_build.plan) ? f.pre_rows - 1 : -1;
    for (int i = 0; i < n; ++i) {
      f.gp[i].sync = nullptr;
      f.gp[i].flags = nullptr;
      f.gp[i].sync_target = 0;
      f.gp[i].pre_lines = ho.lines;
      f.gp[i].n_pre_lines = n_lines;
      f.gp[i].plan_line = plan_line;
    }
  }
}

static int launch_fused(aoship_layer *l, const Ws &w, const aos_shrink_params &sp, const aos_gemv_params *gp, int n,
                        const Handoff &ho, int swiglu, int slot, const char *what,
                        const aos_hsum_params *hs = nullptr) {
  aos_gemv_fused_params f;
  make_fused(l, w.gen, sp, gp, n, ho, hs, f);
  aos_launch_ctx c = launch_ctx(l, slot, w.events);
  return launch_err(aos_launch_gemv_fused(&f, swiglu, &c), what);
}

/* ---- the one-token MLP launch (aoship_mlp1.hip) ---- */

static int g_cu_count[AOS_MAX_DEVICES];

static int device_cus() {
  if (g_device < 0 || g_device >= AOS_MAX_DEVICES) return 0;
  if (!g_cu_count[g_device]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, g_device) != hipSuccess) return 0;
    g_cu_count[g_device] = n;
  }
  return g_cu_count[g_device];
}

#define AOS_MLP1_STATIC_LDS 2048 /* the kernel's static LDS (the router's selection arrays, flags), at most */

/* Whether the one-token launch applies to this layer (its shape fits the LDS of two workgroups per
 * CU, at most AOS_MLP1_MAXN adapters of rank <= AOS_MLP1_MAXR, the plain router when rp is set) and
 * its parameters; flags == nullptr sizes its tagged words (flag_words, 32-bit words of the layer's
 * flag memory). */
static bool plan_mlp1(aoship_layer *l, const aos_route_params *rp, const uint16_t *x, const aoship_ring_t *ring,
                      uint16_t *y, void *flags, aos_mlp1_params &q, size_t &flag_words) {
  memset(&q, 0, sizeof(q));
  flag_words = 0;
  if (!l->mlp1 || l->separate_shrinks || l->one_launch_mlp || !l->producer_lines) return false;
  const Q4Mat &Wg = l->mats[MOD_GATE], &Wu = l->mats[MOD_UP], &Wd = l->mats[MOD_DOWN];
  const int H = Wg.in, I = Wg.out;
  const int cus = device_cus();
  if (cus <= 0) return false;
  const int nwg = 2 * cus;
  const long UG = (long)Wg.RB * Wg.G, UD = (long)Wd.RB * Wd.G;
  /* the kernel forms unit indices and share bounds (units x waves) in 32 bits */
  if (UG * 4L * nwg >= (1L << 32) || UD * (long)nwg >= (1L << 32)) return false;
  if ((UG + 4L * nwg - 1) / (4L * nwg) > Wg.G) return false; /* a G wave spans at most two row blocks */
  const int dmax = (int)((UD + nwg - 1) / nwg);
  const int dwave = (dmax + 3) / 4;
  if (dwave > AOS_MLP1_MAX_DU || dwave > Wd.G) return false;
  const int slots = Wg.G > dmax ? Wg.G : dmax;
  const int doff = ((128 + slots * 136) + 255) & ~255;
  const int lds = doff + dmax * 1024;
  if (lds + AOS_MLP1_STATIC_LDS > AOS_MLP1_LDS_MAX) return false;
  const int n = (int)l->table.size();
  const aos_lora_tab tg = lora_tab(l, MOD_GATE, H, I), tu = lora_tab(l, MOD_UP, H, I), td = lora_tab(l, MOD_DOWN, I, H);
  if (n > AOS_MLP1_MAXN || tg.rpad > AOS_MLP1_MAXR || tu.rpad > AOS_MLP1_MAXR || td.rpad > AOS_MLP1_MAXR) return false;
  if (rp && (rp->T != 1 || rp->n < 1 || rp->n > AOS_MLP1_MAXN || rp->d < 4 || rp->d % 4 || rp->scope || rp->tie_key ||
             rp->post_allowed || rp->active_ids || rp->strengths || rp->hashes || rp->decisions))
    return false;
  const int tiles_g = (n * tg.rpad + 31) / 32, tiles_u = (n * tu.rpad + 31) / 32;
  const int rw4 = rp ? (rp->n + 3) / 4 * 4 : 0;
  const int avail = 4 * nwg - rw4, tiles = tiles_g + tiles_u;
  /* K pieces per x-shrink tile: at most two groups per wave (one round of loads), at most half the
   * D waves (the rest expand gate/up row blocks) */
  int ks = tiles ? avail / 2 / tiles : 1;
  if (ks > (Wg.G + 1) / 2) ks = (Wg.G + 1) / 2;
  if (ks < 1) return false;
  if (4 * nwg - rw4 - tiles * ks < Wg.RB) return false; /* one D wave per gate/up row block's expand */
  const int hc = 8 * td.rpad;
  if (hc > nwg) return false;
  Bump b(flags, (size_t)-1);
  q.gpart = b.take<uint64_t>((size_t)4 * nwg * 64);
  q.dpart = b.take<uint64_t>((size_t)4 * nwg * 32);
  q.htag = b.take<uint64_t>((size_t)I);
  q.hpart = b.take<uint64_t>((size_t)Wg.RB * (hc ? hc : 1));
  q.ex = b.take<uint64_t>((size_t)Wg.RB * 64);
  q.sh = b.take<uint64_t>((size_t)(hc ? hc : 1));
  q.spart = b.take<uint64_t>((size_t)(tiles ? tiles : 1) * ks * 32);
  q.sx = b.take<uint64_t>((size_t)(n ? n : 1) * (tg.rpad + tu.rpad + 1));
  q.pri = b.take<uint64_t>(AOS_MLP1_MAXN);
  q.ringt = b.take<uint64_t>(16);
  flag_words = (b.off + 255) / 4;
  q.wg = Wg.dev();
  q.wu = Wu.dev();
  q.wd = Wd.dev();
  q.x = x;
  q.y = y;
  q.ring_in = ring;
  if (rp) {
    q.route = 1;
    q.rp = *rp;
  }
  q.n = n;
  q.bound = l->bound.as<const uint8_t>();
  q.scale = l->scale_all.as<const float>();
  q.tg = tg;
  q.tu = tu;
  q.td = td;
  q.zero_row = l->zeros.as<uint16_t>();
  q.nwg = nwg;
  q.d_units_max = dmax;
  q.doff = doff;
  q.lds_bytes = lds;
  q.x_tiles_g = tiles_g;
  q.x_tiles_u = tiles_u;
  q.x_ks = ks;
  q.hc = hc;
  q.timeout = l->wait_dev;
  return true;
}

static size_t mlp1_flag_words(aoship_layer *l) {
  aos_mlp1_params q;
  size_t fw = 0;
  aos_route_params rp;
  memset(&rp, 0, sizeof(rp));
  rp.T = 1;
  rp.n = AOS_MLP1_MAXN;
  rp.d = 4;
  /* the largest size: with the router's waves taken */
  if (!plan_mlp1(l, &rp, nullptr, nullptr, nullptr, nullptr, q, fw)) plan_mlp1(l, nullptr, nullptr, nullptr, nullptr, nullptr, q, fw);
  return fw;
}

/* One token through the one-launch MLP, when it applies: 1 launched, 0 not applicable, -1 error.
 * scratch: the allocation-free forward's memory (its tagged words in the scratch's flag region,
 * which must hold them; no profiling events), else the layer's own flag memory. */
static int mlp1_forward(aoship_layer *l, const uint16_t *x, const aoship_ring_t *ring, uint16_t *y,
                        const aos_route_params *rp, const Ws *scratch) {
  aos_mlp1_params q;
  size_t fw = 0;
  if (!plan_mlp1(l, rp, nullptr, nullptr, nullptr, nullptr, q, fw)) return 0;
  void *flags = nullptr;
  uint32_t *genc = &l->gen;
  if (scratch) {
    if (fw * 4 > AOS_SCRATCH_FLAG_BYTES) return 0;
    flags = scratch->flg;
    genc = scratch->gen;
  } else {
    if (ws_reserve(l, 0, 0, fw)) return -1;
    flags = l->flags.p;
  }
  plan_mlp1(l, rp, x, ring, y, flags, q, fw);
  q.gen = next_gen(genc);
  aos_launch_ctx c = launch_ctx(l, KS_MLP1, !scratch);
  if (launch_err(aos_launch_mlp1(&q, &c), rp ? "route + decode mlp (one launch)" : "decode mlp (one launch)"))
    return -1;
  return 1;
}

/* One decode chunk (T <= 32 tokens) of the MLP. rp (may be NULL): the plain router's parameters
 * for these tokens, which then run in the gate/up launch (rings written there); the caller has
 * checked that the gate/up launch is fused. */
static int mlp_decode_chunk(aoship_layer *l, int Tc, const uint16_t *x, const aoship_ring_t *rings, uint16_t *y,
                            const aos_route_params *rp, const Ws *scratch = nullptr) {
  if (Tc == 1 && l->mats[MOD_GATE].valid) {
    const int r = mlp1_forward(l, x, rings, y, rp, scratch);
    if (r) return r < 0 ? -1 : 0;
  }
  MlpPlan P;
  Ws w;
  if (scratch) {
    w = *scratch; /* the caller has checked the sizes */
  } else {
    plan_mlp(l, Tc, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, P);
    if (ws_reserve(l, P.bytes, P.ctr, P.flg)) return -1;
    w = {l->ws.p, l->counters.p, l->flags.p, &l->gen, true};
  }
  plan_mlp(l, Tc, x, rings, y, w.ws, w.ctr, w.flg, P);
  const bool fuse = fuse_shrinks(l);
  const bool fuse_down = fuse && P.gv2.has_expand && P.sh.n_rb[0] > 0;
  /* with both launches fused, the gate/up launch also forms the h shrink's partials over its
   * row blocks, and the down launch only sums them */
  const bool h_in_gu = fuse && P.gv1.has_expand && fuse_down && P.hpart; /* 1-2 tokens (measured: slower at 8) */
  const bool route_in_gu = rp && fuse && P.gv1.has_expand && !P.sx.separate_plan;
  if (h_in_gu && !rp && l->one_launch_mlp) { /* 1-2 tokens: the whole MLP in one launch */
    if (P.sx.separate_plan) {
      aos_launch_ctx c0 = launch_ctx(l, KS_SHRINK_X, w.events);
      if (launch_err(aos_launch_shrink(&P.sx.plan_only, &c0), "adapter plan")) return -1;
    }
    aos_gemv_params g1 = P.gv1;
    g1.htab = P.sh.tab[0];
    g1.hpart = P.hpart;
    g1.hstride = P.sh.s_stride[0];
    g1.hdone = P.hdone;
    g1.hflags = P.hflags;
    g1.n_hflags = (uint32_t)(P.hsum_wgs + P.gv2.nrbg * P.gv2.ks);
    aos_hsum_params hs;
    memset(&hs, 0, sizeof(hs));
    hs.hpart = P.hpart;
    hs.RB = P.gv1.w0.RB;
    hs.T = Tc;
    hs.stride = P.sh.s_stride[0];
    hs.rpad = P.sh.tab[0].rpad;
    hs.plan = P.sh.plan;
    hs.S = P.sh.S[0];
    hs.values_per_wg = AOS_HSUM_V;
    hs.coherent = 1;
    aos_decode_mlp_params mp;
    memset(&mp, 0, sizeof(mp));
    make_fused(l, w.gen, P.sx.sp, &g1, 1, P.ho1, nullptr, mp.gu);
    make_fused(l, w.gen, P.sh, &P.gv2, 1, P.ho2, &hs, mp.dn);
    mp.dn.gen = mp.dn.gp[0].gen = mp.gu.gen; /* one generation for the launch */
    if (mp.dn.lines) mp.dn.hs.gen = mp.gu.gen;
    mp.hflags = P.hflags;
    aos_launch_ctx cm = launch_ctx(l, KS_DECODE_MLP, w.events);
    return launch_err(aos_launch_decode_mlp(&mp, &cm), "decode mlp (lora shrink + q4 gemv gate/up + down)");
  }
  if (rp && !route_in_gu) { /* route first, on the layer's stream */
    aos_launch_ctx cr = {l->stream, nullptr, nullptr};
    if (launch_err(aos_launch_route(rp, &cr), "route")) return -1;
  }
  if (route_in_gu) {
    aos_gemv_params g1 = P.gv1;
    if (h_in_gu) {
      g1.htab = P.sh.tab[0];
      g1.hpart = P.hpart;
      g1.hstride = P.sh.s_stride[0];
    }
    aos_route_gu_params q;
    memset(&q, 0, sizeof(q));
    q.rp = *rp;
    make_fused(l, w.gen, P.sx.sp, &g1, 1, P.ho1, nullptr, q.fp);
    q.route_done = P.route_done;
    q.route_flag = P.route_flag;
    /* with up to 64 adapters each token's priors are spread over a workgroup per four adapters */
    q.rparts = rp->n <= AOS_ROUTE_PARTS_MAXN ? (rp->n + 3) / 4 : 1;
    if (q.rparts < 1) q.rparts = 1;
    q.rpart_ctr = P.rpart_ctr;
    q.rpri = P.rpri;
    aos_launch_ctx cg = launch_ctx(l, KS_GEMV_GU, w.events);
    if (launch_err(aos_launch_route_gate_up(&q, &cg), "route + lora shrink + q4 gemv gate/up")) return -1;
  } else if (fuse && P.gv1.has_expand) {
    if (P.sx.separate_plan) {
      aos_launch_ctx c0 = launch_ctx(l, KS_SHRINK_X, w.events);
      if (launch_err(aos_launch_shrink(&P.sx.plan_only, &c0), "adapter plan")) return -1;
    }
    aos_gemv_params g1 = P.gv1;
    if (h_in_gu) {
      g1.htab = P.sh.tab[0];
      g1.hpart = P.hpart;
      g1.hstride = P.sh.s_stride[0];
    }
    if (launch_fused(l, w, P.sx.sp, &g1, 1, P.ho1, 1, KS_GEMV_GU, "lora shrink + q4 gemv gate/up"))
      return -1;
  } else {
    if (launch_x_shrink(l, P.sx, w.events)) return -1;
    aos_launch_ctx c2 = launch_ctx(l, KS_GEMV_GU, w.events);
    if (launch_err(aos_launch_gemv(&P.gv1, 1, &c2), "q4 gemv gate/up")) return -1;
  }
  if (fuse_down) {
    aos_hsum_params hs;
    memset(&hs, 0, sizeof(hs));
    hs.hpart = P.hpart;
    hs.RB = P.gv1.w0.RB;
    hs.T = Tc;
    hs.stride = P.sh.s_stride[0];
    hs.rpad = P.sh.tab[0].rpad;
    hs.plan = P.sh.plan;
    hs.S = P.sh.S[0];
    hs.values_per_wg = AOS_HSUM_V;
    if (launch_fused(l, w, P.sh, &P.gv2, 1, P.ho2, 0, KS_GEMV_DOWN, "lora shrink + q4 gemv down",
                     h_in_gu ? &hs : nullptr))
      return -1;
  } else {
    aos_launch_ctx c3 = launch_ctx(l, KS_SHRINK_H, w.events);
    if (launch_err(aos_launch_shrink(&P.sh, &c3), "lora shrink down")) return -1;
    aos_launch_ctx c4 = launch_ctx(l, KS_GEMV_DOWN, w.events);
    if (launch_err(aos_launch_gemv(&P.gv2, 0, &c4), "q4 gemv down")) return -1;
  }
  return 0;
}

extern "C" int aoship_mlp_forward(aoship_layer_t *l, const aoship_bf16_t *x, int T,
                                  const aoship_ring_t *rings, aoship_bf16_t *y) {
  if (check_common(l, x, T, rings, y)) return -1;
  if (!l->mats[MOD_GATE].valid || !l->mats[MOD_UP].valid || !l->mats[MOD_DOWN].valid)
    return set_err("aoship_mlp_forward: gate_proj, up_proj and down_proj must be set");
  const Q4Mat &Wg = l->mats[MOD_GATE], &Wu = l->mats[MOD_UP], &Wd = l->mats[MOD_DOWN];
  if (Wu.in != Wg.in || Wu.out != Wg.out || Wd.in != Wg.out || Wd.out != Wg.in)
    return set_err("aoship_mlp_forward: gate/up/down shapes are inconsistent");
  const int H = Wg.in;
  if (T > AOS_DECODE_MAX_T) {
    for (int t0 = 0; t0 < T; t0 += AOS_PREFILL_MAX_T) {
      const int Tc = chunk_prefill_t(T - t0);
      MlpPrefill M;
      plan_mlp_prefill(l, Tc, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, M);
      if (ws_reserve(l, M.bytes, M.ctr, M.flg)) return -1;
      plan_mlp_prefill(l, Tc, x + (size_t)t0 * H, rings + t0, y + (size_t)t0 * H, l->ws.p, l->counters.p,
                       l->flags.p, M);
      l->last_perm = M.P.lora ? M.P.gp.perm : nullptr;
      l->last_perm_T = M.P.lora ? Tc : 0;
      if (launch_gplan(l, M.P)) return -1;
      l->last_am = (M.use_am_x ? 1 : 0) | (M.use_am_h ? 2 : 0) | (M.use_xam ? 4 : 0);
      if (M.use_am_x || M.use_am_h) {
        aos_launch_ctx ca = launch_ctx(l, KS_PAMPLAN);
        if (launch_err(aos_launch_amplan(&M.amp, &ca), "lora adapter-major plan (prefill)")) return -1;
      }
      if (M.use_xam) { /* before the x shrink, which writes the compact rows it lists */
        aos_amx_params q = M.ame;
        q.list = 1;
        aos_launch_ctx cl = launch_ctx(l, KS_PXAML);
        if (launch_err(aos_launch_amx(&q, &cl), "lora adapter-major expand lists (prefill)")) return -1;
      }
      if (!M.fused_x && launch_tshrink(l, M.sx, KS_PSHRINK_X)) return -1;
      if (M.use_am_x && launch_amshrink(l, M.amx, KS_PAMX)) return -1;
      if (M.use_xam) {
        aos_launch_ctx ce = launch_ctx(l, KS_PXAM);
        if (launch_err(aos_launch_amx(&M.ame, &ce), "lora adapter-major expand gate/up (prefill)")) return -1;
      }
      l->last_xe = M.use_xe ? 1 : 0;
      if (M.use_xe) {
        aos_launch_ctx cx = launch_ctx(l, KS_PXEXP);
        if (launch_err(aos_launch_xexp(&M.xe, &cx), "lora tile expand gate/up")) return -1;
      }
      l->last_sk = (M.g1.sk_nwg ? 1 : 0) | (M.g2.sk_nwg ? 2 : 0);
      if (M.g1.s_cols || M.g1.sk_nwg) M.g1.gen = next_gen(&l->gen);
      aos_launch_ctx c2 = launch_ctx(l, KS_GEMM_GU);
      if (launch_err(aos_launch_gemm(&M.g1, 1, &c2), "q4 gemm gate/up")) return -1;
      if (!M.fused_h && launch_tshrink(l, M.sh, KS_PSHRINK_H)) return -1;
      if (M.use_am_h && launch_amshrink(l, M.amh, KS_PAMH)) return -1;
      if (M.g2.s_cols || M.g2.sk_nwg) M.g2.gen = next_gen(&l->gen);
      aos_launch_ctx c4 = launch_ctx(l, KS_GEMM_DOWN);
      if (launch_err(aos_launch_gemm(&M.g2, 0, &c4), "q4 gemm down")) return -1;
    }
    return 0;
  }
  for (int t0 = 0; t0 < T; t0 += AOS_DECODE_MAX_T) {
    const int Tc = (T - t0) < AOS_DECODE_MAX_T ? (T - t0) : AOS_DECODE_MAX_T;
    if (mlp_decode_chunk(l, Tc, x + (size_t)t0 * H, rings + t0, y + (size_t)t0 * H, nullptr)) return -1;
  }
  return 0;
}

/* The decode MLP forward without allocation: the same launches as aoship_mlp_forward for T <= 32
 * tokens, with the workspace, counters and flags in the device's static scratch instead of the
 * layer's workspace. No hipMalloc, hipFree, event or other allocating call is made; a call whose
 * workspace does not fit is rejected. Calls that overlap on one GPU share the scratch and race. */
extern "C" int aoship_mlp_forward_noalloc(aoship_layer_t *l, const aoship_bf16_t *x, int T,
                                          const aoship_ring_t *rings, aoship_bf16_t *y) {
  if (check_common(l, x, T, rings, y)) return -1;
  if (!l->mats[MOD_GATE].valid || !l->mats[MOD_UP].valid || !l->mats[MOD_DOWN].valid)
    return set_err("aoship_mlp_forward_noalloc: gate_proj, up_proj and down_proj must be set");
  const Q4Mat &Wg = l->mats[MOD_GATE], &Wu = l->mats[MOD_UP], &Wd = l->mats[MOD_DOWN];
  if (Wu.in != Wg.in || Wu.out != Wg.out || Wd.in != Wg.out || Wd.out != Wg.in)
    return set_err("aoship_mlp_forward_noalloc: gate/up/down shapes are inconsistent");
  if (T < 1 || T > AOS_DECODE_MAX_T)
    return set_err("aoship_mlp_forward_noalloc: T must be 1.." + std::to_string(AOS_DECODE_MAX_T) +
                   " (decode batches)");
  if (g_device >= AOS_MAX_DEVICES) return set_err("aoship_mlp_forward_noalloc: device index out of range");
  ScratchDev &sd = g_scratch[g_device];
  if (!sd.ptr && scratch_setup(g_device)) return -1;
  MlpPlan P;
  plan_mlp(l, T, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, P);
  if (P.bytes > AOS_SCRATCH_WS_BYTES || P.ctr * 4 > AOS_SCRATCH_CTR_BYTES || P.flg * 4 > AOS_SCRATCH_FLAG_BYTES)
    return set_err("aoship_mlp_forward_noalloc: this layer at " + std::to_string(T) + " tokens needs " +
                   std::to_string(P.bytes) + " workspace bytes, " + std::to_string(P.ctr * 4) + " counter bytes and " +
                   std::to_string(P.flg * 4) + " flag bytes; the scratch holds " +
                   std::to_string(AOS_SCRATCH_WS_BYTES) + ", " + std::to_string(AOS_SCRATCH_CTR_BYTES) + " and " +
                   std::to_string(AOS_SCRATCH_FLAG_BYTES));
  const Ws w = {sd.ptr + AOS_SCRATCH_CTR_BYTES + AOS_SCRATCH_FLAG_BYTES, sd.ptr, sd.ptr + AOS_SCRATCH_CTR_BYTES,
                &sd.gen, false};
  return mlp_decode_chunk(l, T, x, rings, y, nullptr, &w);
}

/* Routing from features and the MLP of one layer in one call: at decode the router runs in the
 * first workgroups of the gate/up launch, beside the x shrink and the weight stream. */
extern "C" int aoship_route_mlp_forward(aoship_router_t *r, const float *features, const float *router_w, int d,
                                        aoship_layer_t *l, const aoship_bf16_t *x, int T, aoship_ring_t *rings,
                                        int32_t *status, aoship_bf16_t *y) {
  if (!r || !features) return set_err("aoship_route_mlp_forward: null router or features");
  if (check_common(l, x, T, rings, y)) return -1;
  if (!l->mats[MOD_GATE].valid || !l->mats[MOD_UP].valid || !l->mats[MOD_DOWN].valid)
    return set_err("aoship_route_mlp_forward: gate_proj, up_proj and down_proj must be set");
  const Q4Mat &Wg = l->mats[MOD_GATE], &Wu = l->mats[MOD_UP], &Wd = l->mats[MOD_DOWN];
  if (Wu.in != Wg.in || Wu.out != Wg.out || Wd.in != Wg.out || Wd.out != Wg.in)
    return set_err("aoship_route_mlp_forward: gate/up/down shapes are inconsistent");
  if (ensure_device()) return -1;
  aos_route_params rp;
  if (route_fill(r, features, router_w, d, nullptr, T, rings, nullptr, status, rp)) return -1;
  const bool plain =
      !(rp.scope || rp.tie_key || rp.post_allowed || rp.active_ids || rp.strengths || rp.hashes || rp.decisions);
  if (T > AOS_DECODE_MAX_T || !plain) { /* routing first, then the layer, both on the layer's stream */
    aos_launch_ctx cr = {l->stream, nullptr, nullptr};
    if (launch_err(aos_launch_route(&rp, &cr), "route")) return -1;
    return aoship_mlp_forward(l, x, T, rings, y);
  }
  return mlp_decode_chunk(l, T, x, rings, y, &rp);
}

/* Prefill chunk of projections sharing x: the group plan, one tile shrink over every module, one
 * GEMM per matrix. The same code sizes the workspace (a Carve over nullptr) and fills it. */
struct ProjPrefill {
  PrefillPlan P;
  aos_tshrink_params sp;
  aos_gemm_params gp[3];
};

static void plan_proj_prefill(aoship_layer *l, Carve &cv, const int *mods, int nm, const uint16_t *xc, int Tc,
                              const aoship_ring_t *rc, uint16_t *const *yc, ProjPrefill &Q) {
  const int in = l->mats[mods[0]].in;
  aos_lora_tab tabs[3];
  for (int i = 0; i < nm; ++i) tabs[i] = lora_tab(l, mods[i], in, l->mats[mods[i]].out);
  plan_prefill_common(l, cv, rc, Tc, tabs, nm, Q.P);
  const uint16_t *perm = Q.P.lora ? Q.P.gp.perm : nullptr;
  plan_tshrink(l, cv, Q.P, xc, perm, Tc, in, 0, nm, Q.sp);
  for (int i = 0; i < nm; ++i)
    plan_gemm(l, Q.P, Q.sp, l->mats[mods[i]], nullptr, xc, perm, perm, Tc, i, i, yc ? yc[i] : nullptr, Q.gp[i]);
}

/* Decode chunk (T <= 32) of projections sharing x: the x shrink (and plan) and the GEMVs, whose
 * K split is sized for their rows together so that they run in one launch. */
struct ProjDecode {
  XShrink xs;
  aos_gemv3_params g3;
  Handoff ho;
};

static void plan_proj_decode(aoship_layer *l, Carve &cv, const int *mods, int nm, const uint16_t *xc, int Tc,
                             const aoship_ring_t *rc, uint16_t *const *yc, ProjDecode &Q) {
  const int in = l->mats[mods[0]].in;
  aos_lora_tab tabs[3];
  for (int i = 0; i < nm; ++i) tabs[i] = lora_tab(l, mods[i], in, l->mats[mods[i]].out);
  aos_plan *plan = cv.b.take<aos_plan>(1);
  plan_x_shrink(l, cv, xc, Tc, in, tabs, nm, plan, rc, Q.xs);
  memset(&Q.g3, 0, sizeof(Q.g3));
  aos_gemv_params *gp = Q.g3.p;
  int rb_all = 0;
  for (int i = 0; i < nm; ++i) rb_all += l->mats[mods[i]].RB;
  for (int i = 0; i < nm; ++i) {
    const Q4Mat &W = l->mats[mods[i]];
    gp[i].w0 = W.dev();
    gp[i].x = xc;
    gp[i].T = Tc;
    gemv_geometry(rb_all, W.G, Tc, false, tabs[i].rpad > 0, gp[i], Tc <= 2 ? AOS_GEMV_WAVES_PROJ12 : AOS_GEMV_WAVES,
                  false, l->geo_wr[2], l->geo_ks[2]);
    gp[i].tab0 = tabs[i];
    gp[i].S0 = Q.xs.sp.S[i];
    gp[i].s_stride0 = Q.xs.sp.s_stride[i];
    gp[i].s_all = Q.xs.sp.all_mode;
    gp[i].plan = plan;
    gp[i].pk0 = plan_list_table(l, Q.xs, i, tabs[i].B);
    gp[i].zero_row = l->zeros.as<uint16_t>();
    gp[i].y = yc ? yc[i] : nullptr;
    gp[i].part = cv.b.take<float>((size_t)W.RB * gp[i].ks * nv_for(Tc) * 64);
    gp[i].counters = cv.counters((size_t)W.RB);
  }
  Q.ho = carve_handoff(cv, shrink_arrive_words(Q.xs.sp), fused_flag_words(gp, nm), shrink_lines(Q.xs.sp));
}

/* Workspace of projections sharing x for calls of up to max_tokens tokens (decode chunks at every
 * power of two up to 32 tokens, and the largest prefill chunk). */
static void size_proj(aoship_layer *l, const int *mods, int nm, int max_tokens, size_t &bytes, size_t &ctr,
                      size_t &flg) {
  auto take = [&](const Carve &cv) {
    bytes = std::max(bytes, cv.b.off + 256);
    ctr = std::max(ctr, cv.coff + 64);
    flg = std::max(flg, cv.foff + 64);
  };
  for (int T = 1; T <= AOS_DECODE_MAX_T && T <= max_tokens; ++T) {
    Carve cv(nullptr, nullptr, nullptr);
    ProjDecode Q;
    plan_proj_decode(l, cv, mods, nm, nullptr, T, nullptr, nullptr, Q);
    take(cv);
  }
  if (max_tokens > AOS_DECODE_MAX_T) {
    Carve cv(nullptr, nullptr, nullptr);
    ProjPrefill Q;
    plan_proj_prefill(l, cv, mods, nm, nullptr, chunk_prefill_t(max_tokens), nullptr, nullptr, Q);
    take(cv);
  }
}

/* One or more projections sharing the input x. */
static int proj_multi(aoship_layer *l, const int *mods, int nm, const uint16_t *x, int T,
                      const aoship_ring_t *rings, uint16_t *const *ys) {
  const int in = l->mats[mods[0]].in;
  for (int i = 0; i < nm; ++i) {
    if (!l->mats[mods[i]].valid) return set_err("projection weights not set");
    if (l->mats[mods[i]].in != in) return set_err("projections sharing x must share in_features");
    if (!ys[i] || !aligned16(ys[i])) return set_err("forward: output must be 16-byte aligned");
  }
  if (T > AOS_DECODE_MAX_T) {
    for (int t0 = 0; t0 < T; t0 += AOS_PREFILL_MAX_T) {
      const int Tc = chunk_prefill_t(T - t0);
      uint16_t *yc[3];
      for (int i = 0; i < nm; ++i) yc[i] = ys[i] + (size_t)t0 * l->mats[mods[i]].out;
      ProjPrefill Q;
      {
        Carve c0(nullptr, nullptr, nullptr);
        plan_proj_prefill(l, c0, mods, nm, x + (size_t)t0 * in, Tc, rings + t0, yc, Q);
        if (ws_reserve(l, c0.b.off + 256, c0.coff + 64, c0.foff + 64)) return -1;
      }
      Carve cv(l->ws.p, l->counters.p, l->flags.p);
      plan_proj_prefill(l, cv, mods, nm, x + (size_t)t0 * in, Tc, rings + t0, yc, Q);
      if (launch_gplan(l, Q.P)) return -1;
      if (launch_tshrink(l, Q.sp, KS_PSHRINK_X)) return -1;
      for (int i = 0; i < nm; ++i) {
        aos_launch_ctx cg = launch_ctx(l, KS_GEMM_PROJ);
        if (launch_err(aos_launch_gemm(&Q.gp[i], 0, &cg), "q4 gemm")) return -1;
      }
    }
    return 0;
  }
  for (int t0 = 0; t0 < T; t0 += AOS_DECODE_MAX_T) {
    const int Tc = (T - t0) < AOS_DECODE_MAX_T ? (T - t0) : AOS_DECODE_MAX_T;
    const uint16_t *xc = x + (size_t)t0 * in;
    uint16_t *yc[3];
    for (int i = 0; i < nm; ++i) yc[i] = ys[i] + (size_t)t0 * l->mats[mods[i]].out;
    ProjDecode Q;
    {
      Carve c0(nullptr, nullptr, nullptr);
      plan_proj_decode(l, c0, mods, nm, xc, Tc, rings + t0, yc, Q);
      if (ws_reserve(l, c0.b.off + 256, c0.coff + 64, c0.foff + 64)) return -1;
    }
    Carve cv(l->ws.p, l->counters.p, l->flags.p);
    plan_proj_decode(l, cv, mods, nm, xc, Tc, rings + t0, yc, Q);
    aos_gemv_params *gp = Q.g3.p;
    bool expands = false;
    for (int i = 0; i < nm; ++i) expands = expands || gp[i].has_expand;
    if (fuse_shrinks(l) && expands && shrink_wgs(Q.xs.sp) > 0) {
      if (Q.xs.separate_plan) {
        aos_launch_ctx c0 = launch_ctx(l, KS_SHRINK_X);
        if (launch_err(aos_launch_shrink(&Q.xs.plan_only, &c0), "adapter plan")) return -1;
      }
      const Ws lw = {l->ws.p, l->counters.p, l->flags.p, &l->gen, true};
      if (launch_fused(l, lw, Q.xs.sp, gp, nm, Q.ho, 0, KS_GEMV_PROJ, "lora shrink + q4 gemv")) return -1;
      continue;
    }
    if (launch_x_shrink(l, Q.xs)) return -1;
    aos_launch_ctx cg = launch_ctx(l, KS_GEMV_PROJ);
    if (nm == 1) {
      if (launch_err(aos_launch_gemv(&gp[0], 0, &cg), "q4 gemv")) return -1;
    } else {
      Q.g3.n = nm;
      int end = 0;
      for (int i = 0; i < 3; ++i) {
        if (i < nm) end += gp[i].nrbg * gp[i].ks;
        Q.g3.wg_end[i] = end;
      }
      if (launch_err(aos_launch_gemv3(&Q.g3, &cg), "q4 gemv")) return -1;
    }
  }
  return 0;
}

extern "C" int aoship_proj_forward(aoship_layer_t *l, const char *module, const aoship_bf16_t *x,
                                   int T, const aoship_ring_t *rings, aoship_bf16_t *y) {
  if (check_common(l, x, T, rings, y)) return -1;
  int m = module_index(module);
  if (m < 0) return set_err(std::string("Unknown module name: ") + (module ? module : "(null)"));
  if (!l->mats[m].valid) return set_err(std::string("base weights not set for ") + module);
  int mods[1] = {m};
  uint16_t *ys[1] = {y};
  return proj_multi(l, mods, 1, x, T, rings, ys);
}

extern "C" int aoship_qkv_forward(aoship_layer_t *l, const aoship_bf16_t *x, int T,
                                  const aoship_ring_t *rings, aoship_bf16_t *q, aoship_bf16_t *k,
                                  aoship_bf16_t *v) {
  if (check_common(l, x, T, rings, q)) return -1;
  int mods[3] = {MOD_Q, MOD_K, MOD_V};
  uint16_t *ys[3] = {q, k, v};
  return proj_multi(l, mods, 3, x, T, rings, ys);
}

extern "C" void aoship_layer_free(aoship_layer_t *l) {
  if (!l) return;
  (void)hipDeviceSynchronize();
  resolve_events(l);
  for (auto e : l->event_pool) (void)hipEventDestroy(e);
  unbind_all(l);
  if (l->wait_host) (void)hipHostFree(l->wait_host);
  delete l;
}

/* ------------------------------------------------------------------------------------------ */
/* decoder model: embedding -> layers (norm, q/k/v + LoRA, RoPE + KV cache, attention, o + LoRA,  */
/* residual, norm, SwiGLU MLP + LoRA, residual) -> final norm -> LM head                       */
/* ------------------------------------------------------------------------------------------ */

struct aoship_model {
  aoship_model_config_t cfg;
  std::vector<aoship_layer *> layers;
  DevBuf emb_q4, emb_s, emb_b, emb_bf16; /* MLX rows, as loaded */
  bool emb_set = false;
  Q4Mat lm;
  DevBuf lm_part, lm_ctr;
  DevBuf attn_ctr; /* [ws_T][num_heads] split arrivals, zero between launches */
  std::vector<DevBuf> norm_in, norm_post, bias; /* bias: [layer * 3 + {q,k,v}] */
  DevBuf norm_final;
  DevBuf kc, vc; /* [layers][nkv][max_seq][hd] bf16 */
  DevBuf inv_freq;
  DevBuf ws;     /* per-call buffers, sized for ws_T tokens */
  int ws_T = 0;
  int cache_len = 0;
  hipStream_t stream = nullptr;
};

extern "C" aoship_model_t *aoship_model_new(const aoship_model_config_t *c) {
  if (!c) {
    set_err("aoship_model_new: null config");
    return nullptr;
  }
  if (ensure_device()) return nullptr;
  if (c->num_layers < 1 || c->hidden < 64 || c->hidden % 64 || c->intermediate < 64 || c->intermediate % 64 ||
      c->num_heads < 1 || c->num_kv_heads < 1 || c->num_heads % c->num_kv_heads || c->head_dim < 8 ||
      c->head_dim % 8 || c->head_dim > AOS_ATTN_MAX_HD || c->vocab < 32 || c->vocab % 32 || c->max_seq < 1 ||
      c->hidden > 16384) {
    set_err("aoship_model_new: unsupported shape (hidden a multiple of 64 up to 16384, intermediate a multiple "
            "of 64, heads divisible by kv heads, head_dim a multiple of 8 up to 256, vocab a multiple of 32)");
    return nullptr;
  }
  if ((c->num_heads * c->head_dim) % 64 || (c->num_kv_heads * c->head_dim) % 32) {
    set_err("aoship_model_new: num_heads * head_dim must be a multiple of 64 and num_kv_heads * head_dim of 32");
    return nullptr;
  }
  auto *m = new aoship_model();
  m->cfg = *c;
  if (!(std::isfinite(m->cfg.rms_eps) && m->cfg.rms_eps >= 0.0f)) m->cfg.rms_eps = 1e-6f;
  const int L = c->num_layers;
  m->norm_in.resize((size_t)L);
  m->norm_post.resize((size_t)L);
  m->bias.resize((size_t)L * 3);
  for (int i = 0; i < L; ++i) {
    aoship_layer_t *l = aoship_layer_new(i, AOSHIP_GROUP_SIZE, AOSHIP_BITS);
    if (!l) {
      aoship_model_free(m);
      return nullptr;
    }
    m->layers.push_back(l);
  }
  /* RoPE inverse frequencies as the fused forward computes them (…real.cpp:3252-3257) */
  const int half = c->head_dim / 2;
  std::vector<float> inv((size_t)half);
  for (int i = 0; i < half; ++i) {
    const float exp_val = -2.0f * (float)i / (float)c->head_dim;
    inv[(size_t)i] = 1.0f / std::pow(c->rope_theta, exp_val);
  }
  std::vector<float> ones((size_t)c->hidden, 1.0f);
  const size_t cache = (size_t)L * c->num_kv_heads * c->max_seq * c->head_dim * 2;
  if (m->inv_freq.upload(inv.data(), inv.size() * 4) || m->kc.alloc(cache, true) || m->vc.alloc(cache, true) ||
      m->norm_final.upload(ones.data(), ones.size() * 4)) {
    aoship_model_free(m);
    return nullptr;
  }
  for (int i = 0; i < L; ++i)
    if (m->norm_in[(size_t)i].upload(ones.data(), ones.size() * 4) ||
        m->norm_post[(size_t)i].upload(ones.data(), ones.size() * 4)) {
      aoship_model_free(m);
      return nullptr;
    }
  return m;
}

extern "C" void aoship_model_free(aoship_model_t *m) {
  if (!m) return;
  (void)hipDeviceSynchronize();
  for (auto *l : m->layers) aoship_layer_free(l);
  delete m;
}

extern "C" aoship_layer_t *aoship_model_layer(aoship_model_t *m, int layer_idx) {
  if (!m || layer_idx < 0 || layer_idx >= (int)m->layers.size()) {
    set_err("aoship_model_layer: layer index out of range");
    return nullptr;
  }
  return m->layers[(size_t)layer_idx];
}

extern "C" int aoship_model_set_embedding(aoship_model_t *m, const uint32_t *packed, const uint16_t *scales_f16,
                                          const uint16_t *biases_f16, const uint16_t *rows_bf16) {
  if (!m) return set_err("aoship_model_set_embedding: null model");
  if (ensure_device()) return -1;
  const size_t V = (size_t)m->cfg.vocab, H = (size_t)m->cfg.hidden;
  m->emb_q4.release();
  m->emb_s.release();
  m->emb_b.release();
  m->emb_bf16.release();
  m->emb_set = false;
  if (packed) {
    if (!scales_f16) return set_err("aoship_model_set_embedding: 4-bit rows need scales");
    if (m->emb_q4.upload(packed, V * H / 2) || m->emb_s.upload(scales_f16, V * (H / 64) * 2)) return -1;
    if (biases_f16 && m->emb_b.upload(biases_f16, V * (H / 64) * 2)) return -1;
  } else if (rows_bf16) {
    if (m->emb_bf16.upload(rows_bf16, V * H * 2)) return -1;
  } else {
    return set_err("aoship_model_set_embedding: no rows given");
  }
  m->emb_set = true;
  return 0;
}

extern "C" int aoship_model_set_lm_head(aoship_model_t *m, const uint32_t *packed, const uint16_t *scales_f16,
                                        const uint16_t *biases_f16) {
  if (!m || !packed || !scales_f16) return set_err("aoship_model_set_lm_head: null argument");
  if (ensure_device()) return -1;
  return q4_upload(m->lm, m->cfg.vocab, m->cfg.hidden, packed, scales_f16, biases_f16);
}

extern "C" int aoship_model_set_norm(aoship_model_t *m, int layer_idx, int which, const float *w) {
  if (!m || !w) return set_err("aoship_model_set_norm: null argument");
  if (ensure_device()) return -1;
  const size_t bytes = (size_t)m->cfg.hidden * 4;
  if (layer_idx == -1) return m->norm_final.upload(w, bytes);
  if (layer_idx < 0 || layer_idx >= m->cfg.num_layers || (which != 0 && which != 1))
    return set_err("aoship_model_set_norm: layer or norm index out of range");
  return (which == 0 ? m->norm_in : m->norm_post)[(size_t)layer_idx].upload(w, bytes);
}

extern "C" int aoship_model_set_bias(aoship_model_t *m, int layer_idx, const char *module, const float *b) {
  if (!m) return set_err("aoship_model_set_bias: null model");
  const int mi = module_index(module);
  if (layer_idx < 0 || layer_idx >= m->cfg.num_layers || mi < MOD_Q || mi > MOD_V)
    return set_err("aoship_model_set_bias: layer out of range or module not q_proj / k_proj / v_proj");
  if (ensure_device()) return -1;
  const int width = (mi == MOD_Q ? m->cfg.num_heads : m->cfg.num_kv_heads) * m->cfg.head_dim;
  DevBuf &d = m->bias[(size_t)layer_idx * 3 + (size_t)(mi - MOD_Q)];
  if (!b) {
    d.release();
    return 0;
  }
  return d.upload(b, (size_t)width * 4);
}

extern "C" int aoship_model_set_adapters(aoship_model_t *m, aoship_lora_adapter_t *const *table, int n) {
  if (!m) return set_err("aoship_model_set_adapters: null model");
  for (auto *l : m->layers)
    if (aoship_layer_set_adapters(l, table, n)) return -1;
  return 0;
}

extern "C" int aoship_model_set_stream(aoship_model_t *m, void *stream) {
  if (!m) return set_err("aoship_model_set_stream: null model");
  m->stream = (hipStream_t)stream;
  for (auto *l : m->layers)
    if (aoship_layer_set_stream(l, stream)) return -1;
  return 0;
}

extern "C" int aoship_model_reset_cache(aoship_model_t *m) {
  if (!m) return set_err("aoship_model_reset_cache: null model");
  m->cache_len = 0;
  return 0;
}

extern "C" int aoship_model_cache_len(const aoship_model_t *m) { return m ? m->cache_len : -1; }

/* per-call buffers: hidden f32, normed / q / k / v / attention / y bf16, rotated q f32, the
 * attention splits' partials */
static int attn_splits(const aoship_model *m, int T, int visible_max) {
  const int chunks = ceil_div(visible_max, 64);
  int s = ceil_div(1024, m->cfg.num_heads * T);
  if (s > chunks) s = chunks;
  return s < 1 ? 1 : s;
}

struct ModelWs {
  float *hidden, *qr, *part;
  uint16_t *normed, *q, *k, *v, *attn, *y;
  size_t bytes;
};

static ModelWs model_ws(const aoship_model *m, int T, void *base) {
  const aoship_model_config_t &c = m->cfg;
  const int splits = attn_splits(m, T, c.max_seq);
  Bump b(base, 0);
  ModelWs w;
  w.hidden = b.take<float>((size_t)T * c.hidden);
  w.qr = b.take<float>((size_t)T * c.num_heads * c.head_dim);
  w.part = b.take<float>((size_t)T * c.num_heads * splits * (c.head_dim + 2));
  w.normed = b.take<uint16_t>((size_t)T * c.hidden);
  w.q = b.take<uint16_t>((size_t)T * c.num_heads * c.head_dim);
  w.k = b.take<uint16_t>((size_t)T * c.num_kv_heads * c.head_dim);
  w.v = b.take<uint16_t>((size_t)T * c.num_kv_heads * c.head_dim);
  w.attn = b.take<uint16_t>((size_t)T * c.num_heads * c.head_dim);
  w.y = b.take<uint16_t>((size_t)T * c.hidden);
  w.bytes = b.off;
  return w;
}

extern "C" int aoship_model_reserve(aoship_model_t *m, int max_tokens) {
  if (!m || max_tokens < 1) return set_err("aoship_model_reserve: bad arguments");
  if (ensure_device()) return -1;
  for (auto *l : m->layers)
    if (aoship_layer_reserve(l, max_tokens)) return -1;
  if (max_tokens > m->ws_T) {
    if (m->ws.alloc(model_ws(m, max_tokens, nullptr).bytes, false) ||
        m->attn_ctr.alloc((size_t)max_tokens * m->cfg.num_heads * 4, true))
      return -1;
    m->ws_T = max_tokens;
  }
  return 0;
}

extern "C" int aoship_model_forward(aoship_model_t *m, const int32_t *ids, int T, int position_offset,
                                    const aoship_ring_t *rings, float *logits) {
  if (!m || !ids || !rings || !logits) return set_err("aoship_model_forward: null argument");
  const aoship_model_config_t &c = m->cfg;
  if (T < 1) return set_err("aoship_model_forward: T must be positive");
  if (position_offset != m->cache_len)
    return set_err("aoship_model_forward: position_offset must equal the cache length (" +
                   std::to_string(m->cache_len) + ")");
  if (position_offset + T > c.max_seq) return set_err("aoship_model_forward: the KV cache is full");
  if (!m->emb_set) return set_err("aoship_model_forward: embedding not set");
  if (!m->lm.valid) return set_err("aoship_model_forward: LM head not set");
  for (auto *l : m->layers)
    if (check_no_timeout(l)) return -1;
  if (ensure_device()) return -1;
  if (T > m->ws_T) {
    const size_t bytes = model_ws(m, T, nullptr).bytes;
    if (m->ws.alloc(bytes, false) || m->attn_ctr.alloc((size_t)T * c.num_heads * 4, true)) return -1;
    m->ws_T = T;
  }
  const ModelWs w = model_ws(m, T, m->ws.p);
  aos_launch_ctx ctx = {m->stream, nullptr, nullptr};
  const int hd = c.head_dim, nh = c.num_heads, nkv = c.num_kv_heads;

  aos_embed_params ep;
  memset(&ep, 0, sizeof(ep));
  ep.ids = ids;
  ep.T = T;
  ep.H = c.hidden;
  ep.vocab = c.vocab;
  ep.q4 = m->emb_q4.p ? m->emb_q4.as<uint32_t>() : nullptr;
  ep.s16 = m->emb_s.p ? m->emb_s.as<uint16_t>() : nullptr;
  ep.b16 = m->emb_b.p ? m->emb_b.as<uint16_t>() : nullptr;
  ep.bf16 = m->emb_bf16.p ? m->emb_bf16.as<uint16_t>() : nullptr;
  ep.hidden = w.hidden;
  if (launch_err(aos_launch_embed(&ep, &ctx), "embedding")) return -1;

  auto norm = [&](const uint16_t *add, const DevBuf &wt, int rows, float *hid, uint16_t *out) {
    aos_norm_params np;
    np.hidden = hid;
    np.add = add;
    np.w = wt.as<float>();
    np.eps = c.rms_eps;
    np.T = rows;
    np.H = c.hidden;
    np.out = out;
    return launch_err(aos_launch_norm(&np, &ctx), "rms norm");
  };
  const size_t layer_cache = (size_t)nkv * c.max_seq * hd;
  for (int li = 0; li < c.num_layers; ++li) {
    aoship_layer *l = m->layers[(size_t)li];
    if (norm(li == 0 ? nullptr : w.y, m->norm_in[(size_t)li], T, w.hidden, w.normed)) return -1;
    if (aoship_qkv_forward(l, w.normed, T, rings, w.q, w.k, w.v)) return -1;
    aos_rope_params rp;
    rp.q = w.q;
    rp.k = w.k;
    rp.v = w.v;
    rp.bq = m->bias[(size_t)li * 3].p ? m->bias[(size_t)li * 3].as<float>() : nullptr;
    rp.bk = m->bias[(size_t)li * 3 + 1].p ? m->bias[(size_t)li * 3 + 1].as<float>() : nullptr;
    rp.bv = m->bias[(size_t)li * 3 + 2].p ? m->bias[(size_t)li * 3 + 2].as<float>() : nullptr;
    rp.inv_freq = m->inv_freq.as<float>();
    rp.T = T;
    rp.nh = nh;
    rp.nkv = nkv;
    rp.hd = hd;
    rp.offset = position_offset;
    rp.max_seq = c.max_seq;
    rp.qr = w.qr;
    rp.kc = m->kc.as<uint16_t>() + (size_t)li * layer_cache;
    rp.vc = m->vc.as<uint16_t>() + (size_t)li * layer_cache;
    /* one token: RoPE, the biases and the cache append run inside the attention launch */
    const bool fuse_rope = T == 1;
    if (!fuse_rope && launch_err(aos_launch_rope(&rp, &ctx), "rope")) return -1;
    aos_attn_params ap;
    memset(&ap, 0, sizeof(ap));
    ap.q = w.qr;
    ap.kc = rp.kc;
    ap.vc = rp.vc;
    ap.T = T;
    ap.nh = nh;
    ap.nkv = nkv;
    ap.hd = hd;
    ap.offset = position_offset;
    ap.max_seq = c.max_seq;
    ap.splits = attn_splits(m, T, position_offset + T);
    ap.chunk = ceil_div(ceil_div(position_offset + T, ap.splits), 64) * 64;
    ap.scale = 1.0f / std::sqrt((float)hd);
    ap.part = w.part;
    ap.out = w.attn;
    ap.counters = m->attn_ctr.as<uint32_t>();
    if (fuse_rope) {
      ap.rope_fused = 1;
      ap.qb = w.q;
      ap.kb = w.k;
      ap.vb = w.v;
      ap.bq = rp.bq;
      ap.bk = rp.bk;
      ap.bv = rp.bv;
      ap.inv_freq = rp.inv_freq;
    }
    if (launch_err(aos_launch_attention(&ap, &ctx), "attention")) return -1;
    if (aoship_proj_forward(l, "o_proj", w.attn, T, rings, w.y)) return -1;
    if (norm(w.y, m->norm_post[(size_t)li], T, w.hidden, w.normed)) return -1;
    if (aoship_mlp_forward(l, w.normed, T, rings, w.y)) return -1;
  }
  /* residual of the last MLP and the final norm, for the last token only */
  const size_t lastH = (size_t)(T - 1) * c.hidden;
  if (norm(w.y + lastH, m->norm_final, 1, w.hidden + lastH, w.normed + lastH)) return -1;
  aos_gemv_params g;
  memset(&g, 0, sizeof(g));
  g.w0 = m->lm.dev();
  g.x = w.normed + lastH;
  g.T = 1;
  g.yf = logits;
  g.zero_row = m->layers[0]->zeros.as<uint16_t>();
  gemv_geometry(m->lm.RB, m->lm.G, 1, false, false, g);
  if (g.ks > 1) {
    const size_t part = (size_t)m->lm.RB * g.ks * 64 * 4;
    if (m->lm_part.bytes < part && m->lm_part.alloc(part, false)) return -1;
    if (m->lm_ctr.bytes < (size_t)m->lm.RB * 4 && m->lm_ctr.alloc((size_t)m->lm.RB * 4, true)) return -1;
    g.part = m->lm_part.as<float>();
    g.counters = m->lm_ctr.as<uint32_t>();
  }
  if (launch_err(aos_launch_gemv(&g, 0, &ctx), "lm head")) return -1;
  m->cache_len += T;
  return 0;
}

/* ---- Liquid blend ---- */

/* LiquidKernel::blend_and_forward (crates/adapteros-lora-kernel-api/src/liquid.rs:147-160),
 * checked as blend_and_forward_reference checks (liquid.rs:163-219), in its order and with its
 * messages. */
extern "C" int aoship_liquid_blend_and_forward(const aoship_liquid_adapter_t *adapters, int n_adapters,
                                               const float *coefficients, int n_coefficients, const float *input,
                                               int in_len, float *output, int out_len, int *precision, void *stream) {
  if (n_adapters <= 0) return set_err("Liquid blend requested with zero adapters");
  if (n_adapters > AOSHIP_LIQUID_MAX_ADAPTERS)
    return set_err("Liquid blend exceeds max adapters (" + std::to_string(n_adapters) + " > " +
                   std::to_string(AOSHIP_LIQUID_MAX_ADAPTERS) + ")");
  if (n_adapters != n_coefficients)
    return set_err("Liquid blend coefficient mismatch: " + std::to_string(n_adapters) + " adapters vs " +
                   std::to_string(n_coefficients) + " coefficients");
  if (!adapters || !coefficients) return set_err("aoship_liquid_blend_and_forward: null adapters or coefficients");
  if (in_len < 0 || out_len < 0) return set_err("aoship_liquid_blend_and_forward: negative length");
  int prec = 0;
  for (int i = 0; i < n_adapters; ++i) {
    const aoship_liquid_adapter_t &a = adapters[i];
    const struct {
      const aoship_liquid_tensor_t *t;
      const char *label;
    } ts[2] = {{&a.down, "down"}, {&a.up, "up"}};
    for (const auto &e : ts) {
      const aoship_liquid_tensor_t &t = *e.t;
      if (t.rows < 0 || t.cols < 0 || (size_t)t.rows * (size_t)t.cols != t.len)
        return set_err(std::string("Liquid tensor ") + e.label + " has inconsistent shape: rows*cols=" +
                       std::to_string((long long)t.rows * t.cols) + " != len=" + std::to_string(t.len));
    }
    if (a.down.cols != in_len)
      return set_err("Liquid adapter " + std::to_string(i) + " input mismatch: down.cols=" +
                     std::to_string(a.down.cols) + " vs input len=" + std::to_string(in_len));
    if (a.up.rows > out_len)
      return set_err("Liquid adapter " + std::to_string(i) + " output mismatch: up.rows=" +
                     std::to_string(a.up.rows) + " vs output len=" + std::to_string(out_len));
    if (a.up.cols != a.down.rows)
      return set_err("Liquid adapter " + std::to_string(i) + " rank mismatch: up.cols=" +
                     std::to_string(a.up.cols) + " vs down.rows=" + std::to_string(a.down.rows));
    if (a.down.bf16 || a.up.bf16) prec = 1;
  }
  /* this backend's own limits */
  aos_liquid_params p;
  memset(&p, 0, sizeof(p));
  p.n = n_adapters;
  p.in = in_len;
  p.out_len = out_len;
  p.x = input;
  p.y = output;
  for (int i = 0; i < n_adapters; ++i) {
    const aoship_liquid_adapter_t &a = adapters[i];
    const int rank = a.down.rows;
    if (rank > AOSHIP_LIQUID_MAX_RANK)
      return set_err("aoship_liquid_blend_and_forward: adapter " + std::to_string(i) + " rank " +
                     std::to_string(rank) + " exceeds " + std::to_string(AOSHIP_LIQUID_MAX_RANK));
    const size_t align_d = a.down.bf16 ? 2 : 4, align_u = a.up.bf16 ? 2 : 4;
    if ((a.down.len && (!a.down.data || (uintptr_t)a.down.data % align_d)) ||
        (a.up.len && (!a.up.data || (uintptr_t)a.up.data % align_u)))
      return set_err("aoship_liquid_blend_and_forward: adapter " + std::to_string(i) +
                     " weights must be non-NULL and aligned to their element size");
    p.down[i] = a.down.data;
    p.up[i] = a.up.data;
    p.down_bf16[i] = a.down.bf16 ? 1 : 0;
    p.up_bf16[i] = a.up.bf16 ? 1 : 0;
    p.rank[i] = rank;
    p.up_rows[i] = a.up.rows;
    p.coef[i] = coefficients[i];
    p.scaling[i] = a.alpha / (float)rank; /* liquid.rs:228 */
  }
  if ((in_len > 0 && (!input || (uintptr_t)input % 4)) || (out_len > 0 && (!output || (uintptr_t)output % 4)))
    return set_err("aoship_liquid_blend_and_forward: input and output must be non-NULL, 4-byte aligned device "
                   "float arrays");
  if (ensure_device()) return -1;
  if (precision) *precision = prec;
  if (out_len == 0) return 0;
  aos_launch_ctx c = {stream, nullptr, nullptr};
  return launch_err(aos_launch_liquid(&p, &c), "liquid blend");
}
