// C++ host-side tests of adapter-os_amd/host/aos_kernel_api.hpp, written like the reference's own
// Rust tests they restate (each names its source). Mode "cpu" runs the tests that touch no GPU;
// mode "gpu" runs the device ones. Prints "ok <name>" per test; exits 1 on the first failure.
// The ingest modes read safetensors files that tests/test_host_cpp.py writes with the safetensors
// Python package: "ingest-adapter FILE [METADATA_JSON]", "ingest-lora FILE RANK ALPHA TARGETS" and
// "ingest-base FILE KEY" print what the parser read as one JSON line (no GPU); "gpu-ingest DIR ..." loads the same weights from the
// files and from raw arrays and checks that the layer forwards agree bit for bit.
#include <cmath>
#include <cinttypes>
#include <cstdio>
#include <fstream>
#include <sstream>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

#include "../../adapter-os_amd/host/aos_kernel_api.hpp"

using namespace adapteros;

namespace {

int g_failed = 0;

#define CHECK(cond)                                                              \
  do {                                                                           \
    if (!(cond)) {                                                               \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
      throw std::runtime_error("check failed");                                  \
    }                                                                            \
  } while (0)

void run(const char *name, const std::function<void()> &fn) {
  try {
    fn();
    std::printf("ok %s\n", name);
  } catch (const std::exception &e) {
    std::printf("FAIL %s: %s\n", name, e.what());
    ++g_failed;
  }
  std::fflush(stdout);
}

template <class F>
ErrorKind error_kind_of(F &&f) {
  try {
    f();
  } catch (const AosError &e) {
    return e.kind();
  }
  throw std::runtime_error("expected an AosError");
}

std::vector<AdapterInfo> infos(const std::vector<uint64_t> &stable_ids) {
  std::vector<AdapterInfo> v;
  for (size_t i = 0; i < stable_ids.size(); ++i) v.push_back({"test_adapter_" + std::to_string(i), stable_ids[i]});
  return v;
}

// ---- CPU: RouterRing (crates/adapteros-lora-kernel-api/src/lib.rs:1442-1520) ----

void cpu_tests() {
  run("router_ring_new_valid_k", [] {
    for (size_t k = 0; k <= 8; ++k) {
      RouterRing r = RouterRing::with_k(k);
      CHECK(r.k == k && r.len() == k && r.position == 0);
      for (int i = 0; i < 8; ++i) CHECK(r.indices[i] == 0 && r.gates_q15[i] == 0);
    }
  });
  run("router_ring_is_empty", [] {
    CHECK(RouterRing::with_k(0).is_empty());
    CHECK(!RouterRing::with_k(1).is_empty());
  });
  run("router_ring_set_valid_entries", [] {
    RouterRing r = RouterRing::with_k(4);
    r.set({1, 2, 3, 4}, {1000, 2000, 1500, 500});
    CHECK((r.active_indices() == std::vector<uint16_t>{1, 2, 3, 4}));
    CHECK((r.active_gates() == std::vector<int16_t>{1000, 2000, 1500, 500}));
    CHECK(r.k == 4);
  });
  run("router_ring_set_with_max_adapter_valid", [] {
    RouterRing r = RouterRing::with_k(3);
    r.set_with_max_adapter({0, 5, 9}, {100, 200, 300}, 10);
    CHECK((r.active_indices() == std::vector<uint16_t>{0, 5, 9}));
    CHECK((r.active_gates() == std::vector<int16_t>{100, 200, 300}));
  });
  run("router_ring_zero_fills_unused_entries", [] {
    RouterRing r = RouterRing::with_k(8);
    r.indices.fill(9);
    r.gates_q15.fill(999);
    r.set({1, 2, 3}, {100, 200, 300});
    for (int i = 0; i < 3; ++i) CHECK(r.indices[i] == i + 1 && r.gates_q15[i] == 100 * (i + 1));
    for (int i = 3; i < 8; ++i) CHECK(r.indices[i] == 0 && r.gates_q15[i] == 0);
  });
  run("router_ring_active_slices", [] {
    RouterRing r = RouterRing::with_k(2);
    r.set({10, 20}, {500, 600});
    CHECK((r.active_indices() == std::vector<uint16_t>{10, 20}));
    CHECK(r.len() == 2);
  });
  // release-build invariants (lib.rs:122-193)
  run("router_ring_release_invariants", [] {
    RouterRing r = RouterRing::with_k(12);
    CHECK(r.k == 8);
    r.set({1, 2}, {5});
    CHECK(r.k == 0 && r.indices[0] == 0);
    r.set_with_max_adapter({1, 20}, {5, 6}, 10);
    CHECK(r.k == 0 && r.indices[1] == 0);
  });
  run("decision_to_router_ring", [] {  // router/src/types.rs:699-706
    Decision d{{3, 1}, {20000, 12767}};
    RouterRing r = d.to_router_ring();
    CHECK(r.k == 2 && r.indices[0] == 3 && r.gates_q15[1] == 12767);
    aoship_ring_t dev = r.to_device();
    CHECK(sizeof(dev) == 40 && dev.top_k == 2 && dev.adapter_indices[1] == 1);
    Decision big;
    big.indices.assign(9, 0);
    big.gates_q15.assign(9, 1);
    CHECK(error_kind_of([&] { big.to_router_ring(); }) == ErrorKind::Validation);
  });
  run("router_new_k_above_max", [] {  // router.rs:769-777
    CHECK(error_kind_of([] { Router r(9, 1.0f, 0.02f); }) == ErrorKind::Routing);
  });
  // FIPS 180-4 examples and RFC 5869 appendix A test cases 1 and 3
  run("sha256_hmac_hkdf_known_answers", [] {
    auto hx = [](const uint8_t *p, size_t n) { return det::B3Hash::hex(p, n); };
    CHECK(hx(det::sha256((const uint8_t *)"abc", 3).data(), 32) ==
          "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad");
    CHECK(hx(det::sha256(nullptr, 0).data(), 32) == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855");
    const std::string m448 = "abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq";
    CHECK(hx(det::sha256((const uint8_t *)m448.data(), m448.size()).data(), 32) ==
          "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1");
    std::vector<uint8_t> ikm(22, 0x0b), salt, info;
    for (int i = 0; i <= 12; ++i) salt.push_back((uint8_t)i);
    for (int i = 0xf0; i <= 0xf9; ++i) info.push_back((uint8_t)i);
    auto okm = det::hkdf_sha256(salt.data(), salt.size(), ikm.data(), ikm.size(), info.data(), info.size(), 42);
    CHECK(hx(okm.data(), okm.size()) ==
          "3cb25f25faacd57a90434f64d0362f2a2d2d0a90cf1a5a4c5db02d56ecc4c5bf34007208d5b887185865");
    okm = det::hkdf_sha256(nullptr, 0, ikm.data(), ikm.size(), nullptr, 0, 42);
    CHECK(hx(okm.data(), okm.size()) ==
          "8da4e775a563c18f715f802a063c5a31b8a11f5c5ee1879ec3454e5f3c738d2d9d201395faa4b61a96c8");
  });
  run("b3hash_hex_forms", [] {  // hash.rs:57-84
    const det::B3Hash h = det::B3Hash::hash("hello world");
    CHECK(h.to_hex() == "d74981efa70a0c880b8d8c1985d075dbcbf679b99a5f9914e5aaf96b831a9e24");
    CHECK(h.to_short_hex() == "d74981efa70a0c88");
    CHECK(det::B3Hash::from_hex("D74981EFA70A0C880B8D8C1985D075DBCBF679B99A5F9914E5AAF96B831A9E24") == h);
    CHECK(!det::B3Hash::from_hex("d74981") && !det::B3Hash::from_hex(std::string(64, 'g')));
  });
  // policy_mask.rs:246-315 set semantics
  run("routing_policy_pass_bytes", [] {
    const std::vector<std::string> ids = {"a", "b", "c", "d"};
    const std::vector<std::optional<std::string>> cl = {std::string("x"), std::nullopt, std::string("y"),
                                                        std::string("x")};
    RoutingPolicy p;
    CHECK((routing_policy_pass_bytes(p, ids, cl) == std::vector<uint8_t>{1, 1, 1, 1}));
    p.denied_adapter_ids = std::vector<std::string>{"c", "nonexistent"};
    CHECK((routing_policy_pass_bytes(p, ids, cl) == std::vector<uint8_t>{1, 1, 0, 1}));
    p.allowed_clusters = std::vector<std::string>{"x"};  // an adapter without cluster fails it
    CHECK((routing_policy_pass_bytes(p, ids, cl) == std::vector<uint8_t>{1, 0, 0, 1}));
    RoutingPolicy q;
    q.denied_clusters = std::vector<std::string>{"x"};  // an adapter without cluster passes it
    q.allowed_adapter_ids = std::vector<std::string>{"a", "b", "c"};
    CHECK((routing_policy_pass_bytes(q, ids, cl) == std::vector<uint8_t>{0, 1, 1, 0}));
    CHECK(error_kind_of([&] { routing_policy_pass_bytes(q, ids, {std::nullopt}); }) == ErrorKind::PolicyViolation);
  });
}

// ---- GPU ----

void gpu_tests() {
  run("test_deterministic_top_k_ordering", [] {  // router/tests/determinism.rs:38-87
    Router router(3, 1.0f, 0.01f);
    std::vector<float> priors{0.5f, 0.5f, 0.5f, 0.3f, 0.2f};
    auto info = infos({300, 100, 200, 400, 500});
    auto mask = PolicyMask::allow_all(info.size());
    Decision d1 = router.route_with_adapter_info({}, priors, info, mask);
    Decision d2 = router.route_with_adapter_info({}, priors, info, mask);
    CHECK(d1.indices == d2.indices && d1.gates_q15 == d2.gates_q15);
    CHECK((d1.indices == std::vector<uint16_t>{1, 2, 0}));
    Router router2(3, 1.0f, 0.01f);
    Decision d3 = router2.route_with_adapter_info({}, priors, info, mask);
    CHECK(d1.indices == d3.indices && d1.gates_q15 == d3.gates_q15);
  });
  run("test_entropy_computation", [] {  // router/tests/abstain_edge_cases.rs:121-162
    Router router(3, 1.0f, 0.01f);
    auto info = infos({0, 0, 0});
    auto mask = PolicyMask::allow_all(3);
    Decision d1 = router.route_with_adapter_info({}, {0.33f, 0.33f, 0.34f}, info, mask);
    Decision d2 = router.route_with_adapter_info({}, {2.0f, 0.1f, 0.1f}, info, mask);
    CHECK(d1.entropy > d2.entropy);
    CHECK(d1.indices.size() == 3 && d2.indices.size() == 3);
    CHECK(d1.candidates.size() == 3 && d1.candidates[0].adapter_idx == d1.indices[0]);
    CHECK(d2.candidates[0].raw_score == 2.0f && d2.candidates[0].gate_q15 == d2.gates_q15[0]);
  });
  run("test_entropy_uniform_four", [] {  // compute_entropy of four equal gates: log2(4)
    Router router(4, 1.0f, 0.02f);
    Decision d = router.route_with_adapter_info({}, {0.5f, 0.5f, 0.5f, 0.5f}, infos({1, 2, 3, 4}),
                                                PolicyMask::allow_all(4));
    CHECK(d.entropy == 2.0f && d.candidates.size() == 4 && d.candidates[3].raw_score == 0.5f);
  });
  run("test_empty_decision_zero_entropy", [] {  // abstain_edge_cases.rs:60-76
    Router router(2, 1.0f, 0.02f);
    std::vector<AdapterInfo> info{{"adapter-1", 0}, {"adapter-2", 0}};
    Decision d = router.route_with_adapter_info({}, {1.0f, 1.0f}, info, PolicyMask::deny(info, {"adapter-1", "adapter-2"}));
    CHECK(d.indices.empty() && d.entropy == 0.0f && d.candidates.empty());
  });
  run("test_score_sorting_descending_with_stable_id_tiebreak", [] {  // determinism.rs:537-574
    Router router(3, 1.0f, 0.01f);
    auto info = infos({10, 200, 100, 300, 400});
    Decision d = router.route_with_adapter_info({}, {0.9f, 0.5f, 0.5f, 0.5f, 0.1f}, info,
                                                PolicyMask::allow_all(info.size()));
    CHECK(d.indices[0] == 0 && d.indices[1] == 2 && d.indices[2] == 1);
  });
  run("test_router_produces_zero_gates_for_masked_adapters", [] {  // q15_edge_cases.rs:74-135
    Router router(2, 1.0f, 0.02f);
    std::vector<AdapterInfo> info{{"adapter-1", 0}, {"adapter-2", 0}};
    Decision d = router.route_with_adapter_info({}, {1.0f, 1.0f}, info, PolicyMask::deny(info, {"adapter-2"}));
    CHECK(d.indices.size() == 1 && d.indices[0] == 0 && d.gates_q15[0] == 32767);
  });
  run("test_router_produces_max_gate_for_single_adapter", [] {  // q15_edge_cases.rs:155-192
    Router router(1, 1.0f, 0.02f);
    Decision d = router.route_with_adapter_info({}, {1.0f}, {{"adapter-1", 0}}, PolicyMask::allow_all(1));
    CHECK(d.indices.size() == 1 && d.gates_q15[0] == 32767 && d.gates_f32()[0] == 1.0f);
  });
  run("test_router_q15_gates_sum_correctly", [] {  // router/src/tests.rs:1402-1450 (deterministic mode)
    Router router(3, 1.0f, 0.02f);
    auto info = infos({0, 0, 0});
    Decision d = router.route_with_adapter_info({}, {1.0f, 1.0f, 1.0f}, info, PolicyMask::allow_all(3));
    int sum = 0;
    float sf = 0.0f;
    for (size_t i = 0; i < d.gates_q15.size(); ++i) {
      sum += d.gates_q15[i];
      sf += d.gates_f32()[i];
    }
    CHECK(std::fabs(sf - 1.0f) < 0.01f);
    CHECK(std::abs(sum - 32767) <= (int)d.gates_q15.size());
  });
  run("test_non_finite_prior_is_determinism_violation", [] {  // router.rs:611-625
    Router router(2, 1.0f, 0.02f);
    auto info = infos({0, 0, 0});
    CHECK(error_kind_of([&] { router.route_with_adapter_info({}, {0.1f, NAN, 0.3f}, info, PolicyMask::allow_all(3)); }) ==
          ErrorKind::DeterminismViolation);
  });

  run("mlx_lora_projection_math_and_gate_scaling", [] {  // mlx-ffi/src/lora_cpp_tests.rs:57-119
    // W = I (the 2x2 case inside a 32 x 64 int4 projection: q = 1, scale 1, bias 0),
    // x = [2, 3], A = [[1, 1]], B = [[1], [2]], alpha = rank = 1, gate q = 16384.
    HipKernels k(0, 1);
    const int out = 32, in = 64;
    std::vector<uint32_t> packed((size_t)out * in / 8, 0u);
    for (int o = 0; o < out; ++o) packed[(size_t)o * (in / 8) + o / 8] |= 1u << (4 * (o % 8));
    std::vector<uint16_t> scales((size_t)out, 0x3C00), biases((size_t)out, 0);
    k.set_base(0, "q_proj", out, in, packed.data(), scales.data(), biases.data());
    LoraModuleWeights w;
    w.in_features = in;
    w.out_features = out;
    w.A.assign(in, 0.0f);
    w.A[0] = w.A[1] = 1.0f;
    w.B.assign(out, 0.0f);
    w.B[0] = 1.0f;
    w.B[1] = 2.0f;
    k.load_adapter_with_metadata(1, {LoraLayerWeights{{"q_proj", w}}}, AdapterLoadMetadata{"a1", 1, 1.0f, {"q_proj"}});
    k.reserve(1);
    std::vector<uint16_t> xh(in, 0);
    xh[0] = 0x4000;  // bf16 2.0
    xh[1] = 0x4040;  // bf16 3.0
    RouterRing ring = RouterRing::with_k(1);
    ring.set({1}, {16384});
    aoship_ring_t rd = ring.to_device();
    uint16_t *dx, *dy;
    aoship_ring_t *dr;
    detail::hip_check(hipMalloc(&dx, in * 2), "hipMalloc");
    detail::hip_check(hipMalloc(&dy, out * 2), "hipMalloc");
    detail::hip_check(hipMalloc(&dr, sizeof(rd)), "hipMalloc");
    detail::hip_check(hipMemcpy(dx, xh.data(), in * 2, hipMemcpyHostToDevice), "hipMemcpy");
    detail::hip_check(hipMemcpy(dr, &rd, sizeof(rd), hipMemcpyHostToDevice), "hipMemcpy");
    auto forward = [&] {
      k.proj_forward(0, "q_proj", dx, 1, dr, dy);
      std::vector<uint16_t> yh(out);
      detail::hip_check(hipMemcpy(yh.data(), dy, out * 2, hipMemcpyDeviceToHost), "hipMemcpy");
      std::vector<float> y(out);
      for (int i = 0; i < out; ++i) {
        uint32_t u = (uint32_t)yh[i] << 16;
        std::memcpy(&y[i], &u, 4);
      }
      return y;
    };
    const float g = 16384.0f / 32767.0f;
    std::vector<float> y = forward();
    CHECK(std::fabs(y[0] - (2.0f + 5.0f * g)) < 2e-2f && std::fabs(y[1] - (3.0f + 10.0f * g)) < 4e-2f);
    for (int i = 2; i < out; ++i) CHECK(y[i] == 0.0f);
    // hot-swap: detached -> base only; attached again -> delta back; unloaded -> base only
    k.detach_adapter(1);
    y = forward();
    CHECK(y[0] == 2.0f && y[1] == 3.0f);
    k.attach_adapter(1);
    y = forward();
    CHECK(std::fabs(y[0] - (2.0f + 5.0f * g)) < 2e-2f);
    k.unload_adapter(1);
    y = forward();
    CHECK(y[0] == 2.0f && y[1] == 3.0f);
    CHECK(error_kind_of([&] { k.attach_adapter(1); }) == ErrorKind::Kernel);
    (void)hipFree(dx);
    (void)hipFree(dy);
    (void)hipFree(dr);
  });
  // router/src/tests.rs:856-925 with the C++ Router: exact ties select the first K of
  // (breaker, stable_id) order for each request seed, and the two seeds select differently
  run("adaptive_routing_applies_seeded_order_for_exact_ties", [] {
    const size_t n = 8, k = 3;
    std::vector<AdapterInfo> info;
    for (size_t i = 0; i < n; ++i) info.push_back({"adaptive_tie_adapter_" + std::to_string(i), i + 1, std::nullopt});
    std::vector<std::vector<uint16_t>> sel;
    for (uint8_t b : {1, 2}) {
      det::Bytes32 seed;
      seed.fill(b);
      const det::DeterminismContext ctx(seed, nullptr, det::RoutingDeterminismMode::Adaptive);
      std::vector<uint64_t> br(n);
      const det::Bytes32 ts = ctx.router_tiebreak_seed();
      CHECK(aoship_adaptive_tie_breakers(ts.data(), (int)n, br.data()) == 0);
      std::vector<uint16_t> order(n);
      for (size_t i = 0; i < n; ++i) order[i] = (uint16_t)i;
      std::sort(order.begin(), order.end(), [&](uint16_t a, uint16_t c) {
        return br[a] != br[c] ? br[a] < br[c] : info[a].stable_id < info[c].stable_id;
      });
      std::vector<uint16_t> want(order.begin(), order.begin() + k);
      std::sort(want.begin(), want.end());
      Router router(k, 1.0f, 0.02f);
      router.set_routing_determinism_mode(true);
      Decision d = router.route_with_adapter_info_with_ctx({}, std::vector<float>(n, 0.5f), info,
                                                           PolicyMask::allow_all(n), &ctx);
      std::vector<uint16_t> got = d.indices;
      std::sort(got.begin(), got.end());
      CHECK(got == want);
      sel.push_back(got);
      // without a determinism context adaptive routing is a configuration error (router.rs:1606-1612)
      CHECK(error_kind_of([&] {
              router.route_with_adapter_info({}, std::vector<float>(n, 0.5f), info, PolicyMask::allow_all(n));
            }) == ErrorKind::Config);
    }
    CHECK(sel[0] != sel[1]);
  });
  // router/src/tests.rs:928-972 (with an empty feature vector): the hash is filled in; its parts are
  // BLAKE3 of the priors, of the indices and gates, and of both hashes
  run("test_decision_hash_computation", [] {
    Router router(3, 1.0f, 0.02f);
    const std::vector<float> priors = {0.1f, 0.9f, 0.5f, 0.3f, 0.7f};
    std::vector<AdapterInfo> info;
    for (size_t i = 0; i < priors.size(); ++i) info.push_back({"adapter_" + std::to_string(i), 0, std::nullopt});
    Decision d = router.route_with_adapter_info({}, priors, info, PolicyMask::allow_all(priors.size()));
    CHECK(d.decision_hash.has_value());
    const DecisionHash &h = *d.decision_hash;
    CHECK(h.tau == 1.0f && h.eps == 0.02f && h.k == 3);
    std::vector<uint8_t> in(priors.size() * 4), out;
    std::memcpy(in.data(), priors.data(), in.size());
    for (uint16_t i : d.indices) {
      out.push_back((uint8_t)i);
      out.push_back((uint8_t)(i >> 8));
    }
    for (int16_t g : d.gates_q15) {
      out.push_back((uint8_t)(uint16_t)g);
      out.push_back((uint8_t)((uint16_t)g >> 8));
    }
    const det::B3Hash hin = det::B3Hash::hash(in.data(), in.size()), hout = det::B3Hash::hash(out.data(), out.size());
    std::vector<uint8_t> comb(hin.bytes.begin(), hin.bytes.end());
    comb.insert(comb.end(), hout.bytes.begin(), hout.bytes.end());
    CHECK(h.input_hash == hin.to_short_hex() && h.output_hash == hout.to_short_hex());
    CHECK(h.combined_hash == det::B3Hash::hash(comb.data(), comb.size()).to_short_hex());
    // reproducible, and off when the config says so (tests.rs:974-1110)
    Router again(3, 1.0f, 0.02f);
    Decision d2 = again.route_with_adapter_info({}, priors, info, PolicyMask::allow_all(priors.size()));
    CHECK(d2.decision_hash->combined_hash == h.combined_hash);
    RouterDeterminismConfig off;
    off.enable_decision_hashing = false;
    again.set_determinism_config(off);
    CHECK(!again.route_with_adapter_info({}, priors, info, PolicyMask::allow_all(priors.size())).decision_hash);
  });
  // worker_enforcement_tests.rs:127-215 through the router's decision policy
  run("routing_policy_on_decisions", [] {
    std::vector<AdapterInfo> info = {{"adapter_a", 0, std::nullopt}, {"adapter_b", 0, std::nullopt}};
    Router router(2, 1.0f, 0.02f);
    RoutingPolicy p;
    p.denied_adapter_ids = std::vector<std::string>{"adapter_b"};
    p.max_adapters_per_token = 2;
    router.set_decision_policy(&p, {"adapter_a", "adapter_b"}, {std::nullopt, std::nullopt});
    Decision d = router.route_with_adapter_info({}, {0.8f, 0.7f}, info, PolicyMask::allow_all(2));
    CHECK(d.indices == std::vector<uint16_t>{0} && d.gates_q15 == std::vector<int16_t>{32767});
    RoutingPolicy all;
    all.allowed_adapter_ids = std::vector<std::string>{"other"};
    router.set_decision_policy(&all, {"adapter_a", "adapter_b"}, {std::nullopt, std::nullopt});
    CHECK(error_kind_of([&] { router.route_with_adapter_info({}, {0.8f, 0.7f}, info, PolicyMask::allow_all(2)); }) ==
          ErrorKind::PolicyViolation);
    router.set_decision_policy(nullptr);
    CHECK(router.route_with_adapter_info({}, {0.8f, 0.7f}, info, PolicyMask::allow_all(2)).indices.size() == 2);
  });
  // router.rs:1587-1602: a scope hint keeps routing inside the matching adapters
  run("scope_hint", [] {
    std::vector<AdapterInfo> info = {{"a", 0, std::string("src/x")},
                                     {"b", 0, std::string("src/y")},
                                     {"c", 0, std::string("src/x")},
                                     {"d", 0, std::nullopt}};
    Router router(2, 1.0f, 0.02f);
    const std::vector<float> priors = {0.1f, 0.9f, 0.3f, 0.8f};
    const std::string hint = "src/x", none = "src/z";
    Decision d = router.route_with_adapter_info_and_scope_with_ctx({}, priors, info, PolicyMask::allow_all(4), &hint,
                                                                   nullptr);
    std::vector<uint16_t> got = d.indices;
    std::sort(got.begin(), got.end());
    CHECK((got == std::vector<uint16_t>{0, 2}));
    // a hint no adapter matches is ignored
    d = router.route_with_adapter_info_and_scope_with_ctx({}, priors, info, PolicyMask::allow_all(4), &none, nullptr);
    CHECK((d.indices == std::vector<uint16_t>{1, 3}));
  });
  run("device_name_and_attestation", [] {  // kernel-api/src/lib.rs:374, 383
    HipKernels k(0, 1);
    CHECK(k.device_name().find("gfx950") != std::string::npos);
    CHECK(k.attest_determinism().find("\"deterministic\":true") != std::string::npos);
  });
}

// ---- ingest: what the parser reads, as JSON for the Python side to check ----

std::string jstr(const std::string &s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    if ((unsigned char)c < 0x20) {
      char b[8];
      std::snprintf(b, sizeof b, "\\u%04x", (unsigned)(unsigned char)c);
      o += b;
      continue;
    }
    o += c;
  }
  return o + "\"";
}

template <class T>
std::string jlist(const std::vector<T> &v) {
  std::string o = "[";
  for (size_t i = 0; i < v.size(); ++i) o += (i ? "," : "") + std::to_string(v[i]);
  return o + "]";
}

std::vector<uint32_t> f32_bits(const std::vector<float> &v) {
  std::vector<uint32_t> b(v.size());
  std::memcpy(b.data(), v.data(), v.size() * 4);
  return b;
}

std::string read_text(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

int ingest_error(const ingest::IngestError &e) {
  std::printf("{\"error\":%s,\"message\":%s}\n",
              jstr(e.kind() == ingest::IngestError::Kind::Parse ? "Parse"
                   : e.kind() == ingest::IngestError::Kind::Io  ? "Io"
                                                                : "Validation")
                  .c_str(),
              jstr(e.what()).c_str());
  return 0;
}

void print_spec(const ingest::AdapterSpec &spec) {
    float alpha = spec.alpha, scale = spec.scale();
    uint32_t ab, sb;
    std::memcpy(&ab, &alpha, 4);
    std::memcpy(&sb, &scale, 4);
    std::string targets = "[";
    for (size_t i = 0; i < spec.target_modules.size(); ++i) targets += (i ? "," : "") + jstr(spec.target_modules[i]);
    targets += "]";
    std::string mods = "[";
    for (size_t i = 0; i < spec.modules.size(); ++i) {
      const auto &m = spec.modules[i];
      mods += (i ? "," : "") + std::string("{\"name\":") + jstr(m.name) + ",\"rank\":" + std::to_string(m.rank) +
              ",\"in\":" + std::to_string(m.in_features) + ",\"out\":" + std::to_string(m.out_features) +
              ",\"A\":" + jlist(f32_bits(m.A)) + ",\"B\":" + jlist(f32_bits(m.B)) + ",\"problem\":" + jstr(m.problem) +
              "}";
    }
    mods += "]";
    std::printf("{\"rank\":%" PRIu64 ",\"alpha_bits\":%u,\"scale_bits\":%u,\"target_modules\":%s,\"modules\":%s}\n",
                spec.rank, ab, sb, targets.c_str(), mods.c_str());
}

int ingest_adapter_mode(const std::string &file, const char *metadata_json) {
  try {
    const ingest::MappedFile f(file);
    const ingest::SafeTensors st = ingest::SafeTensors::parse(f.data(), f.size());
    ingest::Json md;
    if (metadata_json) md = ingest::parse_json(metadata_json);
    print_spec(ingest::read_adapter(st, metadata_json ? &md : nullptr));
  } catch (const ingest::IngestError &e) {
    return ingest_error(e);
  }
  return 0;
}

// LoRAAdapter::load with config (rank, alpha, comma-separated targets)
int ingest_lora_mode(const std::string &file, const char *rank, const char *alpha, const std::string &targets) {
  try {
    ingest::AdapterSpec cfg;
    cfg.rank = std::strtoull(rank, nullptr, 10);
    cfg.alpha = std::strtof(alpha, nullptr);
    cfg.target_modules.clear();
    size_t b = 0;
    while (b < targets.size()) {
      size_t e = targets.find(',', b);
      if (e == std::string::npos) e = targets.size();
      if (e > b) cfg.target_modules.push_back(targets.substr(b, e - b));
      b = e + 1;
    }
    print_spec(ingest::load_lora(file, cfg));
  } catch (const ingest::IngestError &e) {
    return ingest_error(e);
  }
  return 0;
}

int ingest_base_mode(const std::string &file, const std::string &key) {
  try {
    const ingest::MappedFile f(file);
    const ingest::SafeTensors st = ingest::SafeTensors::parse(f.data(), f.size());
    ingest::BaseProjection bp;
    if (!ingest::read_base(st, key, bp)) {
      std::printf("{\"found\":false}\n");
      return 0;
    }
    std::printf("{\"found\":true,\"out\":%d,\"in\":%d,\"packed\":%s,\"scales\":%s,\"biases\":%s}\n",
                bp.out_features, bp.in_features, jlist(bp.packed).c_str(), jlist(bp.scales_f16).c_str(),
                jlist(bp.biases_f16).c_str());
  } catch (const ingest::IngestError &e) {
    return ingest_error(e);
  }
  return 0;
}

// ---- seeds: the DeterminismContext chain for a request seed (hex) and an optional router seed text ----

int seeds_mode(const std::string &request_hex, const char *router_seed_text) {
  const std::optional<det::B3Hash> rs = det::B3Hash::from_hex(request_hex);
  if (!rs) {
    std::fprintf(stderr, "request seed must be 64 hex digits\n");
    return 2;
  }
  const det::DeterminismContext ctx =
      router_seed_text ? det::DeterminismContext(rs->bytes, std::string(router_seed_text), det::RoutingDeterminismMode::Adaptive)
                       : det::DeterminismContext(rs->bytes, nullptr, det::RoutingDeterminismMode::Adaptive);
  const det::Bytes32 ts = ctx.router_tiebreak_seed();
  const det::B3Hash manifest = det::B3Hash::hash("manifest");
  const det::DeterminismContext with_manifest(rs->bytes, &manifest, det::RoutingDeterminismMode::Adaptive);
  std::printf("{\"router_seed_hex\":%s,\"tiebreak_seed\":%s,\"router_seed_with_manifest\":%s,\"low64\":%llu}\n",
              jstr(ctx.router_seed_hex()).c_str(), jstr(det::B3Hash::hex(ts.data(), 32)).c_str(),
              jstr(with_manifest.router_seed_hex()).c_str(), (unsigned long long)ctx.request_seed_low64());
  return 0;
}

// ---- gpu-ingest: safetensors-loaded layers against array-loaded ones, bit for bit ----

template <class T>
std::vector<T> read_raw(const std::string &path, size_t n) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot open " + path);
  std::vector<T> v(n);
  f.read(reinterpret_cast<char *>(v.data()), (std::streamsize)(n * sizeof(T)));
  if ((size_t)f.gcount() != n * sizeof(T)) throw std::runtime_error("short read " + path);
  return v;
}

// DIR holds base.safetensors, adapter1.safetensors (+ adapter1.json metadata), adapter2.safetensors
// and the same arrays raw: L<l>.<module>.{packed,scales,biases}.bin, a<id>.<module>.{A,B}.bin.
int gpu_ingest_mode(const std::string &dir, int L, int H, int I, int KV, int r1, float alpha1, int r2) {
  const char *mods[] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"};
  auto shape = [&](const std::string &m, int &out, int &in) {
    in = m == "down_proj" ? I : H;
    out = (m == "gate_proj" || m == "up_proj") ? I : (m == "k_proj" || m == "v_proj") ? KV : H;
  };
  run("gpu_ingest_safetensors_matches_arrays", [&] {
    HipKernels ks(0, L), ka(0, L);
    const ingest::MappedFile base(dir + "/base.safetensors");
    CHECK(ks.load_base_safetensors(base.data(), base.size()) == 7 * L);
    for (int l = 0; l < L; ++l)
      for (const char *m : mods) {
        int out, in;
        shape(m, out, in);
        const std::string pre = dir + "/L" + std::to_string(l) + "." + m + ".";
        auto p = read_raw<uint32_t>(pre + "packed.bin", (size_t)out * in / 8);
        auto sc = read_raw<uint16_t>(pre + "scales.bin", (size_t)out * in / 64);
        auto bi = read_raw<uint16_t>(pre + "biases.bin", (size_t)out * in / 64);
        ka.set_base(l, m, out, in, p.data(), sc.data(), bi.data());
      }
    // adapter 1: prefix keys, metadata (rank, alpha) and an lm_head pair the device path skips
    const ingest::MappedFile a1(dir + "/adapter1.safetensors");
    const std::string md1 = read_text(dir + "/adapter1.json");
    const ingest::AdapterSpec s1 = ks.load_adapter_with_metadata(1, a1.data(), a1.size(), md1.c_str());
    CHECK(s1.rank == (uint64_t)r1 && s1.alpha == alpha1);
    CHECK(ks.load_warnings().size() == 1 && ks.load_warnings()[0].find("lm_head") != std::string::npos);
    // adapter 2: suffix keys, no metadata (rank 4, alpha 16)
    const ingest::MappedFile a2(dir + "/adapter2.safetensors");
    ks.load_adapter(2, a2.data(), a2.size());
    CHECK(ks.load_warnings().empty());
    auto arrays = [&](int id, const std::vector<std::string> &names, int r) {
      std::vector<LoraLayerWeights> w((size_t)L);
      for (const auto &m : names) {
        int out, in;
        shape(m, out, in);
        LoraModuleWeights mw;
        mw.in_features = in;
        mw.out_features = out;
        const std::string pre = dir + "/a" + std::to_string(id) + "." + m + ".";
        mw.A = read_raw<float>(pre + "A.bin", (size_t)r * in);
        mw.B = read_raw<float>(pre + "B.bin", (size_t)out * r);
        for (int l = 0; l < L; ++l) w[(size_t)l][m] = mw;
      }
      return w;
    };
    ka.load_adapter_with_metadata(1, arrays(1, {"q_proj", "v_proj", "o_proj", "gate_proj", "down_proj"}, r1),
                                  AdapterLoadMetadata{"a1", (uint32_t)r1, alpha1, {}});
    ka.load_adapter_with_metadata(2, arrays(2, {"k_proj", "up_proj"}, r2), AdapterLoadMetadata{"a2", 4, 16.0f, {}});
    const int Tmax = 40;
    ks.reserve(Tmax);
    ka.reserve(Tmax);
    auto x = read_raw<uint16_t>(dir + "/x.bin", (size_t)Tmax * I);
    uint16_t *dx, *dy1, *dy2, *dq1, *dq2;
    aoship_ring_t *dr;
    const size_t ybytes = (size_t)Tmax * I * 2;
    detail::hip_check(hipMalloc(&dx, x.size() * 2), "hipMalloc");
    detail::hip_check(hipMalloc(&dy1, ybytes), "hipMalloc");
    detail::hip_check(hipMalloc(&dy2, ybytes), "hipMalloc");
    detail::hip_check(hipMalloc(&dq1, 3 * ybytes), "hipMalloc");
    detail::hip_check(hipMalloc(&dq2, 3 * ybytes), "hipMalloc");
    detail::hip_check(hipMalloc(&dr, sizeof(aoship_ring_t) * Tmax), "hipMalloc");
    detail::hip_check(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice), "hipMemcpy");
    std::vector<aoship_ring_t> rings((size_t)Tmax);
    for (int t = 0; t < Tmax; ++t) {
      RouterRing ring = RouterRing::with_k(2);
      const int16_t g = (int16_t)(1000 + (t * 977) % 30000);
      ring.set({(uint16_t)(1 + t % 2), (uint16_t)(2 - t % 2)}, {g, (int16_t)(32767 - g)});
      rings[(size_t)t] = ring.to_device();
    }
    detail::hip_check(hipMemcpy(dr, rings.data(), sizeof(aoship_ring_t) * Tmax, hipMemcpyHostToDevice), "hipMemcpy");
    auto same = [&](const uint16_t *a, const uint16_t *b, size_t n) {
      std::vector<uint16_t> ha(n), hb(n);
      detail::hip_check(hipMemcpy(ha.data(), a, n * 2, hipMemcpyDeviceToHost), "hipMemcpy");
      detail::hip_check(hipMemcpy(hb.data(), b, n * 2, hipMemcpyDeviceToHost), "hipMemcpy");
      bool nonzero = false;
      for (size_t i = 0; i < n; ++i) nonzero = nonzero || (ha[i] & 0x7FFF);
      return nonzero && std::memcmp(ha.data(), hb.data(), n * 2) == 0;
    };
    for (int T : {1, 5, Tmax})
      for (int l = 0; l < L; ++l) {
        std::printf("  case T=%d layer=%d\n", T, l);
        std::fflush(stdout);
        ks.mlp_forward(l, dx, T, dr, dy1);
        ka.mlp_forward(l, dx, T, dr, dy2);
        CHECK(same(dy1, dy2, (size_t)T * H));
        ks.qkv_forward(l, dx, T, dr, dq1, dq1 + (size_t)T * H, dq1 + (size_t)T * (H + KV));
        ka.qkv_forward(l, dx, T, dr, dq2, dq2 + (size_t)T * H, dq2 + (size_t)T * (H + KV));
        CHECK(same(dq1, dq2, (size_t)T * (H + 2 * KV)));
        ks.proj_forward(l, "o_proj", dx, T, dr, dy1);
        ka.proj_forward(l, "o_proj", dx, T, dr, dy2);
        CHECK(same(dy1, dy2, (size_t)T * H));
      }
    for (void *p : {(void *)dx, (void *)dy1, (void *)dy2, (void *)dq1, (void *)dq2, (void *)dr}) (void)hipFree(p);
  });
  std::printf("gpu-ingest: %d failed\n", g_failed);
  return g_failed ? 1 : 0;
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  if (mode == "ingest-adapter" && (argc == 3 || argc == 4)) return ingest_adapter_mode(argv[2], argc == 4 ? argv[3] : nullptr);
  if (mode == "ingest-base" && argc == 4) return ingest_base_mode(argv[2], argv[3]);
  if (mode == "seeds" && (argc == 3 || argc == 4)) return seeds_mode(argv[2], argc == 4 ? argv[3] : nullptr);
  if (mode == "ingest-lora" && argc == 6) return ingest_lora_mode(argv[2], argv[3], argv[4], argv[5]);
  if (mode == "gpu-ingest" && argc == 10)
    return gpu_ingest_mode(argv[2], std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5]), std::atoi(argv[6]),
                           std::atoi(argv[7]), (float)std::atof(argv[8]), std::atoi(argv[9]));
  if (mode == "cpu")
    cpu_tests();
  else if (mode == "gpu")
    gpu_tests();
  else {
    std::fprintf(stderr,
                 "usage: %s cpu | gpu | ingest-adapter FILE [METADATA_JSON] | ingest-base FILE KEY |\n"
                 "       ingest-lora FILE RANK ALPHA TARGET[,TARGET...] | seeds REQUEST_SEED_HEX [ROUTER_SEED] |\n"
                 "       gpu-ingest DIR LAYERS HIDDEN INTERMEDIATE KV_OUT RANK1 ALPHA1 RANK2\n",
                 argv[0]);
    return 2;
  }
  std::printf("%s: %d failed\n", mode.c_str(), g_failed);
  return g_failed ? 1 : 0;
}
