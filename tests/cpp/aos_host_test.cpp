// C++ host-side tests of adapter-os_amd/host/aos_kernel_api.hpp, written like the reference's own
// Rust tests they restate (each names its source). Mode "cpu" runs the tests that touch no GPU;
// mode "gpu" runs the device ones. Prints "ok <name>" per test; exits 1 on the first failure.
#include <cmath>
#include <cstdio>
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
  run("device_name_and_attestation", [] {  // kernel-api/src/lib.rs:374, 383
    HipKernels k(0, 1);
    CHECK(k.device_name().find("gfx950") != std::string::npos);
    CHECK(k.attest_determinism().find("\"deterministic\":true") != std::string::npos);
  });
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  if (mode == "cpu")
    cpu_tests();
  else if (mode == "gpu")
    gpu_tests();
  else {
    std::fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
    return 2;
  }
  std::printf("%s: %d failed\n", mode.c_str(), g_failed);
  return g_failed ? 1 : 0;
}
