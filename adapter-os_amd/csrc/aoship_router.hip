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
#include "aoship_device.h"
#include "aoship_gemv.h"
#include "aoship_internal.h"
#include "aoship_route.h"
#include <hip/hip_ext.h>

namespace {

/* Routing from priors already in memory: one wave per token. */
template <bool X>
__global__ void __launch_bounds__(64) aos_route_kernel(aos_route_params p) {
  const int t = blockIdx.x;
  route_one<false, X>(p, p.priors_in + (size_t)t * p.n, t, threadIdx.x);
}

/* Routing from router features: one workgroup per token; wave w computes the priors of
 * adapters w, w + W, ... into LDS (and priors_out), then wave 0 routes. */
template <bool X>
__device__ __forceinline__ void route_features_block(const aos_route_params &p, int t, float *lds) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  float *lds_f = lds, *lds_priors = lds + p.d;
  /* the loads of the wave's first weight row and, in wave 0, of the selection's per-adapter
   * inputs go out before the features are staged */
  const int nk = p.d >> 8;
  float4 wv[16];
  if (nk > 0 && wave < p.n) dot_load(p.router_w + (size_t)wave * p.d, 0, nk, lane, wv);
  RouteMeta meta = {1, 1, 0ull};
  if (wave == 0) meta = route_meta<X>(p, lane);
  const float4 *f4 = (const float4 *)(p.features + (size_t)t * p.d);
  for (int e = threadIdx.x; e < p.d / 4; e += blockDim.x) ((float4 *)lds_f)[e] = f4[e];
  __syncthreads();
  for (int a = wave; a < p.n; a += nw) {
    const float *wr = p.router_w + (size_t)a * p.d;
    if (a != wave && nk > 0) dot_load(wr, 0, nk, lane, wv);
    const float v = dot_finish(lds_f, wr, p.d, lane, wv);
    if (lane == 0) {
      lds_priors[a] = v;
      if (p.priors_out) p.priors_out[(size_t)t * p.n + a] = v;
    }
  }
  __syncthreads();
  if (wave == 0) route_one<true, X>(p, lds_priors, t, lane, &meta);
}

template <bool X>
__global__ void __launch_bounds__(1024) aos_route_features_kernel(aos_route_params p) {
  extern __shared__ float lds[]; /* features [d], then priors [n] */
  route_features_block<X>(p, blockIdx.x, lds);
}

/* The router's workgroups (one per token, the plain router), then the x shrink and the gate/up
 * GEMV of the layer those rings feed: the shrink does not depend on the rings, so it and the
 * weight stream run while the tokens are routed; only the adapter plan, and through it the
 * GEMV's LoRA expand, waits for them. */
/* Part r of token t's routing in the route + gate/up launch (rparts > 1, 4 waves): wave w computes
 * the priors of adapters 4 r + w, 4 (r + rparts) + w, ... exactly as route_features_block does
 * (same loads, order and butterfly), stores them device-coherently and counts the workgroup in on
 * the token's line; the last part loads the token's priors into LDS and routes it. Returns true in
 * the workgroup that routed the token. */
__device__ __forceinline__ bool route_part_block(const aos_route_gu_params &q, int t, int r, float *lds) {
  const aos_route_params &p = q.rp;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int R = q.rparts;
  float *lds_f = lds, *lds_priors = lds + p.d;
  const int nk = p.d >> 8;
  const int a0 = 4 * r + wave;
  float4 wv[16];
  if (nk > 0 && a0 < p.n) dot_load(p.router_w + (size_t)a0 * p.d, 0, nk, lane, wv);
  RouteMeta meta = {1, 1, 0ull};
  if (wave == 0) meta = route_meta<false>(p, lane);
  const float4 *f4 = (const float4 *)(p.features + (size_t)t * p.d);
  for (int e = threadIdx.x; e < p.d / 4; e += blockDim.x) ((float4 *)lds_f)[e] = f4[e];
  __syncthreads();
  float *pri = q.rpri + (size_t)t * AOS_ROUTE_PARTS_MAXN;
  for (int a = a0; a < p.n; a += 4 * R) {
    const float *wr = p.router_w + (size_t)a * p.d;
    if (a != a0 && nk > 0) dot_load(wr, 0, nk, lane, wv);
    const float v = dot_finish(lds_f, wr, p.d, lane, wv);
    if (lane == 0) {
      aos_publish(pri + a, v);
      if (p.priors_out) p.priors_out[(size_t)t * p.n + a] = v;
    }
  }
  aos_mem_wait();
  __syncthreads();
  uint32_t *last = (uint32_t *)(lds_priors + p.n); /* the LDS word after the priors */
  uint32_t *ctr = q.rpart_ctr + (size_t)t * 32;
  if (threadIdx.x == 0) {
    *last = aos_arrive(ctr) == (uint32_t)R - 1u ? 1u : 0u;
    if (*last) aos_reset(ctr);
  }
  __syncthreads();
  if (!*last) return false;
  for (int a = threadIdx.x; a < p.n; a += blockDim.x) lds_priors[a] = aos_collect(pri + a);
  __syncthreads();
  if (wave == 0) route_one<true, false>(p, lds_priors, t, lane, &meta);
  return true;
}

/* LDS offset of the plan's staged tables in a router workgroup: after the features, the priors and
 * the arrival word */
__host__ __device__ constexpr size_t rgu_tabs_off(int d, int n) { return ((size_t)(d + n + 4) * 4 + 15) & ~(size_t)15; }

template <int NV>
__global__ void __launch_bounds__(256) aos_route_gu_kernel(aos_route_gu_params q) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int T = q.rp.T, R = q.rparts;
  const int b = blockIdx.x;
  /* with per-producer lines and at most AOS_PLAN_TABS_N adapters (the split router), the router
   * that finishes the last token builds the plan itself and raises the plan workgroup's line; the
   * plan workgroup then stands aside */
  const bool plan_by_router = q.fp.lines != nullptr && q.fp.sp.plan_build.plan != nullptr && R > 1 &&
                              q.rp.n <= AOS_PLAN_TABS_N;
  if (b < T * R) {
    const int t = b / R;
    aos_shrink::PlanTabs *lt = (aos_shrink::PlanTabs *)(smem + rgu_tabs_off(q.rp.d, q.rp.n));
    aos_shrink::PlanTabRegs tr = {};
    if (plan_by_router) tr = aos_shrink::plan_tabs_fetch(q.fp.sp.plan_build);
    if (R > 1) {
      if (!route_part_block(q, t, b - t * R, (float *)smem)) return;
    } else {
      route_features_block<false>(q.rp, t, (float *)smem);
    }
    if (plan_by_router) aos_shrink::plan_tabs_store(q.fp.sp.plan_build, tr, lt); /* read after the barriers below */
    /* one token whose router builds the plan: from its own ring, which no other workgroup reads.
     * Otherwise the ring (plain stores of wave 0) is written again with device-scope stores, which
     * the plan's device-scope loads see, and the routers count in. */
    const bool solo = plan_by_router && T == 1;
    __syncthreads();
    if (!solo) {
      uint32_t *rw = (uint32_t *)(q.rp.rings + t);
      if (threadIdx.x < 10)
        __hip_atomic_store(rw + threadIdx.x, rw[threadIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      aos_mem_wait();
    }
    __shared__ uint32_t last_router;
    __syncthreads();
    /* the last router to finish resets the count, builds the plan (or has the plan workgroup build
     * it) and raises the launch's routing flag */
    if (threadIdx.x == 0) {
      last_router = solo ? 1u : (aos_arrive(q.route_done) == (uint32_t)T - 1u ? 1u : 0u);
      if (last_router && !solo) aos_reset(q.route_done);
    }
    __syncthreads();
    if (!last_router) return;
    if (plan_by_router) {
      aos_shrink::build_plan(q.fp.sp.plan_build, lt, solo);
      aos_mem_wait();
      __syncthreads();
      if (threadIdx.x == 0) aos_raise(q.fp.lines + (size_t)(q.fp.pre_rows - 1) * 32, q.fp.gen);
    }
    if (threadIdx.x == 0) aos_raise(q.route_flag, q.fp.gen);
    return;
  }
  const int b2 = b - T * R;
  if (b2 < q.fp.n_pre) {
    if (plan_by_router && b2 % q.fp.pre_rows == q.fp.pre_rows - 1) return; /* the plan workgroup */
    aos_gemv::fused_producer<NV, 4>(q.fp, b2, smem, q.route_flag);
    return;
  }
  const int r = b2 - q.fp.n_pre;
  aos_gemv::gemv_body<NV, true, 4, 4, false, true, true>(q.fp.gp[0], r % q.fp.gp[0].nrbg, r / q.fp.gp[0].nrbg);
}

template <int NV>
int launch_rgu(const aos_route_gu_params *q, const aos_launch_ctx *ctx) {
  const int nwg = q->rp.T * q->rparts + q->fp.n_pre + (int)q->fp.n_cons;
  size_t lds = rgu_tabs_off(q->rp.d, q->rp.n) + sizeof(aos_shrink::PlanTabs);
  if ((size_t)q->fp.sp.lds_bytes > lds) lds = (size_t)q->fp.sp.lds_bytes;
  if ((size_t)q->fp.gp[0].lds_bytes > lds) lds = (size_t)q->fp.gp[0].lds_bytes;
  AOS_LAUNCH(ctx, aos_route_gu_kernel<NV>, dim3(nwg), dim3(256), lds, *q);
  return (int)hipGetLastError();
}

}  // namespace

static_assert(sizeof(aos_route_gu_params) <= 4096, "kernel arguments");

extern "C" int aos_launch_route_gate_up(const aos_route_gu_params *q, const aos_launch_ctx *ctx) {
  const aos_gemv_fused_params &fp = q->fp;
  const int T = q->rp.T;
  if (T < 1 || T > AOS_DECODE_MAX_T || !q->rp.features || !q->route_done || !q->route_flag || !q->fp.gen)
    return (int)hipErrorInvalidValue;
  if (q->rp.scope || q->rp.tie_key || q->rp.post_allowed || q->rp.active_ids || q->rp.strengths || q->rp.hashes ||
      q->rp.decisions)
    return (int)hipErrorInvalidValue; /* the plain router only */
  if (!aos_fused_params_ok(&fp, 1) || fp.hsum || fp.gp[0].T != T || !fp.sp.plan_build.plan)
    return (int)hipErrorInvalidValue;
  if ((size_t)(q->rp.d + q->rp.n) * sizeof(float) > 60 * 1024) return (int)hipErrorInvalidValue;
  if (q->rparts < 1 || q->rparts > 16 || (q->rparts > 1 && (q->rp.n > AOS_ROUTE_PARTS_MAXN ||
                                                           4 * q->rparts < q->rp.n || !q->rpart_ctr || !q->rpri)))
    return (int)hipErrorInvalidValue;
  if (T <= 1) return launch_rgu<1>(q, ctx);
  if (T <= 2) return launch_rgu<2>(q, ctx);
  if (T <= 8) return launch_rgu<4>(q, ctx);
  if (T <= 16) return launch_rgu<8>(q, ctx);
  return launch_rgu<16>(q, ctx);
}

extern "C" int aos_launch_route(const aos_route_params *p, const aos_launch_ctx *ctx) {
  const bool x =
      p->scope || p->tie_key || p->post_allowed || p->active_ids || p->strengths || p->hashes || p->decisions;
  if (p->features) {
    const int waves = p->n < 16 ? p->n : 16;
    const size_t lds = (size_t)(p->d + p->n) * sizeof(float);
    if (x) AOS_LAUNCH(ctx, aos_route_features_kernel<true>, dim3(p->T), dim3(64 * waves), lds, *p);
    else AOS_LAUNCH(ctx, aos_route_features_kernel<false>, dim3(p->T), dim3(64 * waves), lds, *p);
  } else {
    if (x) AOS_LAUNCH(ctx, aos_route_kernel<true>, dim3(p->T), dim3(64), 0, *p);
    else AOS_LAUNCH(ctx, aos_route_kernel<false>, dim3(p->T), dim3(64), 0, *p);
  }
  return (int)hipGetLastError();
}

AOS_DEFINE_SPIN_SETTER(aos_spin_setter_router)
