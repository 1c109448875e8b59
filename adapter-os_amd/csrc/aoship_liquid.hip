/*
 * aoship_liquid.hip — LiquidKernel::blend_and_forward on gfx950: the weighted sum of up to three
 * LoRA deltas applied to one activation vector (crates/adapteros-lora-kernel-api/src/liquid.rs:
 * 147-160; result of blend_and_forward_reference, :163-257):
 *     output[o] = sum over adapters a with coef_a != 0 of
 *                 coef_a * (up_a[o, :] . (down_a . input)) * (alpha_a / rank_a),   o < up_a.rows
 *
 * One launch, no cross-workgroup hand-off: every workgroup forms the rank vectors down_a . input
 * (at most 3 x 1024 values) in LDS, each row by one wave in a fixed order (lane l sums elements
 * l, l + 64, ... in order, then a xor butterfly), so every workgroup holds the same values run to
 * run. It then writes its share of the outputs, one thread per output row, adapters in order.
 * The grid is bounded so that the repeated shrink reads at most about 8M weight elements in
 * total (L2 and last-level-cache hits after the first workgroups).
 */
#include "aoship_device.h"
#include "aoship_internal.h"
#include <hip/hip_ext.h>

namespace {

__device__ __forceinline__ float liquid_at(const void *p, int bf16, size_t i) {
  return bf16 ? aos_bf16_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

constexpr int LQ_NT = 512;

__global__ void __launch_bounds__(LQ_NT) aos_liquid_kernel(aos_liquid_params p) {
  __shared__ float rb[AOS_LIQUID_MAX][AOS_LIQUID_RANK_MAX];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), nw = LQ_NT / 64;
  /* the rank vectors: row j of the concatenated ranks belongs to adapter a */
  const int rows = p.rank[0] + p.rank[1] + p.rank[2];
  for (int row = wave; row < rows; row += nw) {
    int a = 0, r = row;
    while (a < AOS_LIQUID_MAX - 1 && r >= p.rank[a]) {
      r -= p.rank[a];
      ++a;
    }
    if (p.coef[a] == 0.0f) continue; /* skipped adapters contribute nothing (uniform) */
    const size_t base = (size_t)r * p.in;
    float acc = 0.0f;
    for (int c = lane; c < p.in; c += 64) acc += liquid_at(p.down[a], p.down_bf16[a], base + c) * p.x[c];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc = acc + aos_shfl_f(acc, lane ^ o);
    if (lane == 0) rb[a][r] = acc;
  }
  __syncthreads();
  for (int o = blockIdx.x * LQ_NT + tid; o < p.out_len; o += gridDim.x * LQ_NT) {
    float out = 0.0f;
    for (int a = 0; a < p.n; ++a) {
      if (p.coef[a] == 0.0f || o >= p.up_rows[a]) continue;
      const int rk = p.rank[a];
      const size_t base = (size_t)o * rk;
      float acc = 0.0f;
      for (int j = 0; j < rk; ++j) acc += liquid_at(p.up[a], p.up_bf16[a], base + j) * rb[a][j];
      out += p.coef[a] * acc * p.scaling[a];
    }
    p.y[o] = out;
  }
}

}  // namespace

extern "C" int aos_launch_liquid(const aos_liquid_params *p, const aos_launch_ctx *ctx) {
  if (p->n < 1 || p->n > AOS_LIQUID_MAX || p->in < 0 || p->out_len < 1) return (int)hipErrorInvalidValue;
  size_t shrink = 0;
  for (int a = 0; a < AOS_LIQUID_MAX; ++a) {
    if (p->rank[a] < 0 || p->rank[a] > AOS_LIQUID_RANK_MAX || (a >= p->n && p->rank[a] != 0))
      return (int)hipErrorInvalidValue;
    shrink += (size_t)p->rank[a] * (size_t)p->in;
  }
  int grid = (p->out_len + LQ_NT - 1) / LQ_NT;
  const size_t budget = (size_t)8 << 20; /* weight elements re-read by the whole grid */
  const size_t cap = shrink > 0 ? budget / shrink : (size_t)grid;
  if ((size_t)grid > cap) grid = cap > 0 ? (int)cap : 1;
  if (grid > 256) grid = 256;
  AOS_LAUNCH(ctx, aos_liquid_kernel, dim3(grid), dim3(LQ_NT), 0, *p);
  return (int)hipGetLastError();
}

AOS_DEFINE_SPIN_SETTER(aos_spin_setter_liquid)
