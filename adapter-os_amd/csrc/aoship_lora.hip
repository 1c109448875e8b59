/*
 * aoship_lora.hip — the decode path's LoRA shrink launch (the shrink and the adapter plan
 * themselves are in aoship_shrink.h).
 *
 * The plan (union of the tokens' adapters and their coefficients) is built by one extra
 * workgroup of the first shrink launch, which needs no plan itself because it covers every
 * bound adapter.
 */
#include "aoship_shrink.h"
#include <hip/hip_ext.h>

namespace {

template <int NV, int W, int D>
__global__ void __launch_bounds__(64 * W) aos_shrink_kernel(aos_shrink_params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  aos_shrink::shrink_block<NV, W, D>(p, blockIdx.x, blockIdx.y, smem);
}

template <int NV>
int launch_nv(const aos_shrink_params *p, const aos_launch_ctx *ctx) {
  const int rb_total = p->n_rb[0] + (p->nmod > 1 ? p->n_rb[1] : 0) + (p->nmod > 2 ? p->n_rb[2] : 0);
  dim3 grid(rb_total + (p->plan_build.plan ? 1 : 0), p->ks);
  if (grid.x == 0) { /* no adapter rows and no plan to build (no bound adapter has the module) */
    AOS_SKIP(ctx);
    return 0;
  }
  AOS_LAUNCH(ctx, (aos_shrink_kernel<NV, 4, 4>), grid, dim3(256), (size_t)p->lds_bytes, *p);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int aos_launch_shrink(const aos_shrink_params *p, const aos_launch_ctx *ctx) {
  const int T = p->T;
  if (T < 1 || T > AOS_DECODE_MAX_T) return (int)hipErrorInvalidValue;
  if (T <= 1) return launch_nv<1>(p, ctx);
  if (T <= 2) return launch_nv<2>(p, ctx);
  if (T <= 8) return launch_nv<4>(p, ctx);
  if (T <= 16) return launch_nv<8>(p, ctx);
  return launch_nv<16>(p, ctx);
}

AOS_DEFINE_SPIN_SETTER(aos_spin_setter_lora)
