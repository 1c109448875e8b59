/*
 * aoship_gemv.hip — decode path (T <= 32 tokens): int4 GEMV + fused LoRA expand (+ SwiGLU).
 *
 * Computes, per output row o and token t, the MLX forward's
 *   linear(x, W) + apply_lora(x)                    (mlx_cpp_wrapper_real.cpp:3372-3419)
 * and in SwiGLU mode h = (g * sigmoid(g)) * u for the gate/up pair (:3509-3522).
 *
 * HBM-bound design for gfx950:
 *   - weights stream in the q4-tile layout: one 16-byte load per lane brings a full 1 KiB
 *     chunk (32 rows x one 64-element group);
 *   - each wave keeps D groups of loads in flight in a register ring (refilled as it consumes
 *     them); x is staged once per workgroup in LDS, where the per-group sums of x used by the
 *     bias term are also formed;
 *   - nibbles become bfloat16 (128 + q) with one and-or per pair (exact), and
 *     v_mfma_f32_32x32x16_bf16 forms t = sum (128 + q) x per group with the tokens as the M
 *     dimension (padded to 32); the group's scale and bias are applied to the accumulator:
 *         y += s * t + (b - 128 s) * sum(x over the group)
 *     so no per-element dequantisation arithmetic is needed;
 *   - K is split across the W waves of a workgroup and across ks workgroups per row block; the
 *     LoRA expand sum_u coef(t, u) S[t, u] B_u[o, :] (S from the shrink launch before) is added
 *     by the row block's workgroups, which take the (adapter, 16-rank) steps round-robin over
 *     workgroups and waves; in the SwiGLU kernel each wave loads its first step's operands before
 *     its K loop, so the expand adds no memory round trip at the end; all partials are summed in a fixed order
 *     (waves through LDS, workgroups by the last one to finish), so results are bit-identical
 *     run to run with no floating-point atomics.
 */
#include "aoship_gemv.h"
#include <hip/hip_ext.h>

namespace {

using namespace aos_gemv;

template <int NV, bool SW, int W, int D>
__global__ void __launch_bounds__(64 * W) aos_gemv_kernel(aos_gemv_params p) {
  gemv_body<NV, SW, W, D>(p, blockIdx.x, blockIdx.y);
}

/* Up to three matrices sharing x (q, k and v) in one launch: workgroup b of the 1-D grid is row
 * block b % RB, K split b / RB of the matrix whose range of workgroups holds it. */
template <int NV, int W, int D>
__global__ void __launch_bounds__(64 * W) aos_gemv3_kernel(aos_gemv3_params mp) {
  const int b = blockIdx.x;
  if (b < mp.wg_end[0]) {
    gemv_body<NV, false, W, D>(mp.p[0], b % mp.p[0].nrbg, b / mp.p[0].nrbg);
  } else if (b < mp.wg_end[1]) {
    const int r = b - mp.wg_end[0];
    gemv_body<NV, false, W, D>(mp.p[1], r % mp.p[1].nrbg, r / mp.p[1].nrbg);
  } else {
    const int r = b - mp.wg_end[1];
    gemv_body<NV, false, W, D>(mp.p[2], r % mp.p[2].nrbg, r / mp.p[2].nrbg);
  }
}

/* A shrink (workgroups [0, n_pre)) and the GEMVs consuming its S (the rest) in one launch. Each
 * shrink workgroup, once its stores are complete, counts itself into sync; the last one raises
 * every GEMV workgroup's ready flag. */
template <int NV, bool SW, int W, int D>
__global__ void __launch_bounds__(64 * W) aos_gemv_fused_kernel(aos_gemv_fused_params fp) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int b = blockIdx.x;
  if (b < fp.n_pre) {
    fused_producer<NV, W>(fp, b, smem, nullptr);
    return;
  }
  int r = b - fp.n_pre, m = 0;
  if (!SW && r >= fp.wg_end[0]) {
    m = r < fp.wg_end[1] ? 1 : 2;
    r -= fp.wg_end[m - 1];
  }
  /* matrix m's parameters read in place from the argument segment (fp is its first and only
   * argument): one call site for the three matrices */
  const aos_gemv_params &g = *(const aos_gemv_params *)((const char *)__builtin_amdgcn_kernarg_segment_ptr() +
                                                        offsetof(aos_gemv_fused_params, gp) +
                                                        (size_t)m * sizeof(aos_gemv_params));
  gemv_body<NV, SW, W, D>(g, r % g.nrbg, r / g.nrbg);
}

/* The decode MLP of 1-2 tokens in one launch (4-wave workgroups throughout):
 *   [0, gu.n_pre)             the x shrink and the plan (gate/up's producers);
 *   next gu.n_cons            the gate/up GEMV with its expand; h and the h shrink's partials go
 *                             out device-coherent, and the last row block raises hflags;
 *   next dn.n_pre             the sum of those partials (each waits for its line of hflags);
 *   last dn.n_cons            the down GEMV: weights first, then h once its line of hflags is
 *                             raised, then the expand once the sums are out (dn's flags).
 * Every wait is for workgroups with lower ids: those are dispatched first and wait on none of
 * the later ones, so the grid drains whatever the residency. */
#ifndef AOS_MLP_GU_RING
#define AOS_MLP_GU_RING 4 /* groups in flight per wave: gate/up GEMV of the one-launch MLP */
#endif
#ifndef AOS_MLP_DN_RING
#define AOS_MLP_DN_RING 12 /* ... and its down GEMV */
#endif
template <int NV>
__global__ void __launch_bounds__(256) aos_decode_mlp_kernel(aos_decode_mlp_params mp) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const aos_gemv_fused_params &gu = mp.gu, &dn = mp.dn;
  int b = blockIdx.x;
  if (b < gu.n_pre) {
    fused_producer<NV, 4>(gu, b, smem, nullptr);
    return;
  }
  b -= gu.n_pre;
  if (b < (int)gu.n_cons) {
    gemv_body<NV, true, 4, AOS_MLP_GU_RING, false, false>(gu.gp[0], b % gu.gp[0].nrbg, b / gu.gp[0].nrbg);
    return;
  }
  b -= (int)gu.n_cons;
  if (b < dn.n_pre) {
    fused_producer<NV, 4>(dn, b, smem, nullptr, mp.hflags + (size_t)b * 32);
    return;
  }
  b -= dn.n_pre;
  gemv_body<NV, false, 4, AOS_MLP_DN_RING, true>(dn.gp[0], b % dn.gp[0].nrbg, b / dn.gp[0].nrbg,
                                    mp.hflags + (size_t)(dn.n_pre + b) * 32);
}

template <int NV>
int launch_mlp_nv(const aos_decode_mlp_params *mp, const aos_launch_ctx *ctx) {
  const int nwg = mp->gu.n_pre + (int)mp->gu.n_cons + mp->dn.n_pre + (int)mp->dn.n_cons;
  size_t lds = (size_t)mp->gu.sp.lds_bytes;
  const size_t l_hs = (size_t)HSUM_V * 64 * 4 * 4;
  const size_t roles[3] = {(size_t)mp->gu.gp[0].lds_bytes, l_hs, (size_t)mp->dn.gp[0].lds_bytes};
  for (size_t r : roles) lds = lds > r ? lds : r;
  AOS_LAUNCH(ctx, aos_decode_mlp_kernel<NV>, dim3(nwg), dim3(256), lds, *mp);
  return (int)hipGetLastError();
}

#ifndef AOS_GU_RING
#define AOS_GU_RING 4 /* groups in flight per wave: gate/up GEMV */
#endif
#ifndef AOS_ONE_RING
#define AOS_ONE_RING 4 /* ... single-matrix GEMVs (measured: 12 in flight lengthen every dependent round trip) */
#endif
template <int NV>
int launchf_nv(const aos_gemv_fused_params *fp, int swiglu, const aos_launch_ctx *ctx) {
  const int nwg = fp->n_pre + (int)fp->n_cons;
  size_t lds = fp->hsum ? (size_t)HSUM_V * 64 * (fp->gp[0].waves) * 4 : (size_t)fp->sp.lds_bytes;
  for (int i = 0; i < fp->n; ++i) lds = lds > (size_t)fp->gp[i].lds_bytes ? lds : (size_t)fp->gp[i].lds_bytes;
  if (swiglu) {
    AOS_LAUNCH(ctx, (aos_gemv_fused_kernel<NV, true, 4, AOS_GU_RING>), dim3(nwg), dim3(256), lds, *fp);
  } else if (fp->gp[0].waves == 4) {
    AOS_LAUNCH(ctx, (aos_gemv_fused_kernel<NV, false, 4, AOS_ONE_RING>), dim3(nwg), dim3(256), lds, *fp);
  } else {
    AOS_LAUNCH(ctx, (aos_gemv_fused_kernel<NV, false, 8, AOS_ONE_RING>), dim3(nwg), dim3(512), lds, *fp);
  }
  return (int)hipGetLastError();
}

template <int NV>
int launch3_nv(const aos_gemv3_params *mp, const aos_launch_ctx *ctx) {
  const int nwg = mp->wg_end[mp->n - 1];
  size_t lds = 0;
  for (int i = 0; i < mp->n; ++i) lds = lds > (size_t)mp->p[i].lds_bytes ? lds : (size_t)mp->p[i].lds_bytes;
  if (mp->p[0].waves == 4) {
    AOS_LAUNCH(ctx, (aos_gemv3_kernel<NV, 4, 12>), dim3(nwg), dim3(256), lds, *mp);
  } else {
    AOS_LAUNCH(ctx, (aos_gemv3_kernel<NV, 8, 12>), dim3(nwg), dim3(512), lds, *mp);
  }
  return (int)hipGetLastError();
}

template <int NV>
int launch_nv(const aos_gemv_params *p, int swiglu, const aos_launch_ctx *ctx) {
  dim3 grid(p->nrbg, p->ks);
  const size_t lds = p->lds_bytes;
  if (swiglu) {
    AOS_LAUNCH(ctx, (aos_gemv_kernel<NV, true, 4, 4>), grid, dim3(256), lds, *p);
  } else if (p->waves == 4) {
    AOS_LAUNCH(ctx, (aos_gemv_kernel<NV, false, 4, 12>), grid, dim3(256), lds, *p);
  } else {
    AOS_LAUNCH(ctx, (aos_gemv_kernel<NV, false, 8, 12>), grid, dim3(512), lds, *p);
  }
  return (int)hipGetLastError();
}

}  // namespace

/* Row-block groups of a GEMV: wr divides the waves, nrbg = ceil(RB / wr), and the h shrink and
 * the one-launch hand-off (which use the workgroup's LDS per row block) only with wr == 1. */
static bool rbg_ok(const aos_gemv_params &p) {
  if (p.wr < 1 || p.waves % p.wr || p.w0.RB < 1 || p.nrbg != (p.w0.RB + p.wr - 1) / p.wr) return false;
  return p.wr == 1 || (!p.hpart && !p.hdone);
}

extern "C" int aos_launch_gemv(const aos_gemv_params *p, int swiglu, const aos_launch_ctx *st) {
  const int waves = p->waves;
  if (waves != 4 && waves != 8) return (int)hipErrorInvalidValue;
  if (!rbg_ok(*p)) return (int)hipErrorInvalidValue;
  if (swiglu && waves != 4) return (int)hipErrorInvalidValue;
  const int T = p->T;
  if (T < 1 || T > AOS_DECODE_MAX_T) return (int)hipErrorInvalidValue;
  if (T <= 1) return launch_nv<1>(p, swiglu, st);
  if (T <= 2) return launch_nv<2>(p, swiglu, st);
  if (T <= 8) return launch_nv<4>(p, swiglu, st);
  if (T <= 16) return launch_nv<8>(p, swiglu, st);
  return launch_nv<16>(p, swiglu, st);
}

extern "C" int aos_launch_gemv3(const aos_gemv3_params *mp, const aos_launch_ctx *st) {
  const int n = mp->n;
  if (n < 1 || n > 3) return (int)hipErrorInvalidValue;
  const int waves = mp->p[0].waves, T = mp->p[0].T;
  if (waves != 4 && waves != 8) return (int)hipErrorInvalidValue;
  if (T < 1 || T > AOS_DECODE_MAX_T) return (int)hipErrorInvalidValue;
  int end = 0;
  for (int i = 0; i < 3; ++i) {
    if (i < n) {
      const aos_gemv_params &p = mp->p[i];
      if (p.waves != waves || p.T != T || !rbg_ok(p) || p.ks < 1) return (int)hipErrorInvalidValue;
      end += p.nrbg * p.ks;
    }
    if (mp->wg_end[i] != end) return (int)hipErrorInvalidValue;
  }
  if (T <= 1) return launch3_nv<1>(mp, st);
  if (T <= 2) return launch3_nv<2>(mp, st);
  if (T <= 8) return launch3_nv<4>(mp, st);
  if (T <= 16) return launch3_nv<8>(mp, st);
  return launch3_nv<16>(mp, st);
}

extern "C" int aos_launch_gemv_fused(const aos_gemv_fused_params *fp, int swiglu, const aos_launch_ctx *st) {
  if (!aos_fused_params_ok(fp, swiglu)) return (int)hipErrorInvalidValue;
  const int T = fp->gp[0].T;
  if (T <= 1) return launchf_nv<1>(fp, swiglu, st);
  if (T <= 2) return launchf_nv<2>(fp, swiglu, st);
  if (T <= 8) return launchf_nv<4>(fp, swiglu, st);
  if (T <= 16) return launchf_nv<8>(fp, swiglu, st);
  return launchf_nv<16>(fp, swiglu, st);
}

/* Checks of one fused parameter block's own consistency (shared by the fused, the route + gate/up
 * and the one-launch MLP launchers). */
extern "C" int aos_fused_params_ok(const aos_gemv_fused_params *fp, int swiglu) {
  const int n = fp->n;
  if (n < 1 || n > 3 || (swiglu && n != 1)) return false;
  const int waves = fp->gp[0].waves, T = fp->gp[0].T;
  if (waves != 4 && waves != 8) return false;
  if (swiglu && waves != 4) return false;
  if (T < 1 || T > AOS_DECODE_MAX_T || (fp->hsum ? fp->hs.T : fp->sp.T) != T) return false;
  if (!fp->gen || fp->n_pre < 1 || fp->pre_rows < 1 || fp->n_pre % fp->pre_rows) return false;
  const bool lines = fp->lines != nullptr;
  /* per-producer lines: one per row block of the shrink (and the plan) or per sum workgroup;
   * the plan's line is the last when the shrink builds the plan */
  const int plan_line = (!fp->hsum && fp->sp.plan_build.plan) ? fp->pre_rows - 1 : -1;
  if (lines) {
    if (fp->n_lines != (fp->hsum ? fp->n_pre : fp->pre_rows)) return false;
    if (fp->hsum ? (fp->hs.lines != fp->lines || fp->hs.gen != fp->gen)
                 : (fp->sp.lines != fp->lines || fp->sp.gen != fp->gen))
      return false;
  } else if (!fp->sync || !fp->flags || (fp->hsum ? fp->hs.lines != nullptr : fp->sp.lines != nullptr)) {
    return false;
  }
  if (fp->hsum ? (fp->pre_rows != fp->n_pre || !fp->hs.hpart || !fp->hs.S || fp->hs.values_per_wg != HSUM_V ||
                  (size_t)fp->n_pre * HSUM_V < (size_t)fp->hs.T * fp->hs.stride)
               : fp->n_pre / fp->pre_rows != fp->sp.ks)
    return false;
  int end = 0;
  for (int i = 0; i < 3; ++i) {
    if (i < n) {
      const aos_gemv_params &p = fp->gp[i];
      if (p.waves != waves || p.T != T || !rbg_ok(p) || p.ks < 1 || p.gen != fp->gen) return false;
      if (lines ? (p.pre_lines != fp->lines || p.n_pre_lines != fp->n_lines || p.plan_line != plan_line ||
                   p.sync != nullptr)
                : (p.sync != fp->sync || p.flags != fp->flags + (size_t)end * 32 ||
                   p.sync_target != (uint32_t)fp->n_pre || p.pre_lines != nullptr))
        return false;
      end += p.nrbg * p.ks;
    }
    if (fp->wg_end[i] != end) return false;
  }
  return fp->n_cons == (uint32_t)end;
}

extern "C" int aos_launch_decode_mlp(const aos_decode_mlp_params *mp, const aos_launch_ctx *st) {
  const aos_gemv_fused_params &gu = mp->gu, &dn = mp->dn;
  if (!aos_fused_params_ok(&gu, 1) || !aos_fused_params_ok(&dn, 0)) return (int)hipErrorInvalidValue;
  const aos_gemv_params &g1 = gu.gp[0], &g2 = dn.gp[0];
  const int T = g1.T;
  /* 1-2 tokens, 4-wave workgroups in every role, one generation, the h shrink formed by gate/up
   * and summed by dn's producers, h handed over through hdone and hflags */
  if (T > 2 || g2.T != T || g2.waves != 4 || dn.n != 1 || gu.hsum || !dn.hsum || !dn.hs.coherent) return (int)hipErrorInvalidValue;
  if (dn.gen != gu.gen || g1.x == nullptr || g2.x != g1.y || !g1.hpart || g1.hpart != dn.hs.hpart ||
      dn.hs.RB != g1.w0.RB || g1.hstride != dn.hs.stride || !g1.hdone || !mp->hflags || g1.hflags != mp->hflags ||
      g1.n_hflags != (uint32_t)dn.n_pre + dn.n_cons || g2.w0.in != g1.w0.out)
    return (int)hipErrorInvalidValue;
  if (T <= 1) return launch_mlp_nv<1>(mp, st);
  return launch_mlp_nv<2>(mp, st);
}

AOS_DEFINE_SPIN_SETTER(aos_spin_setter_gemv)
