/*
 * aoship_lora.hip — LoRA shrink S = coef * (X . A^T) on the matrix cores.
 *
 * The MLX forward computes each adapter's delta as ((x @ A^T) @ B^T) * (scale * blend)
 * (mlx_cpp_wrapper_real.cpp:3394-3419). Here the first product ("shrink", rank r outputs per
 * adapter) is computed once per call for every adapter in the union of the tokens' rings, with
 * each token's coefficient folded in; the second product ("expand") runs inside the base-layer
 * kernels as extra K steps of the same accumulators.
 *
 * Grid: (column tiles of 32 (adapter, rank-row) pairs, module, K chunks). A workgroup of 4 waves
 * covers 4 * SG groups of K; every wave issues all of its operand loads (x fragments and A rows,
 * 16 bytes per lane per step) before its v_mfma_f32_32x32x16_bf16 chain. Waves are summed in LDS
 * in wave order and the K chunks by the last workgroup to finish the tile, in chunk order, so the
 * result is deterministic.
 */
#include "aoship_device.h"
#include "aoship_internal.h"
#include <hip/hip_ext.h>
#include "aoship_union.h"

namespace {

constexpr int SG = AOS_SHRINK_GROUPS_PER_WAVE;

__global__ void __launch_bounds__(256) aos_shrink_kernel(aos_shrink_params p) {
  __shared__ uint32_t bits[AOS_UNION_WORDS];
  __shared__ uint16_t list[256];
  __shared__ int cnt;
  __shared__ float red[4][16][64];
  __shared__ uint32_t last_flag;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ct = blockIdx.x, mod = blockIdx.y, kchunk = blockIdx.z;
  const aos_lora_tab &tab = p.tab[mod];
  const int rpad = tab.rpad;
  if (rpad == 0) return;
  const int U = aos_build_union(p.rings, 0, p.T, tab, bits, list, &cnt);
  if (ct * 32 >= U * rpad) return; /* uniform over the whole tile's K chunks */

  const int G = p.in >> 6;
  const int ga = (kchunk * 4 + wave) * SG;
  const int ng = ga >= G ? 0 : (G - ga < SG ? G - ga : SG);
  const int i = lane & 31, c = lane >> 5;
  const int col = ct * 32 + i;
  const int u = col / rpad, j = col - u * rpad;
  const uint16_t *arow = (u < U) ? tab.A[list[u]] + (size_t)j * p.in : nullptr;
  const uint16_t *xrow = (i < p.T) ? p.x + (size_t)i * p.in : nullptr;

  u32x4 xa[SG * 4], ab[SG * 4];
#pragma unroll
  for (int s = 0; s < SG * 4; ++s) {
    xa[s] = u32x4{0u, 0u, 0u, 0u};
    ab[s] = u32x4{0u, 0u, 0u, 0u};
    if (s < ng * 4) {
      const int k0 = 64 * ga + 16 * s + 8 * c;
      if (xrow) xa[s] = *(const u32x4 *)(xrow + k0);
      if (arow) ab[s] = *(const u32x4 *)(arow + k0);
    }
  }
  f32x16 acc = {};
#pragma unroll
  for (int s = 0; s < SG * 4; ++s)
    if (s < ng * 4) acc = aos_mfma32(xa[s], ab[s], acc);

#pragma unroll
  for (int v = 0; v < 16; ++v) red[wave][v][lane] = acc[v];
  __syncthreads();
  /* wave w owns registers 4w..4w+3 from here on */
  float tot[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int v = 4 * wave + r;
    tot[r] = ((red[0][v][lane] + red[1][v][lane]) + red[2][v][lane]) + red[3][v][lane];
  }

  if (p.kc > 1) {
    const int slot = mod * p.n_col_tiles + ct;
    float *part = p.part + ((size_t)slot * p.kc + kchunk) * (16 * 64);
#pragma unroll
    for (int r = 0; r < 4; ++r) aos_publish(part + (4 * wave + r) * 64 + lane, tot[r]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      uint32_t old = aos_arrive(&p.counters[slot]);
      last_flag = (old == (uint32_t)p.kc - 1u) ? 1u : 0u;
      if (last_flag) aos_reset(&p.counters[slot]);
    }
    __syncthreads();
    if (!last_flag) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) tot[r] = 0.0f;
    for (int kk = 0; kk < p.kc; ++kk) {
      const float *pp = p.part + ((size_t)slot * p.kc + kk) * (16 * 64);
#pragma unroll
      for (int r = 0; r < 4; ++r) tot[r] += aos_collect(pp + (4 * wave + r) * 64 + lane);
    }
  }

  /* S[t][col] = coef(t, adapter) * total (bfloat16) */
  if (u < U) {
    const int stride = p.umax * rpad;
    const int a = list[u];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = aos_acc_m(4 * wave + r, lane);
      if (m < p.T) {
        const float cf = aos_coef(p.rings[m], a, tab);
        p.S[mod][(size_t)m * stride + col] = aos_f32_to_bf16(cf * tot[r]);
      }
    }
  }
}

}  // namespace

extern "C" int aos_launch_shrink(const aos_shrink_params *p, const aos_launch_ctx *ctx) {
  dim3 grid(p->n_col_tiles, p->nmod, p->kc);
  AOS_LAUNCH(ctx, aos_shrink_kernel, grid, dim3(256), 0, *p);
  return (int)hipGetLastError();
}
