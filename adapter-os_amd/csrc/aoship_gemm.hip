/*
 * aoship_gemm.hip — prefill path (T > 32 tokens): adapter plan, LoRA shrink and the int4 GEMM
 * with fused LoRA expand (+ SwiGLU), all on the matrix cores.
 *
 * Computes the MLX forward's linear(x, W) + apply_lora(x) (mlx_cpp_wrapper_real.cpp:3372-3419)
 * for a block of tokens, and in SwiGLU mode h = (g * sigmoid(g)) * u (:3509-3522); the ring ->
 * (adapter, scale * q / 32767) mapping is prepare_lora_for_ring
 * (crates/adapteros-lora-mlx-ffi/src/backend.rs:398-428).
 *
 * Launch sequence of one call:
 *   1. pplan         (one per M tile) union of the adapters the tokens use (ascending), the
 *                                     tile's per-token coefficients over the union and the
 *                                     bitmask of union slots any of its 128 tokens uses;
 *   3. pshrink       S = x . A^T over the union's rank rows, float32, K split into ks partial
 *                                     sums; pfinish adds them in split order and applies each
 *                                     token's coefficient: SA = bf16(coef * S);
 *   4. gemm          int4 GEMM, the expand over the tile's union slots added to the same
 *                                     accumulators after the K loop.
 *
 * GEMM tiling for gfx950 (v_mfma_f32_32x32x16_bf16, 64-wide waves):
 *   - a workgroup of 4 waves covers 32 * MT tokens; each wave owns NR 32-row blocks of weights
 *     (SwiGLU: the same rows of gate and up) for all the tokens of the tile;
 *   - weights come straight from the q4-tile layout (one 16-byte load per lane per group and row
 *     block) into registers through a ring D groups deep and are dequantised there to bfloat16
 *     B fragments (w = s * q + b in float32, hardware round-to-nearest-even packing), so each
 *     weight is read and dequantised once per workgroup;
 *   - the token tile of each group (32 * MT rows x 64 bf16) is staged in LDS, double buffered,
 *     with an XOR swizzle of its 16-byte chunks so that fragment reads are free of bank
 *     conflicts; the four waves share it;
 *   - workgroups are ordered so that the token tiles of one weight block run back to back on one
 *     XCD, whose L2 then serves the weight re-reads.
 */
#include "aoship_device.h"
#include "aoship_internal.h"
#include <hip/hip_ext.h>

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* Two floats -> packed bfloat16 pair (round to nearest even, v_cvt_pk_bf16_f32). */
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  bf16x2_t v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

/* Byte k of w as a float (one v_cvt_f32_ubyte<k>). */
template <int k>
__device__ __forceinline__ float ubyte(uint32_t w) {
  return (float)((w >> (8 * k)) & 0xffu);
}

/* Dequantise one nibble-shuffled word (nibbles stored as e0 e2 e4 e6 e1 e3 e5 e7) into the
 * bf16 pairs (e0,e1) (e2,e3) (e4,e5) (e6,e7) of w = s * q + b. */
__device__ __forceinline__ u32x4 dequant_word(uint32_t w, float s, float b) {
  const uint32_t lo = w & 0x0F0F0F0Fu;        /* bytes: e0 e4 e1 e5 */
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu; /* bytes: e2 e6 e3 e7 */
  u32x4 r;
  r.x = pk_bf16(fmaf(s, ubyte<0>(lo), b), fmaf(s, ubyte<2>(lo), b));
  r.y = pk_bf16(fmaf(s, ubyte<0>(hi), b), fmaf(s, ubyte<2>(hi), b));
  r.z = pk_bf16(fmaf(s, ubyte<1>(lo), b), fmaf(s, ubyte<3>(lo), b));
  r.w = pk_bf16(fmaf(s, ubyte<1>(hi), b), fmaf(s, ubyte<3>(hi), b));
  return r;
}

/* LDS token tile: rows of 64 bf16 (eight 16-byte chunks); chunk c of row r sits in slot
 * c ^ (r & 7). */
__device__ __forceinline__ int tile_off(int r, int chunk) { return r * 128 + ((chunk ^ (r & 7)) << 4); }

/* Stage the [BM x 64] bf16 slice of group g of the token rows m0... Rows past the last token
 * repeat it: they only feed accumulator rows that are never stored. */
template <int BM>
struct Stager {
  static constexpr int CH = BM * 8 / 256; /* 16-byte chunks per thread */
  u32x4 v[CH];
  __device__ __forceinline__ void load(const uint16_t *x, int in, int T, int m0, int g, int tid) {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int idx = tid + k * 256;
      const int r = idx >> 3, ch = idx & 7;
      const int tok = m0 + r < T ? m0 + r : T - 1;
      v[k] = *(const u32x4 *)(x + (size_t)tok * in + (size_t)g * 64 + ch * 8);
    }
  }
  __device__ __forceinline__ void store(unsigned char *buf, int tid) const {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int idx = tid + k * 256;
      const int r = idx >> 3, ch = idx & 7;
      *(u32x4 *)(buf + tile_off(r, ch)) = v[k];
    }
  }
};

/* ------------------------------------------------------------------------------------------ */
/* plan                                                                                       */
/* ------------------------------------------------------------------------------------------ */

/* One workgroup per M tile of AOS_GEMM_BM tokens. Every workgroup scans all the rings and
 * derives the same union (workgroup 0 stores it); each then writes the coefficient rows of its
 * own tokens and its tile's slot mask. */
__global__ void __launch_bounds__(256) aos_pplan_kernel(aos_pplan_params p) {
  __shared__ uint32_t bits[AOS_MAX_ADAPTERS / 32];
  __shared__ uint32_t mask[AOS_MAX_ADAPTERS / 32];
  __shared__ int base[AOS_MAX_ADAPTERS / 32 + 1];
  const int tid = threadIdx.x;
  const int words = (p.n + 31) >> 5;
  for (int w = tid; w < words; w += 256) bits[w] = 0u;
  for (int w = tid; w < p.mwords; w += 256) mask[w] = 0u;
  __syncthreads();
  /* union over every token's active slots: one ring per thread and step, read in 8-byte words */
  for (int t = tid; t < p.T; t += 256) {
    const u32x2 *rw = (const u32x2 *)(p.rings + t);
    const u32x2 w0 = rw[0], w1 = rw[1], w2 = rw[2], w3 = rw[3], w4 = rw[4];
    const uint32_t k = w0.x;
    const uint32_t idx[4] = {w1.x, w1.y, w2.x, w2.y}; /* adapter_indices, two per word */
    const uint32_t gq[4] = {w3.x, w3.y, w4.x, w4.y};  /* gates_q15, two per word */
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int a = (int)((idx[s >> 1] >> (16 * (s & 1))) & 0xffffu);
      const int q = (int)(int16_t)((gq[s >> 1] >> (16 * (s & 1))) & 0xffffu);
      if (s < (int)k && q > 0 && a < p.n && p.bound[a] && !((bits[a >> 5] >> (a & 31)) & 1u))
        atomicOr(&bits[a >> 5], 1u << (a & 31));
    }
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int w = 0; w < words; ++w) {
      base[w] = acc;
      acc += __builtin_popcount(bits[w]);
    }
    base[words] = acc;
    if (blockIdx.x == 0) p.plan->U = acc;
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int a = tid; a < p.n; a += 256) {
      const uint32_t m = bits[a >> 5];
      if ((m >> (a & 31)) & 1u) {
        const int u = base[a >> 5] + __builtin_popcount(m & ((1u << (a & 31)) - 1u));
        p.plan->list[u] = (uint16_t)a;
        p.plan->slot[a] = (int16_t)u;
      } else {
        p.plan->slot[a] = -1;
      }
    }
  }
  /* this tile's coefficient rows: zero, then each token's slots in ring order by one thread */
  const int t0 = blockIdx.x * AOS_GEMM_BM;
  const int tn = (p.T - t0) < AOS_GEMM_BM ? (p.T - t0) : AOS_GEMM_BM;
  const int cs = p.cstride;
  for (int e = tid; e < tn * cs; e += 256) p.coef[(size_t)t0 * cs + e] = 0.0f;
  __syncthreads();
  if (tid < tn) {
    const aoship_ring_t &r = p.rings[t0 + tid];
    float *row = p.coef + (size_t)(t0 + tid) * cs;
    for (int s = 0; s < 8; ++s) {
      const int a = r.adapter_indices[s];
      const int q = r.gates_q15[s];
      if (s < (int)r.top_k && q > 0 && a < p.n && p.bound[a]) {
        const uint32_t m = bits[a >> 5];
        const int u = base[a >> 5] + __builtin_popcount(m & ((1u << (a & 31)) - 1u));
        row[u] += p.scale[a] * ((float)q / 32767.0f);
        if (!((mask[u >> 5] >> (u & 31)) & 1u)) atomicOr(&mask[u >> 5], 1u << (u & 31));
      }
    }
  }
  __syncthreads();
  for (int w = tid; w < p.mwords; w += 256) p.tile_mask[(size_t)blockIdx.x * p.mwords + w] = mask[w];
}

/* ------------------------------------------------------------------------------------------ */
/* shrink over the union, finished with the coefficients (bf16 SA)                            */
/* ------------------------------------------------------------------------------------------ */

template <int MT>
__global__ void __launch_bounds__(256) aos_pshrink_kernel(aos_pshrink_params p) {
  constexpr int BM = 32 * MT;
  constexpr int TILE = BM * 128;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, c = lane >> 5;
  const int mi = blockIdx.z / p.ks, kz = blockIdx.z - mi * p.ks;
  const aos_lora_tab &tab = p.tab[mi];
  const int rpad = tab.rpad;
  const int U = p.plan->U < p.umax ? p.plan->U : p.umax;
  const int col0 = blockIdx.y * 128;
  /* uniform over the workgroup and over the K splits of this tile: all of them leave together */
  if (rpad == 0 || col0 >= U * rpad) return;
  const int m0 = blockIdx.x * BM;
  const int G = p.in / 64;
  const int g_lo = kz * p.gpk;
  const int g_hi = (g_lo + p.gpk) < G ? (g_lo + p.gpk) : G;

  /* this lane's A row: column col = col0 + 32 wave + i of module mi */
  const int col = col0 + 32 * wave + i;
  const int u = col / rpad, j = col - u * rpad;
  const uint16_t *arow = p.zero_row;
  size_t kstep = 0;
  if (u < U) {
    const uint16_t *A = tab.A[p.plan->list[u]];
    if (A) {
      arow = A + (size_t)j * p.in;
      kstep = 1;
    }
  }

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x16{};

  Stager<BM> st;
  u32x4 an[4];
  st.load(p.x, p.in, p.T, m0, g_lo, tid);
  st.store(smem, tid);
#pragma unroll
  for (int s = 0; s < 4; ++s) an[s] = *(const u32x4 *)(arow + kstep * ((size_t)g_lo * 64 + 16 * s + 8 * c));
  lds_barrier();
  for (int g = g_lo; g < g_hi; ++g) {
    const unsigned char *tb = smem + ((g - g_lo) & 1) * TILE;
    u32x4 a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = an[s];
    const int gn = g + 1 < g_hi ? g + 1 : g_hi - 1;
    st.load(p.x, p.in, p.T, m0, gn, tid);
#pragma unroll
    for (int s = 0; s < 4; ++s) an[s] = *(const u32x4 *)(arow + kstep * ((size_t)gn * 64 + 16 * s + 8 * c));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = mt * 32 + i;
      u32x4 xv[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) xv[s] = *(const u32x4 *)(tb + tile_off(r, 2 * s + c)); /* K 16 s + 8 c */
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[mt] = aos_mfma32(xv[s], a[s], acc[mt]);
    }
    st.store(smem + (((g - g_lo) & 1) ^ 1) * TILE, tid);
    lds_barrier();
  }

  const int scol = p.s_off[mi] + col;
  const bool col_live = col < U * rpad;
  const int uc = col_live ? u : 0;
  if (p.ks == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int tok = m0 + mt * 32 + aos_acc_m(v, lane);
        if (col_live && tok < p.T)
          p.SA[(size_t)tok * p.s_stride + scol] =
              aos_f32_to_bf16(p.coef[(size_t)tok * p.cstride + uc] * acc[mt][v]);
      }
    return;
  }
  /* K split: plain float32 partial sums, added in split order by aos_pfinish_kernel */
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int tok = m0 + mt * 32 + aos_acc_m(v, lane);
      if (col_live && tok < p.T) p.part[((size_t)kz * p.T + tok) * p.s_stride + scol] = acc[mt][v];
    }
}

/* SA[t][col] = bf16(coef[t][u(col)] * sum_kz part[kz][t][col]), four columns per thread. */
__global__ void __launch_bounds__(256) aos_pfinish_kernel(aos_pshrink_params p) {
  const int q4 = p.s_stride / 4; /* s_stride is a multiple of 16 */
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (size_t)p.T * q4) return;
  const int t = (int)(e / q4);
  const int col = (int)(e - (size_t)t * q4) * 4;
  int mi = 0;
  for (int k = 1; k < p.nmod; ++k)
    if (col >= p.s_off[k]) mi = k;
  const int rpad = p.tab[mi].rpad;
  if (rpad == 0) return;
  const int u = (col - p.s_off[mi]) / rpad;
  const int U = p.plan->U < p.umax ? p.plan->U : p.umax;
  if (u >= U) return;
  const size_t kstride = (size_t)p.T * p.s_stride;
  const float *pp = p.part + (size_t)t * p.s_stride + col;
  float4 sum = *(const float4 *)pp;
  for (int k = 1; k < p.ks; ++k) {
    const float4 v = *(const float4 *)(pp + k * kstride);
    sum.x += v.x;
    sum.y += v.y;
    sum.z += v.z;
    sum.w += v.w;
  }
  const float cf = p.coef[(size_t)t * p.cstride + u];
  u32x2 o;
  o.x = (uint32_t)aos_f32_to_bf16(cf * sum.x) | ((uint32_t)aos_f32_to_bf16(cf * sum.y) << 16);
  o.y = (uint32_t)aos_f32_to_bf16(cf * sum.z) | ((uint32_t)aos_f32_to_bf16(cf * sum.w) << 16);
  *(u32x2 *)(p.SA + (size_t)t * p.s_stride + col) = o;
}

/* ------------------------------------------------------------------------------------------ */
/* int4 GEMM + LoRA expand (+ SwiGLU)                                                          */
/* ------------------------------------------------------------------------------------------ */

/* First union slot >= from whose bit is set in the tile mask and whose adapter has module B;
 * -1 if none. Uniform. */
__device__ __forceinline__ int next_slot(const aos_gemm_params &p, const aos_lora_tab &tab, const uint32_t *mask,
                                         int from) {
  for (int w = from >> 5; w < p.mwords; ++w) {
    uint32_t bits = mask[w];
    if (w == (from >> 5)) bits &= ~0u << (from & 31);
    while (bits) {
      const int u = w * 32 + __builtin_ctz(bits);
      bits &= bits - 1u;
      if (tab.B[p.plan->list[u]] != nullptr) return u;
    }
  }
  return -1;
}

/* Expand of one module: for each (slot u, 16 rank rows j0) step the A operand is SA[t][s_off +
 * u * rpad + j0 + 8c ..] (coefficient already applied) and the B operand the adapter's B rows of
 * this wave's row block(s). Fragments of the next step are loaded before the current step's
 * matrix-core work. Rows of dead row blocks and tokens past T read clamped (valid) addresses;
 * their accumulators are never stored. */
template <int MT, int NX>
__device__ __forceinline__ void expand_module(const aos_gemm_params &p, const aos_lora_tab &tab, int s_off,
                                              const int (&row)[2], int m0, int mbi,
                                              int lane, f32x16 (&acc0)[MT], f32x16 (&acc1)[MT]) {
  const int rpad = tab.rpad;
  if (rpad == 0) return;
  const int i = lane & 31, c = lane >> 5;
  const uint32_t *mask = p.tile_mask + (size_t)mbi * p.mwords;
  int u = next_slot(p, tab, mask, 0);
  if (u < 0) return;
  int j0 = 0;
  const uint16_t *sa_row[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int t = m0 + mt * 32 + i;
    sa_row[mt] = p.SA + (size_t)(t < p.T ? t : p.T - 1) * p.sa_stride + s_off + 8 * c;
  }
  u32x4 bv[NX], av[MT];
  auto load = [&](int uu, int jj, u32x4 (&b)[NX], u32x4 (&a)[MT]) {
    const uint16_t *B = tab.B[p.plan->list[uu]];
#pragma unroll
    for (int x = 0; x < NX; ++x) b[x] = *(const u32x4 *)(B + (size_t)row[x] * rpad + jj + 8 * c);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) a[mt] = *(const u32x4 *)(sa_row[mt] + (size_t)uu * rpad + jj);
  };
  load(u, j0, bv, av);
  while (true) {
    int un = u, jn = j0 + 16;
    if (jn == rpad) {
      jn = 0;
      un = next_slot(p, tab, mask, u + 1);
    }
    u32x4 bn[NX], an[MT];
    if (un >= 0) load(un, jn, bn, an);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc0[mt] = aos_mfma32(av[mt], bv[0], acc0[mt]);
      if (NX == 2) acc1[mt] = aos_mfma32(av[mt], bv[NX - 1], acc1[mt]);
    }
    if (un < 0) break;
    u = un;
    j0 = jn;
#pragma unroll
    for (int x = 0; x < NX; ++x) bv[x] = bn[x];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) av[mt] = an[mt];
  }
}

/* SW: SwiGLU (gate and up rows, NR = 2); NR: row blocks per wave; MT: 32-token sub-tiles;
 * D: weight ring depth (divides the group count); DB: token tile loads two groups ahead (two
 * register stages); APF: next sub-tile's LDS fragments loaded before the current MFMAs. Two
 * workgroups per CU (two waves per SIMD) let one wave's dequantisation overlap the other's
 * matrix-core work. */
template <bool SW, int NR, int MT, int D, bool DBT, bool APF>
__global__ void __launch_bounds__(256, 2) aos_gemm_kernel(aos_gemm_params p) {
  static_assert(!SW || NR == 2, "SwiGLU pairs gate and up rows");
  constexpr int BM = 32 * MT;
  constexpr int TILE = BM * 128;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, c = lane >> 5;

  /* XCD-aware order: workgroup b runs on XCD b % 8; tiles are numbered with the token tile
   * fastest and dealt out so that each XCD gets a contiguous range of them. */
  const int nt = p.mb * p.nb;
  const int b = blockIdx.x;
  int tile = b;
  if (nt % 8 == 0) tile = (b & 7) * (nt / 8) + (b >> 3);
  const int mbi = tile % p.mb, nbk = tile / p.mb;
  const int m0 = mbi * BM;
  const int G = p.w0.G, in = p.w0.in, RB = p.w0.RB;

  /* weight row blocks of this wave */
  const int rb0 = SW ? nbk * 4 + wave : nbk * 4 * NR + NR * wave;
  const int rb1 = SW ? rb0 : rb0 + 1;
  const bool live0 = rb0 < RB;
  const bool live1 = SW ? live0 : (NR == 2 && rb1 < RB);
  const int r0 = live0 ? rb0 : RB - 1;
  const int r1 = SW ? r0 : (live1 ? rb1 : r0);
  const aos_q4_dev &W0 = p.w0;
  const aos_q4_dev &W1 = SW ? p.w1 : p.w0;
  const u32x4 *q0 = (const u32x4 *)W0.qt + (size_t)r0 * G * 64 + lane;
  const u32x4 *q1 = (const u32x4 *)W1.qt + (size_t)r1 * G * 64 + lane;
  const uint32_t *s0p = W0.sb + (size_t)r0 * G * 32 + i;
  const uint32_t *s1p = W1.sb + (size_t)r1 * G * 32 + i;

  f32x16 acc0[MT], acc1[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc0[mt] = f32x16{};
    acc1[mt] = f32x16{};
  }

  /* prologue: weight ring D groups deep (D divides G), first token tile */
  u32x4 wq0[D], wq1[D];
  uint32_t ws0[D], ws1[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    wq0[d] = q0[(size_t)d * 64];
    ws0[d] = s0p[(size_t)d * 32];
    if (NR == 2) {
      wq1[d] = q1[(size_t)d * 64];
      ws1[d] = s1p[(size_t)d * 32];
    }
  }
  /* Token tiles: LDS holds groups g and g + 1 (double buffer); registers hold the loads in
   * flight. With D even, two register stages let the loads run two groups ahead of their LDS
   * store. */
  constexpr bool DB = DBT && (D % 2) == 0;
  Stager<BM> st0, st1;
  st0.load(p.x, in, p.T, m0, 0, tid);
  st0.store(smem, tid);
  if (DB) st1.load(p.x, in, p.T, m0, G > 1 ? 1 : 0, tid);
  lds_barrier();

  /* one K group: ld receives group g + 2 (g + 1 without DB), sto holds group g + 1 */
  auto group = [&](const int g, const int d, Stager<BM> &ld, Stager<BM> &sto) {
    const unsigned char *tb = smem + (g & 1) * TILE;
    /* token fragments of the first sub-tile: their LDS latency overlaps the dequantisation */
    u32x4 a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = *(const u32x4 *)(tb + tile_off(i, 4 * c + s));
    {
      const int ahead = DB ? 2 : 1;
      const int gx = g + ahead < G ? g + ahead : G - 1;
      ld.load(p.x, in, p.T, m0, gx, tid);
    }
    /* dequantise this group's row blocks into B fragments */
    u32x4 f0[4], f1[4];
    {
      const float sc = aos_f16_to_f32(ws0[d] & 0xffffu), bi = aos_f16_to_f32(ws0[d] >> 16);
#pragma unroll
      for (int s = 0; s < 4; ++s) f0[s] = dequant_word(wq0[d][s], sc, bi);
    }
    if (NR == 2) {
      const float sc = aos_f16_to_f32(ws1[d] & 0xffffu), bi = aos_f16_to_f32(ws1[d] >> 16);
#pragma unroll
      for (int s = 0; s < 4; ++s) f1[s] = dequant_word(wq1[d][s], sc, bi);
    }
    /* refill the ring slot */
    {
      const int gn = g + D < G ? g + D : G - 1;
      wq0[d] = q0[(size_t)gn * 64];
      ws0[d] = s0p[(size_t)gn * 32];
      if (NR == 2) {
        wq1[d] = q1[(size_t)gn * 64];
        ws1[d] = s1p[(size_t)gn * 32];
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      u32x4 an[4];
      if (APF && mt + 1 < MT) {
#pragma unroll
        for (int s = 0; s < 4; ++s) an[s] = *(const u32x4 *)(tb + tile_off((mt + 1) * 32 + i, 4 * c + s));
      }
      if (!APF && mt > 0) {
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = *(const u32x4 *)(tb + tile_off(mt * 32 + i, 4 * c + s));
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        /* word s of lane (i, c) covers K elements 32 c + 8 s .. +7: chunk 4 c + s */
        acc0[mt] = aos_mfma32(a[s], f0[s], acc0[mt]);
        if (NR == 2) acc1[mt] = aos_mfma32(a[s], f1[s], acc1[mt]);
      }
      if (APF && mt + 1 < MT) {
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = an[s];
      }
    }
    sto.store(smem + ((g & 1) ^ 1) * TILE, tid);
    lds_barrier();
  };

  for (int g0 = 0; g0 < G; g0 += D) {
    if (DB) {
#pragma unroll
      for (int d = 0; d < D; d += 2) {
        group(g0 + d, d, st0, st1);
        group(g0 + d + 1, d + 1, st1, st0);
      }
    } else {
#pragma unroll
      for (int d = 0; d < D; ++d) group(g0 + d, d, st0, st0);
    }
  }

  /* LoRA expand over the tile's union slots */
  const int row0 = r0 * 32 + i, row1 = r1 * 32 + i;
  if (SW) {
    const int rows[2] = {row0, row0};
    expand_module<MT, 1>(p, p.tab0, p.s_off0, rows, m0, mbi, lane, acc0, acc0);
    expand_module<MT, 1>(p, p.tab1, p.s_off1, rows, m0, mbi, lane, acc1, acc1);
  } else {
    const int rows[2] = {row0, row1};
    expand_module<MT, NR>(p, p.tab0, p.s_off0, rows, m0, mbi, lane, acc0, acc1);
  }

  /* epilogue */
  const int out = p.w0.out;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int tok = m0 + mt * 32 + aos_acc_m(v, lane);
      if (tok >= p.T) continue;
      if (SW) {
        if (!live0) continue;
        const float gt = acc0[mt][v], up = acc1[mt][v];
        const float sg = 1.0f / (1.0f + expf(-gt));
        p.y[(size_t)tok * out + row0] = aos_f32_to_bf16((gt * sg) * up);
      } else {
        if (live0) p.y[(size_t)tok * out + row0] = aos_f32_to_bf16(acc0[mt][v]);
        if (NR == 2 && live1) p.y[(size_t)tok * out + row1] = aos_f32_to_bf16(acc1[mt][v]);
      }
    }
  }
}

}  // namespace

extern "C" int aos_launch_pplan(const aos_pplan_params *p, const aos_launch_ctx *ctx) {
  const int mtiles = (p->T + AOS_GEMM_BM - 1) / AOS_GEMM_BM;
  AOS_LAUNCH(ctx, aos_pplan_kernel, dim3(mtiles), dim3(256), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_pshrink(const aos_pshrink_params *p, const aos_launch_ctx *ctx) {
  constexpr int MT = AOS_GEMM_BM / 32;
  dim3 grid(p->mtiles, p->cblocks, p->ks * p->nmod);
  AOS_LAUNCH(ctx, aos_pshrink_kernel<MT>, grid, dim3(256), 2 * AOS_GEMM_BM * 128, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_pfinish(const aos_pshrink_params *p, const aos_launch_ctx *ctx) {
  const size_t n = (size_t)p->T * (p->s_stride / 4);
  AOS_LAUNCH(ctx, aos_pfinish_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, *p);
  return (int)hipGetLastError();
}

/* Measured on the 7B-shaped layer at 2048 tokens: the SwiGLU kernel is fastest with a shallow
 * ring and single staging (fewer registers), the single-matrix kernel with the deep pipeline. */
template <bool SW, int NR>
static void launch_gemm_d(const aos_gemm_params *p, const aos_launch_ctx *ctx) {
  constexpr int MT = AOS_GEMM_BM / 32;
  constexpr int D4 = SW ? 2 : 4;
  constexpr bool DBT = !SW, APF = !SW;
  const size_t lds = 2 * AOS_GEMM_BM * 128;
  const dim3 grid(p->mb * p->nb);
  const int G = p->w0.G;
  if (G % D4 == 0)
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, NR, MT, D4, DBT, APF>), grid, dim3(256), lds, *p);
  else if (G % 2 == 0)
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, NR, MT, 2, DBT, APF>), grid, dim3(256), lds, *p);
  else
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, NR, MT, 1, DBT, APF>), grid, dim3(256), lds, *p);
}

extern "C" int aos_launch_gemm(const aos_gemm_params *p, int swiglu, const aos_launch_ctx *ctx) {
  if (swiglu)
    launch_gemm_d<true, 2>(p, ctx);
  else
    launch_gemm_d<false, 1>(p, ctx);
  return (int)hipGetLastError();
}
