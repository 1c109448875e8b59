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

/* Byte k of w as a float: one v_cvt_f32_ubyte<k> (left to itself the compiler extracts each
 * nibble with v_bfe_u32 and converts byte 0, twice the instructions). */
template <int k>
__device__ __forceinline__ float ubyte(uint32_t w) {
  float r;
  if (k == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
  else if (k == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
  else if (k == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
  return r;
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
 * c ^ ((r >> 1) & 7). A row is 128 bytes, half of the 64 four-byte banks: even and odd rows use
 * the two halves, and the slot rotation spreads 8 rows of equal parity over the 8 slots, so 16
 * consecutive rows read one chunk each without a bank conflict. */
__device__ __forceinline__ int tile_off(int r, int chunk) { return r * 128 + ((chunk ^ ((r >> 1) & 7)) << 4); }

/* Stage the [BM x 64] bf16 slice of group g of the token rows m0... with NT threads. Rows past
 * the last token repeat it: they only feed accumulator rows that are never stored. */
template <int BM, int NT = 256>
struct Stager {
  static constexpr int CH = BM * 8 / NT; /* 16-byte chunks per thread */
  u32x4 v[CH];
  __device__ __forceinline__ void load(const uint16_t *x, int in, int T, int m0, int g, int tid) {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int idx = tid + k * NT;
      const int r = idx >> 3, ch = idx & 7;
      const int tok = m0 + r < T ? m0 + r : T - 1;
      v[k] = *(const u32x4 *)(x + (size_t)tok * in + (size_t)g * 64 + ch * 8);
    }
  }
  /* 64 columns of the rows of a tile-based buffer (rows bytes apart, rows >= nrows repeat the
   * last): byte columns cb .. cb + 127; chunks at or past lim bytes read as zeros (an offset
   * past the buffer's end). */
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t rs, int row_bytes, int nrows, int cb, int lim,
                                           int tid) {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int idx = tid + k * NT;
      const int r = idx >> 3, ch = idx & 7;
      const int rr = r < nrows ? r : nrows - 1;
      const int c = cb + ch * 16;
      const int off = c < lim ? rr * row_bytes + c : (int)0x80000000;
      v[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
  }
  __device__ __forceinline__ void store(unsigned char *buf, int tid) const {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int idx = tid + k * NT;
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
 * own tokens and its tile's slot mask. Every ring a thread scans, the bound flags and the
 * scales are loaded before anything waits, so the scan costs one memory round trip. */
constexpr int PLAN_NT = 1024;
constexpr int PLAN_RINGS = AOS_PREFILL_MAX_T / PLAN_NT; /* rings per thread */

__global__ void __launch_bounds__(PLAN_NT) aos_pplan_kernel(aos_pplan_params p) {
  __shared__ uint32_t bits[AOS_MAX_ADAPTERS / 32];
  __shared__ uint32_t mask[AOS_MAX_ADAPTERS / 32];
  __shared__ int base[AOS_MAX_ADAPTERS / 32 + 1];
  __shared__ uint8_t bound_s[AOS_MAX_ADAPTERS];
  __shared__ float scale_s[AOS_MAX_ADAPTERS];
  const int tid = threadIdx.x;
  const int words = (p.n + 31) >> 5;
  u32x2 rw[PLAN_RINGS][5];
#pragma unroll
  for (int j = 0; j < PLAN_RINGS; ++j) {
    const int t = tid + j * PLAN_NT;
    const u32x2 *r = (const u32x2 *)(p.rings + (t < p.T ? t : p.T - 1));
#pragma unroll
    for (int w = 0; w < 5; ++w) rw[j][w] = r[w];
  }
  for (int a = tid; a < p.n; a += PLAN_NT) {
    bound_s[a] = p.bound[a];
    scale_s[a] = p.scale[a];
  }
  for (int w = tid; w < words; w += PLAN_NT) bits[w] = 0u;
  for (int w = tid; w < p.mwords; w += PLAN_NT) mask[w] = 0u;
  __syncthreads();
  /* union over every token's active slots */
#pragma unroll
  for (int j = 0; j < PLAN_RINGS; ++j) {
    if (tid + j * PLAN_NT >= p.T) continue;
    const uint32_t k = rw[j][0].x;
    const uint32_t idx[4] = {rw[j][1].x, rw[j][1].y, rw[j][2].x, rw[j][2].y}; /* adapter_indices */
    const uint32_t gq[4] = {rw[j][3].x, rw[j][3].y, rw[j][4].x, rw[j][4].y};  /* gates_q15 */
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int a = (int)((idx[s >> 1] >> (16 * (s & 1))) & 0xffffu);
      const int q = (int)(int16_t)((gq[s >> 1] >> (16 * (s & 1))) & 0xffffu);
      if (s < (int)k && q > 0 && a < p.n && bound_s[a] && !((bits[a >> 5] >> (a & 31)) & 1u))
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
    for (int a = tid; a < p.n; a += PLAN_NT) {
      const uint32_t m = bits[a >> 5];
      if ((m >> (a & 31)) & 1u) {
        const int u = base[a >> 5] + __builtin_popcount(m & ((1u << (a & 31)) - 1u));
        p.plan->list[u] = (uint16_t)a;
        p.plan->slot[a] = (int16_t)u;
        if (u < p.cstride)
          for (int k = 0; k < p.nmod; ++k)
            p.bp[(size_t)k * p.cstride + u] = p.tab[k].rpad && a < p.tab[k].n ? p.tab[k].B[a] : nullptr;
      } else {
        p.plan->slot[a] = -1;
      }
    }
    for (int u = base[words] + tid; u < p.cstride; u += PLAN_NT)
      for (int k = 0; k < p.nmod; ++k) p.bp[(size_t)k * p.cstride + u] = nullptr;
  }
  /* this tile's coefficient rows: zero, then each token's slots by one thread, summed in ring
   * order per union slot (a slot named twice adds up in order) */
  const int t0 = blockIdx.x * AOS_GEMM_BM;
  const int tn = (p.T - t0) < AOS_GEMM_BM ? (p.T - t0) : AOS_GEMM_BM;
  const int cs = p.cstride;
  for (int e = tid; e < tn * cs; e += PLAN_NT) p.coef[(size_t)t0 * cs + e] = 0.0f;
  __syncthreads();
  if (tid < tn) {
    const aoship_ring_t &r = p.rings[t0 + tid];
    float *row = p.coef + (size_t)(t0 + tid) * cs;
    int us[8];
    float cv[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int a = r.adapter_indices[s];
      const int q = r.gates_q15[s];
      us[s] = -1;
      cv[s] = 0.0f;
      if (s < (int)r.top_k && q > 0 && a < p.n && bound_s[a]) {
        const uint32_t m = bits[a >> 5];
        const int u = base[a >> 5] + __builtin_popcount(m & ((1u << (a & 31)) - 1u));
        const float c = scale_s[a] * ((float)q / 32767.0f);
        int first = s;
#pragma unroll
        for (int s2 = 0; s2 < s; ++s2)
          if (first == s && us[s2] == u) first = s2;
        if (first == s) {
          us[s] = u;
          cv[s] = 0.0f + c;
        } else {
          cv[first] += c;
        }
        if (!((mask[u >> 5] >> (u & 31)) & 1u)) atomicOr(&mask[u >> 5], 1u << (u & 31));
      }
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (us[s] >= 0) row[us[s]] = cv[s];
  }
  __syncthreads();
  for (int w = tid; w < p.mwords; w += PLAN_NT) p.tile_mask[(size_t)blockIdx.x * p.mwords + w] = mask[w];
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

/* Expand K steps: the LoRA expand of a token tile runs as extra K steps of 64 columns after the
 * weight groups. The token operand is SA (coefficient-scaled shrink of the union slots), the
 * weight operand the union adapters' B rows (bf16). A step is listed as (module << 15) | j, j =
 * index of its 64 columns among the module's union columns u * rpad + r; a tile lists only the
 * steps that hold a slot one of its tokens uses.
 *
 * LDS after the token tiles: 16 bytes of counts, the slot mask words of the BM / 128 plan tiles
 * the token tile spans, LBP B pointers per module (two modules), then the step list. */
constexpr int LBP = 256;
constexpr int MASK_WORDS = AOS_MAX_ADAPTERS / 32;
__host__ __device__ constexpr int gemm_aux(int bm) { return 16 + 4 * MASK_WORDS * (bm / AOS_GEMM_BM) + 2 * LBP * 8; }

/* Workgroup b of a grid of mb token tiles x nb weight blocks -> (token tile, weight block).
 * Workgroup b runs on XCD b % 8. With a multiple of 8 token tiles each XCD takes its own token
 * tiles against every weight block (its L2 keeps those token rows while the weights stream);
 * otherwise each XCD takes a contiguous range of tiles (token tile fastest), so a weight block's
 * token tiles share its L2. */
__device__ __forceinline__ void gemm_tile_of(int b, int mb, int nb, int &mbi, int &nbk) {
  if (mb % 8 == 0) {
    const int mpx = mb / 8, k = b >> 3;
    mbi = (b & 7) * mpx + k % mpx;
    nbk = k / mpx;
  } else {
    const int nt = mb * nb;
    int tile = b;
    if (nt % 8 == 0) tile = (b & 7) * (nt / 8) + (b >> 3);
    mbi = tile % mb;
    nbk = tile / mb;
  }
}

/* The expand steps of one token tile (BM tokens, WV waves, NM modules). Each lane's B fragment
 * word w of a step holds union columns k = 64 j + koff[w] .. +7 of the lane's weight row:
 * B_{list[u]}[row][k - u * rpad .. +7] with u = k / rpad, zeros past the union or for an adapter
 * without the module (rpad is a multiple of 16, so 8 columns never straddle two slots). Words
 * w and w + 1 share a slot when NW / NP = 2 (koff 16-aligned for w even). */
template <int BM, int WV, int NM, int NW, int NP>
struct Expand {
  static constexpr int MR = BM / AOS_GEMM_BM; /* plan tiles per token tile */
  static constexpr int TILE = BM * 128;
  const aos_gemm_params &p;
  unsigned char *smem;
  int *ls_n;
  uint32_t *mw;
  const uint16_t **lbp;
  uint16_t *ls;
  int wave, lane, m0, mbi, row, Ue;
  bool lora, bp_lds;

  /* row: the lane's weight row (of every module) */
  __device__ Expand(const aos_gemm_params &p_, unsigned char *smem_, int ntile, int wave_, int lane_, int m0_,
                    int mbi_, int row_)
      : p(p_), smem(smem_), wave(wave_), lane(lane_), m0(m0_), mbi(mbi_), row(row_) {
    unsigned char *aux = smem + ntile * TILE;
    ls_n = (int *)aux;
    mw = (uint32_t *)(aux + 16);
    lbp = (const uint16_t **)(aux + 16 + 4 * MASK_WORDS * MR);
    ls = (uint16_t *)(aux + gemm_aux(BM));
    lora = (p.tab0.rpad | (NM == 2 ? p.tab1.rpad : 0)) != 0;
    Ue = p.plan->U < p.umax ? p.plan->U : p.umax;
    bp_lds = p.umax <= LBP;
  }

  /* At kernel start: the tile's slot mask words and (union bound <= LBP) the union's B pointers
   * go straight to LDS; their loads complete during the K loop. */
  __device__ void prefetch() {
    if (!lora) return;
    constexpr int NT = 64 * WV;
    const int ptiles = (p.T + AOS_GEMM_BM - 1) / AOS_GEMM_BM;
    const int pr0 = mbi * MR;
    const int npr = ptiles - pr0 < MR ? ptiles - pr0 : MR;
    const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.tile_mask + (size_t)pr0 * p.mwords), (short)0, npr * p.mwords * 4, 0x00020000);
#pragma unroll
    for (int r = 0; r < MR; ++r)
      for (int w0 = wave * 64; w0 < p.mwords; w0 += NT)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rm, (__attribute__((address_space(3))) void *)(mw + r * MASK_WORDS + w0), 4,
            r < npr ? (r * p.mwords + w0 + lane) * 4 : (int)0x80000000, 0, 0, 0);
    if (bp_lds) {
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const __amdgpu_buffer_rsrc_t rb =
            __builtin_amdgcn_make_buffer_rsrc((void *)(m ? p.bp1 : p.bp0), (short)0, p.umax * 8, 0x00020000);
        for (int d0 = wave * 64; d0 < 2 * p.umax; d0 += NT)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rb, (__attribute__((address_space(3))) void *)((uint32_t *)(lbp + m * LBP) + d0), 4,
              (d0 + lane) * 4, 0, 0, 0);
      }
    }
  }

  /* After the K loop (all waves): wave 0 lists the tile's steps, ascending module then column.
   * Returns the step count; n0 receives the count of module 0's steps. */
  __device__ int build(int &n0) {
    n0 = 0;
    if (!lora) return 0;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    if (wave == 0) {
      int n = 0;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if (m == 1 && lane == 0) ls_n[1] = n < p.lsteps_max ? n : p.lsteps_max;
        const int rpad = m ? p.tab1.rpad : p.tab0.rpad;
        const int nj = rpad ? (Ue * rpad + 63) >> 6 : 0;
        for (int j0 = 0; j0 < nj; j0 += 64) {
          const int j = j0 + lane;
          bool act = false;
          if (j < nj) {
            const int ulo = (64 * j) / rpad;
            int uhi = (64 * j + 63) / rpad;
            uhi = uhi < Ue - 1 ? uhi : Ue - 1;
            for (int u = ulo; u <= uhi; ++u) {
              uint32_t wd = 0;
#pragma unroll
              for (int r = 0; r < MR; ++r) wd |= mw[r * MASK_WORDS + (u >> 5)];
              act |= ((wd >> (u & 31)) & 1u) != 0;
            }
          }
          const uint64_t bal = __ballot(act);
          const int at = n + __popcll(bal & ((1ull << lane) - 1ull));
          if (act && at < p.lsteps_max) ls[at] = (uint16_t)((m << 15) | j);
          n += __popcll(bal);
        }
      }
      if (lane == 0) ls_n[0] = n < p.lsteps_max ? n : p.lsteps_max;
    }
    lds_barrier();
    const int nls = __builtin_amdgcn_readfirstlane(ls_n[0]);
    n0 = NM == 2 ? __builtin_amdgcn_readfirstlane(ls_n[1]) : nls;
    return nls;
  }

  __device__ void step_of(int l, int nls, int &m, int &j, int &rpad) const {
    l = l < nls ? l : nls - 1;
    const int d = __builtin_amdgcn_readfirstlane((int)ls[l > 0 ? l : 0]);
    m = d >> 15;
    j = d & 0x7fff;
    rpad = m ? p.tab1.rpad : p.tab0.rpad;
  }

  /* Runs the nls steps in chunks of LC steps within one module. A chunk's token tiles (the
   * steps' SA columns, through a buffer resource over the tile's rows; chunks past the union
   * read as zeros) go straight from memory to LDS regions 0 .. LC - 1, its B fragments to
   * registers; one wait per chunk, the next chunk's B pointers loading meanwhile. mma(m, n, bv)
   * adds the chunk's n steps of module m (token tile q at smem + q * TILE). */
  template <int LC, class Mma>
  __device__ void run(int nls, int n0, const int (&koff)[NW], Mma &&mma) {
    const int rows = p.T - m0 < BM ? p.T - m0 : BM;
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.SA + (size_t)m0 * p.sa_stride), (short)0, rows * p.sa_stride * 2, 0x00020000);
    auto load_ptrs = [&](int l, const uint16_t *(&pr)[NP]) {
      int m, j, rpad;
      step_of(l, nls, m, j, rpad);
      const uint16_t *const *bp = m ? p.bp1 : p.bp0;
#pragma unroll
      for (int h = 0; h < NP; ++h) {
        int u = (64 * j + koff[h * (NW / NP)]) / rpad;
        u = u < Ue ? u : Ue - 1;
        pr[h] = bp_lds ? lbp[m * LBP + u] : bp[u];
      }
    };
    auto load_frags = [&](int l, const uint16_t *const (&pr)[NP], u32x4 (&bv)[NW]) {
      int m, j, rpad;
      step_of(l, nls, m, j, rpad);
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const uint16_t *b = pr[w / (NW / NP)];
        const int k = 64 * j + koff[w];
        const int u = k / rpad;
        const uint16_t *src = (u < Ue && b) ? b + (size_t)row * rpad + (k - u * rpad) : p.zero;
        bv[w] = *(const u32x4 *)src;
      }
    };
    /* token tile of step l into LDS region q: BM / 8 blocks of 8 rows (1 KB), lane l of a block
     * writing bytes 16 l, i.e. row 8 b + l / 8, slot l % 8, which holds chunk slot ^ ((r >> 1) & 7) */
    auto dma_tile = [&](int q, int l) {
      int m, j, rpad;
      step_of(l, nls, m, j, rpad);
      const int off = m ? p.s_off1 : p.s_off0;
      const int cb = (off + 64 * j) * 2, lim = (off + Ue * rpad) * 2, rb = p.sa_stride * 2;
#pragma unroll
      for (int k = 0; k < BM / 8 / WV; ++k) {
        const int bk = k * WV + wave;
        const int r = bk * 8 + (lane >> 3);
        const int ch = (lane & 7) ^ ((r >> 1) & 7);
        const int rr = r < rows ? r : rows - 1;
        const int col = cb + ch * 16;
        const int vo = col < lim ? rr * rb + col : (int)0x80000000;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsa, (__attribute__((address_space(3))) void *)(smem + q * TILE + bk * 1024), 16, vo, 0, 0, 0);
      }
    };
    const uint16_t *pr[LC][NP];
    auto chunk_ptrs = [&](int l) {
      const int e = l < n0 ? n0 : nls;
#pragma unroll
      for (int q = 0; q < LC; ++q) load_ptrs(l + q < e ? l + q : e - 1, pr[q]);
    };
    chunk_ptrs(0);
    int l0 = 0;
    while (l0 < nls) {
      const int end = l0 < n0 ? n0 : nls;
      const int n = end - l0 < LC ? end - l0 : LC;
      u32x4 bv[LC][NW];
#pragma unroll
      for (int q = 0; q < LC; ++q) {
        if (q < n) {
          dma_tile(q, l0 + q);
          load_frags(l0 + q, pr[q], bv[q]);
        }
      }
      if (l0 + n < nls) chunk_ptrs(l0 + n);
      /* the LDS writes of the buffer loads are complete once vmcnt drains */
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();
      mma(l0 < n0 ? 0 : 1, n, bv);
      lds_barrier();
      l0 += n;
    }
  }
};

/* Single-matrix kernel (and SwiGLU for short prefills) on v_mfma_f32_32x32x16_bf16.
 * SW: SwiGLU (gate and up rows of one 32-row block per wave) or a single matrix (one 32-row
 * block per wave); MT: 32-token sub-tiles (token tile of 32 MT rows, a multiple of the 128-token
 * plan tile); D: weight ring depth (divides the group count); DB: token tile loads two groups
 * ahead (two register stages); APF: next sub-tile's LDS fragments loaded before the current
 * MFMAs; WV: waves per workgroup; OCC: waves per SIMD the registers are sized for; LC: expand
 * steps per chunk (their token tiles occupy LC LDS regions). */
template <bool SW, int MT, int D, bool DBT, bool APF, int WV, int OCC, int LC>
__global__ void __launch_bounds__(64 * WV, OCC) aos_gemm_kernel(aos_gemm_params p) {
  static_assert(MT % 4 == 0, "token tiles are whole plan tiles");
  constexpr int BM = 32 * MT;
  constexpr int TILE = BM * 128;
  constexpr int NT = 64 * WV;
  constexpr int NTILE = LC > 2 ? LC : 2;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, c = lane >> 5;
  int mbi, nbk;
  gemm_tile_of(blockIdx.x, p.mb, p.nb, mbi, nbk);
  const int m0 = mbi * BM;
  const int G = p.w0.G, in = p.w0.in, RB = p.w0.RB;

  /* this wave's 32-row block (of gate and of up for SW); dead blocks past the last read it and
   * store nothing */
  const int rb = nbk * WV + wave;
  const bool live = rb < RB;
  const int r0 = live ? rb : RB - 1;
  const aos_q4_dev &W0 = p.w0;
  const aos_q4_dev &W1 = SW ? p.w1 : p.w0;
  const u32x4 *q0 = (const u32x4 *)W0.qt + (size_t)r0 * G * 64 + lane;
  const u32x4 *q1 = (const u32x4 *)W1.qt + (size_t)r0 * G * 64 + lane;
  const uint32_t *s0p = W0.sb + (size_t)r0 * G * 32 + i;
  const uint32_t *s1p = W1.sb + (size_t)r0 * G * 32 + i;
  const int row = r0 * 32 + i;

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
    if (SW) {
      wq1[d] = q1[(size_t)d * 64];
      ws1[d] = s1p[(size_t)d * 32];
    }
  }
  /* Token tiles: LDS holds groups g and g + 1 (double buffer); registers hold the loads in
   * flight. With D even, two register stages let the loads run two groups ahead of their LDS
   * store. */
  constexpr bool DB = DBT && (D % 2) == 0;
  Stager<BM, NT> st0, st1;
  st0.load(p.x, in, p.T, m0, 0, tid);
  Expand<BM, WV, SW ? 2 : 1, 4, 2> ex(p, smem, NTILE, wave, lane, m0, mbi, row);
  ex.prefetch();
  st0.store(smem, tid);
  lds_barrier();

  /* token tile of weight group gx (clamped: the tiles staged past the last group are not read) */
  auto stage = [&](Stager<BM, NT> &st, const int gx) { st.load(p.x, in, p.T, m0, gx < G ? gx : G - 1, tid); };
  if (DB) stage(st1, 1);

  /* dequantise ring slot d into B fragments, then refill it with group gn */
  auto dequant_slot = [&](const int d, const int gn, u32x4 (&f0)[4], u32x4 (&f1)[4]) {
    {
      const float sc = aos_f16_to_f32(ws0[d] & 0xffffu), bi = aos_f16_to_f32(ws0[d] >> 16);
#pragma unroll
      for (int s = 0; s < 4; ++s) f0[s] = dequant_word(wq0[d][s], sc, bi);
    }
    if (SW) {
      const float sc = aos_f16_to_f32(ws1[d] & 0xffffu), bi = aos_f16_to_f32(ws1[d] >> 16);
#pragma unroll
      for (int s = 0; s < 4; ++s) f1[s] = dequant_word(wq1[d][s], sc, bi);
    }
    const int gc = gn < G ? gn : G - 1;
    wq0[d] = q0[(size_t)gc * 64];
    ws0[d] = s0p[(size_t)gc * 32];
    if (SW) {
      wq1[d] = q1[(size_t)gc * 64];
      ws1[d] = s1p[(size_t)gc * 32];
    }
  };

  /* one K group: ld receives group g + 2 (g + 1 without DB), sto holds group g + 1 */
  auto group = [&](const int g, const int d, Stager<BM, NT> &ld, Stager<BM, NT> &sto) {
    const unsigned char *tb = smem + (g & 1) * TILE;
    /* token fragments of the first sub-tile: their LDS latency overlaps the dequantisation */
    u32x4 a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = *(const u32x4 *)(tb + tile_off(i, 4 * c + s));
    stage(ld, g + (DB ? 2 : 1));
    u32x4 f0[4], f1[4];
    dequant_slot(d, g + D, f0, f1);
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
        if (SW) acc1[mt] = aos_mfma32(a[s], f1[s], acc1[mt]);
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

  /* LoRA expand: word s of lane (i, c) covers step columns 32 c + 8 s .. +7 */
  int n0;
  const int nls = ex.build(n0);
  if (nls > 0) {
    const int koff[4] = {32 * c, 32 * c + 8, 32 * c + 16, 32 * c + 24};
    auto mma_into = [&](int n, const u32x4 (&bv)[LC][4], f32x16 (&acc)[MT]) {
#pragma unroll
      for (int q = 0; q < LC; ++q) {
        if (q >= n) continue;
        const unsigned char *tb = smem + q * TILE;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          u32x4 a[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) a[s] = *(const u32x4 *)(tb + tile_off(mt * 32 + i, 4 * c + s));
#pragma unroll
          for (int s = 0; s < 4; ++s) acc[mt] = aos_mfma32(a[s], bv[q][s], acc[mt]);
        }
      }
    };
    ex.template run<LC>(nls, n0, koff, [&](int m, int n, const u32x4 (&bv)[LC][4]) {
      if (!SW || m == 0)
        mma_into(n, bv, acc0);
      else
        mma_into(n, bv, acc1);
    });
  }

  /* epilogue */
  if (!live) return;
  const int out = p.w0.out;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int tok = m0 + mt * 32 + aos_acc_m(v, lane);
      if (tok >= p.T) continue;
      if (SW) {
        const float gt = acc0[mt][v], up = acc1[mt][v];
        const float sg = 1.0f / (1.0f + expf(-gt));
        p.y[(size_t)tok * out + row] = aos_f32_to_bf16((gt * sg) * up);
      } else {
        p.y[(size_t)tok * out + row] = aos_f32_to_bf16(acc0[mt][v]);
      }
    }
  }
}

}  // namespace

extern "C" int aos_launch_pplan(const aos_pplan_params *p, const aos_launch_ctx *ctx) {
  const int mtiles = (p->T + AOS_GEMM_BM - 1) / AOS_GEMM_BM;
  if (p->T < 1 || p->T > AOS_PREFILL_MAX_T || p->n > AOS_MAX_ADAPTERS) return (int)hipErrorInvalidValue;
  AOS_LAUNCH(ctx, aos_pplan_kernel, dim3(mtiles), dim3(PLAN_NT), 0, *p);
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

/* Kernel shapes (measured on the 7B-shaped layer at 2048 tokens): 128-token tiles at two waves
 * per SIMD, so that one wave's dequantisation overlaps the other's matrix-core work; SwiGLU with
 * a shallow ring and single staging in 4-wave workgroups (two per CU), the single-matrix kernel
 * with the deep pipeline in 8-wave workgroups. */
template <bool SW, int MT, int D, bool DBT, bool APF, int WV, int OCC, int LC>
static void launch_gemm_cfg(const aos_gemm_params *p, const aos_launch_ctx *ctx) {
  constexpr int BM = 32 * MT, NTILE = LC > 2 ? LC : 2;
  aos_gemm_params q = *p;
  q.mb = (q.T + BM - 1) / BM;
  q.nb = (q.w0.RB + WV - 1) / WV;
  const size_t lds = (size_t)NTILE * BM * 128 + gemm_aux(BM) + ((size_t)q.lsteps_max * 2 + 15) / 16 * 16;
  const dim3 grid(q.mb * q.nb), block(64 * WV);
  const int G = q.w0.G;
  if (G % D == 0)
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, MT, D, DBT, APF, WV, OCC, LC>), grid, block, lds, q);
  else if (G % 2 == 0)
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, MT, 2, DBT, APF, WV, OCC, LC>), grid, block, lds, q);
  else
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, MT, 1, DBT, APF, WV, OCC, LC>), grid, block, lds, q);
}

extern "C" int aos_launch_gemm(const aos_gemm_params *p, int swiglu, const aos_launch_ctx *ctx) {
  if (swiglu)
    launch_gemm_cfg<true, 4, 2, false, false, 4, 2, 2>(p, ctx);
  else
    launch_gemm_cfg<false, 4, 4, true, true, 8, 2, 4>(p, ctx);
  return (int)hipGetLastError();
}
