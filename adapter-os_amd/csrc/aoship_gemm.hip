/*
 * aoship_gemm.hip — prefill path (T > 32 tokens): token grouping by adapter set, the LoRA shrink
 * over each tile's adapters, and the int4 GEMM with the fused LoRA expand (+ SwiGLU), all on the
 * matrix cores.
 *
 * Computes the MLX forward's linear(x, W) + apply_lora(x) (mlx_cpp_wrapper_real.cpp:3372-3419)
 * for a block of tokens, and in SwiGLU mode h = (g * sigmoid(g)) * u (:3509-3522); the ring ->
 * (adapter, scale * q / 32767) mapping is prepare_lora_for_ring
 * (crates/adapteros-lora-mlx-ffi/src/backend.rs:398-428).
 *
 * Launch sequence of one call:
 *   1. gplan    group the tokens by their active adapter set (groups in the order of their first
 *               token, tokens in index order: deterministic); for each 128-token tile of that order, the
 *               union of the adapters its tokens use, the tokens' coefficients over it and the
 *               union's A and B pointers;
 *   2. tshrink  S = x . A^T over each tile's union columns, K split into slices; the last slice of
 *               a tile to finish adds the slices in order and stores SA = bf16(coef * S);
 *   3. gemm     int4 GEMM over the sorted tiles (x rows gathered through the permutation), the
 *               expand over the tile's union columns added to the same accumulators after the
 *               K loop, outputs stored in sorted order (h) or scattered back (y).
 * Grouping makes a tile's union the one or two adapter sets of its tokens instead of every
 * adapter the whole batch uses.
 *
 * GEMM tiling for gfx950 (v_mfma_f32_32x32x16_bf16, 64-wide waves):
 *   - a workgroup of WV waves covers 128 tokens; each wave owns a 32-row block of weights
 *     (SwiGLU: the same rows of gate and up) for all the tokens of the tile;
 *   - weights come straight from the q4-tile layout (one 16-byte load per lane per group and row
 *     block) into registers through a ring D groups deep and are dequantised there to bfloat16
 *     B fragments (w = s * q + b in float32, hardware round-to-nearest-even packing), so each
 *     weight is read and dequantised once per workgroup;
 *   - the token tile of each group (128 rows x 64 bf16) is staged in LDS, double buffered,
 *     with an XOR swizzle of its 16-byte chunks so that fragment reads are free of bank
 *     conflicts; the waves share it;
 *   - workgroups are ordered so that the token tiles of one weight block run back to back on one
 *     XCD, whose L2 then serves the weight re-reads.
 */
#include "aoship_device.h"
#include "aoship_internal.h"
#include <hip/hip_ext.h>

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int BM = AOS_GEMM_BM; /* tokens per tile */
constexpr int SC1 = 16;         /* buffer cache policy: device-coherent (sc1) */

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* Workgroup barrier for a ring whose LDS writes come from buffer loads straight to LDS, whose
 * completion each wave has already waited for with a counted vmcnt: this wave's LDS reads have
 * returned (lgkmcnt 0), then s_barrier; the asm's memory clobber keeps the compiler from moving
 * memory accesses across it. (A release fence here would make the compiler drain every
 * outstanding memory load, the ring's later loads included: LDS DMA writes count as vector
 * memory operations.) */
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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

/* Stages the [BM x 64] bf16 slice of group g of a tile's token rows with NT threads. Row r of
 * the tile is token perm[m0 + r] (m0 + r without a permutation); rows past the last token repeat
 * it: they only feed accumulator rows that are never stored. */
template <int NT>
struct Stager {
  static constexpr int CH = BM * 8 / NT; /* 16-byte chunks per thread */
  u32x4 v[CH];
  int off[CH]; /* element offset of each chunk's row and column in group 0 */
  __device__ __forceinline__ void rows(const uint16_t *perm, int in, int T, int m0, int tid) {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int idx = tid + k * NT;
      const int r = idx >> 3, ch = idx & 7;
      const int ps = m0 + r < T ? m0 + r : T - 1;
      const int tok = perm ? (int)perm[ps] : ps;
      off[k] = tok * in + ch * 8;
    }
  }
  __device__ __forceinline__ void load(const uint16_t *x, int g) {
#pragma unroll
    for (int k = 0; k < CH; ++k) v[k] = *(const u32x4 *)(x + off[k] + g * 64);
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
/* group plan                                                                                 */
/* ------------------------------------------------------------------------------------------ */

/* A ring as ten 32-bit words (top_k, position, four words of adapter indices, four of gates). */
struct RingWords {
  uint32_t w[10];
  __device__ __forceinline__ void load(const aoship_ring_t *r) {
    const u32x2 *src = (const u32x2 *)r;
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      const u32x2 v = src[k];
      w[2 * k] = v.x;
      w[2 * k + 1] = v.y;
    }
  }
  __device__ __forceinline__ uint32_t top_k() const { return w[0]; }
  __device__ __forceinline__ int adapter(int s) const { return (int)((w[2 + (s >> 1)] >> (16 * (s & 1))) & 0xffffu); }
  __device__ __forceinline__ int gate(int s) const { return (int)(int16_t)((w[6 + (s >> 1)] >> (16 * (s & 1))) & 0xffffu); }
};

/* The active slots of a ring (prepare_lora_for_ring, backend.rs:409-425: slot s < top_k, gate
 * q > 0, a bound adapter index < n), each adapter once (its first slot): bit s of the result.
 * bound is the layer's bound flags in LDS. */
__device__ __forceinline__ uint32_t ring_set(const RingWords &r, int n, const uint8_t *bound, uint16_t (&ids)[8]) {
  uint32_t act = 0, mask = 0;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int a = r.adapter(s);
    ids[s] = (uint16_t)a;
    if (s < (int)r.top_k() && r.gate(s) > 0 && a < n && bound[a]) act |= 1u << s;
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    bool dup = false;
#pragma unroll
    for (int s2 = 0; s2 < s; ++s2) dup |= ((act >> s2) & 1u) && ids[s2] == ids[s];
    if (((act >> s) & 1u) && !dup) mask |= 1u << s;
  }
  return mask;
}

/* 32-bit hash of an adapter set, independent of the slots' order (a sum of mixed ids, then a
 * finaliser); the empty set hashes to 0 and every other set to a nonzero value, so tokens without
 * adapters sort first. Equal sets hash equally; a collision between different sets only
 * interleaves their tokens. */
__device__ __forceinline__ uint32_t set_hash(const uint16_t (&ids)[8], uint32_t mask) {
  if (!mask) return 0u;
  uint32_t h = 0;
#pragma unroll
  for (int s = 0; s < 8; ++s)
    if ((mask >> s) & 1u) {
      uint32_t v = (uint32_t)ids[s] * 0x9E3779B1u + 0x7F4A7C15u;
      v ^= v >> 16;
      v *= 0x85EBCA6Bu;
      v ^= v >> 13;
      h += v;
    }
  h ^= h >> 15;
  h *= 0x2c1b3c6du;
  h ^= h >> 12;
  return h ? h : 1u;
}

constexpr int GP_NT = 1024;
constexpr int GP_HT = 2 * AOS_PREFILL_MAX_T; /* hash table slots (load factor <= 1/2) */
constexpr int GP_BLK = AOS_PREFILL_MAX_T / 64; /* 64-token blocks: (pass, wave) in token order */
constexpr int GP_SMALL = 64;                   /* groups ranked with ballots; more fall back to a sort */
constexpr uint32_t GP_EMPTY = 0xffffffffu;

/* Dynamic LDS of the plan kernel. */
constexpr int GP_OFF_TABH = 0;
constexpr int GP_OFF_TABF = GP_OFF_TABH + GP_HT * 4;
constexpr int GP_OFF_BOUND = GP_OFF_TABF + GP_HT * 4;
constexpr int GP_OFF_BLK = GP_OFF_BOUND + AOS_MAX_ADAPTERS;
constexpr int GP_OFF_MISC = GP_OFF_BLK + GP_SMALL * GP_BLK * 4;
constexpr int GP_LDS = GP_OFF_MISC + (AOS_MAX_ADAPTERS / 32) * 4 + (AOS_MAX_ADAPTERS / 32 + 1) * 4 +
                       (GP_BLK + GP_SMALL + 2) * 4;

/* Compare-exchange of a bitonic network between this lane's key and the key of lane ^ d: the
 * lower lane keeps the smaller key of an ascending pair. */
__device__ __forceinline__ uint64_t bitonic_lane(uint64_t a, int lane, int d, bool up) {
  const uint64_t b = aos_shfl64(a, lane ^ d);
  const bool lower = (lane & d) == 0;
  const bool take_min = lower == up;
  return take_min ? (a < b ? a : b) : (a > b ? a : b);
}

/* Bitonic sort of key[0, NP) in LDS by the workgroup (element i: thread i % GP_NT); stages whose
 * partner lies in the same wave exchange through lane shuffles. */
__device__ void gp_sort(uint64_t *key, int NP) {
  const int tid = threadIdx.x, lane = tid & 63;
  for (int k = 2; k <= NP; k <<= 1) {
    int j = k >> 1;
    for (; j >= 64; j >>= 1) {
      for (int i = tid; i < NP; i += GP_NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t a = key[i], b = key[ixj];
          if (((i & k) == 0) ? (a > b) : (a < b)) {
            key[i] = b;
            key[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
    for (int i0 = 0; i0 < NP; i0 += GP_NT) {
      const int i = i0 + tid;
      if (i < NP) { /* uniform per wave: NP and GP_NT are multiples of 64 */
        uint64_t v = key[i];
        const bool up = (i & k) == 0;
        for (int d = j; d > 0; d >>= 1) v = bitonic_lane(v, lane, d, up);
        key[i] = v;
      }
    }
    __syncthreads();
  }
}

/* One workgroup per tile; every workgroup derives the same order of all the tokens, then writes
 * its own tile's slice: perm, the tile union (ascending), the pointer tables and the coefficient
 * rows.
 *
 * The order: tokens with equal adapter sets (equal set hashes) form a group; groups come in the
 * order of their first token, tokens within a group in index order. Each token finds its group's
 * first token through an LDS hash table (atomicMin per slot); the group index is the count of
 * first tokens before it. With at most GP_SMALL groups a token's position is its group's start
 * plus its rank among the group's tokens before it, counted with one ballot per (group, 64-token
 * block); otherwise the (first token, token) keys are sorted. */
__global__ void __launch_bounds__(GP_NT) aos_gplan_kernel(aos_gplan_params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char gsm[];
  uint32_t *tab_h = (uint32_t *)(gsm + GP_OFF_TABH);
  uint32_t *tab_f = (uint32_t *)(gsm + GP_OFF_TABF);
  uint8_t *bound_s = (uint8_t *)(gsm + GP_OFF_BOUND);
  uint32_t *blk = (uint32_t *)(gsm + GP_OFF_BLK);               /* [GP_SMALL][GP_BLK] */
  uint32_t *bits = (uint32_t *)(gsm + GP_OFF_MISC);            /* [AOS_MAX_ADAPTERS / 32] */
  int *base = (int *)(bits + AOS_MAX_ADAPTERS / 32);           /* [.. + 1] */
  uint32_t *wsum = (uint32_t *)(base + AOS_MAX_ADAPTERS / 32 + 1); /* [GP_BLK] */
  uint32_t *gstart = wsum + GP_BLK;                            /* [GP_SMALL + 1] */
  uint32_t *ngroups = gstart + GP_SMALL + 1;
  uint16_t *tperm = (uint16_t *)tab_h; /* sorted position -> token, once the table is done */
  uint64_t *key = (uint64_t *)tab_h;   /* sort keys of the fallback, likewise */
  constexpr int RPT = AOS_PREFILL_MAX_T / GP_NT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, T = p.T, n = p.n;
  const uint64_t lt = (1ull << lane) - 1ull;

  for (int a = tid; a < n; a += GP_NT) bound_s[a] = p.bound[a];
  for (int e = tid; e < GP_HT; e += GP_NT) {
    tab_h[e] = GP_EMPTY;
    tab_f[e] = GP_EMPTY;
  }
  RingWords rw[RPT];
#pragma unroll
  for (int q = 0; q < RPT; ++q) {
    const int t = tid + q * GP_NT;
    if (t < T) rw[q].load(p.rings + t);
  }
  __syncthreads();
  /* group of each token: its set's hash, inserted into the table by every token (linear probing:
   * the first insert of a hash claims an empty slot, later ones of the same hash stop there, other
   * hashes probe on; slots are never cleared), and the slot keeps the lowest token */
  uint32_t slot[RPT];
#pragma unroll
  for (int q = 0; q < RPT; ++q) {
    const int t = tid + q * GP_NT;
    slot[q] = 0;
    if (t < T) {
      uint16_t ids[8];
      uint32_t h = set_hash(ids, ring_set(rw[q], n, bound_s, ids));
      h = h == GP_EMPTY ? GP_EMPTY - 1u : h;
      uint32_t sl = (h * 0x9E3779B1u) >> 19; /* 13 bits: GP_HT slots */
      for (;;) {
        const uint32_t old = atomicCAS(&tab_h[sl], GP_EMPTY, h);
        if (old == GP_EMPTY || old == h) break;
        sl = (sl + 1) & (GP_HT - 1);
      }
      atomicMin(&tab_f[sl], (uint32_t)t);
      slot[q] = sl;
    }
  }
  __syncthreads();
  /* group index = number of first tokens before the group's first token: a scan over the
   * 64-token blocks in token order */
  uint32_t first[RPT];
  uint64_t fb[RPT];
#pragma unroll
  for (int q = 0; q < RPT; ++q) {
    const int t = tid + q * GP_NT;
    first[q] = t < T ? tab_f[slot[q]] : GP_EMPTY;
    fb[q] = __ballot(t < T && first[q] == (uint32_t)t);
    if (lane == 0) wsum[q * (GP_NT / 64) + wave] = (uint32_t)__popcll(fb[q]);
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t acc = 0;
    for (int b = 0; b < GP_BLK; ++b) {
      const uint32_t v = wsum[b];
      wsum[b] = acc;
      acc += v;
    }
    *ngroups = acc;
  }
  __syncthreads();
  const uint32_t D = *ngroups;
#pragma unroll
  for (int q = 0; q < RPT; ++q) {
    const int t = tid + q * GP_NT;
    if (t < T && first[q] == (uint32_t)t) tab_f[slot[q]] = wsum[q * (GP_NT / 64) + wave] + (uint32_t)__popcll(fb[q] & lt);
  }
  __syncthreads();
  uint32_t gid[RPT];
#pragma unroll
  for (int q = 0; q < RPT; ++q) gid[q] = tid + q * GP_NT < T ? tab_f[slot[q]] : GP_EMPTY;
  __syncthreads(); /* the table is no longer read: its memory takes the order */

  if (D <= (uint32_t)GP_SMALL) {
    uint32_t rank[RPT];
#pragma unroll
    for (int q = 0; q < RPT; ++q) rank[q] = 0;
    for (uint32_t g = 0; g < D; ++g) {
#pragma unroll
      for (int q = 0; q < RPT; ++q) {
        const uint64_t b = __ballot(gid[q] == g);
        if (lane == 0) blk[g * GP_BLK + q * (GP_NT / 64) + wave] = (uint32_t)__popcll(b);
        if (gid[q] == g) rank[q] = (uint32_t)__popcll(b & lt);
      }
    }
    __syncthreads();
    if (tid < (int)D) { /* block prefix within group tid, and its size */
      uint32_t acc = 0;
      for (int b = 0; b < GP_BLK; ++b) {
        const uint32_t v = blk[tid * GP_BLK + b];
        blk[tid * GP_BLK + b] = acc;
        acc += v;
      }
      gstart[tid + 1] = acc;
    }
    __syncthreads();
    if (tid == 0) {
      gstart[0] = 0;
      for (uint32_t g = 1; g <= D; ++g) gstart[g] += gstart[g - 1];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
      const int t = tid + q * GP_NT;
      if (t < T) tperm[gstart[gid[q]] + blk[gid[q] * GP_BLK + q * (GP_NT / 64) + wave] + rank[q]] = (uint16_t)t;
    }
  } else {
    int NP = 64;
    while (NP < T) NP <<= 1;
#pragma unroll
    for (int q = 0; q < RPT; ++q) {
      const int t = tid + q * GP_NT;
      if (t < NP) key[t] = t < T ? ((uint64_t)first[q] << 32) | (uint32_t)t : ~0ull;
    }
    __syncthreads();
    gp_sort(key, NP);
    /* keys -> tokens in place, a pass of GP_NT at a time: pass j writes bytes 2 i of tperm, which
     * hold keys below (j + 1) * GP_NT / 4, all read by passes up to j */
    for (int j = 0; j * GP_NT < T; ++j) {
      const int i = j * GP_NT + tid;
      const uint16_t t = i < T ? (uint16_t)(uint32_t)key[i] : 0;
      __syncthreads();
      if (i < T) tperm[i] = t;
      __syncthreads();
    }
  }
  __syncthreads();

  const int mt = blockIdx.x, p0 = mt * BM;
  const int mtiles = (T + BM - 1) / BM;
  const int tn = T - p0 < BM ? T - p0 : BM;
  const int words = (n + 31) >> 5;
  for (int w = tid; w < words; w += GP_NT) bits[w] = 0u;
  __syncthreads();
  uint16_t ids[8];
  int tok = 0;
  RingWords r;
  if (tid < tn) {
    tok = tperm[p0 + tid];
    p.perm[p0 + tid] = (uint16_t)tok;
    r.load(p.rings + tok);
    const uint32_t set = ring_set(r, n, bound_s, ids);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if ((set >> q) & 1u) atomicOr(&bits[ids[q] >> 5], 1u << (ids[q] & 31));
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int w = 0; w < words; ++w) {
      base[w] = acc;
      acc += __builtin_popcount(bits[w]);
    }
    base[words] = acc;
    p.tu[mt] = acc;
  }
  __syncthreads();
  const int U = base[words];
  const size_t trow = (size_t)mt * p.tu_cap;
  for (int a = tid; a < n; a += GP_NT) {
    const uint32_t m = bits[a >> 5];
    if ((m >> (a & 31)) & 1u) {
      const int u = base[a >> 5] + __builtin_popcount(m & ((1u << (a & 31)) - 1u));
      p.list[trow + u] = (uint16_t)a;
      for (int k = 0; k < p.nmod; ++k) {
        const aos_lora_tab &tb = p.tab[k];
        const bool has = tb.rpad && a < tb.n;
        p.ap[(size_t)k * mtiles * p.tu_cap + trow + u] = has ? tb.A[a] : nullptr;
        p.bp[(size_t)k * mtiles * p.tu_cap + trow + u] = has ? tb.Bf[a] : nullptr;
      }
    }
  }
  /* coefficient rows of the tile: each token's (slot, coefficient) pairs by one thread, summed in
   * ring order per union slot (an adapter named twice adds up in order), staged in LDS (the hash
   * table's second half is free); then the rows, zeros elsewhere, with consecutive threads on
   * consecutive entries */
  int *cu = (int *)tab_f;
  float *cc = (float *)(tab_f + 8 * BM);
  if (tid < tn) {
    int us[8];
    float cv[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int a = r.adapter(s);
      const int q = r.gate(s);
      us[s] = -1;
      cv[s] = 0.0f;
      if (s < (int)r.top_k() && q > 0 && a < n && bound_s[a]) {
        const uint32_t m = bits[a >> 5];
        const int u = base[a >> 5] + __builtin_popcount(m & ((1u << (a & 31)) - 1u));
        const float c = p.scale[a] * ((float)q / 32767.0f);
        int first_s = s;
#pragma unroll
        for (int s2 = 0; s2 < s; ++s2)
          if (first_s == s && us[s2] == u) first_s = s2;
        if (first_s == s) {
          us[s] = u;
          cv[s] = 0.0f + c;
        } else {
          cv[first_s] += c;
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      cu[tid * 8 + s] = us[s];
      cc[tid * 8 + s] = cv[s];
    }
  }
  __syncthreads();
  for (int e = tid; e < tn * U; e += GP_NT) {
    const int r = e / U, u = e - r * U;
    float v = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (cu[r * 8 + s] == u) v = cc[r * 8 + s];
    p.coef[(size_t)(p0 + r) * p.tu_cap + u] = v;
  }
}

/* ------------------------------------------------------------------------------------------ */
/* tile shrink                                                                                */
/* ------------------------------------------------------------------------------------------ */

/* Union columns of tile mt for the shrink's modules: module i holds tu * rpad[i] columns after
 * those of modules before it. */
__device__ __forceinline__ int tile_cols(const aos_tshrink_params &p, int tu) {
  int c = 0;
  for (int i = 0; i < p.nmod; ++i) c += tu * p.rpad[i];
  return c;
}

/* Workgroup (K slice kz, column set cs of 128 columns, tile mt), kz fastest; wave w takes the
 * 32 columns cs * 128 + 32 w .., all 128 tokens (four 32-token sub-tiles). The slice's token
 * tiles and A fragments are loaded two groups ahead. Once every slice of the (tile, column set)
 * has published its partial sums (the ks workgroups are consecutive: dispatched together, none
 * waits on a later one), slice kz sums rows kz * 128 / ks .. of them over the slices in order. */
__global__ void __launch_bounds__(256) aos_tshrink_kernel(aos_tshrink_params p) {
  constexpr int MT = BM / 32, TILE = BM * 128;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ uint32_t met;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, c = lane >> 5;
  const int kz = blockIdx.x, cs = blockIdx.y, mt = blockIdx.z;
  const int TU = __builtin_amdgcn_readfirstlane(p.tu[mt]);
  if (p.am_tu > 0 && TU >= p.am_tu) return; /* the adapter-major shrink's tile (uniform, as below) */
  const int C = tile_cols(p, TU);
  const int csets = (C + 127) / 128;
  if (cs >= csets) return; /* uniform; such workgroups take no part in the meeting below */
  const int m0 = mt * BM;
  const int tn = p.T - m0 < BM ? p.T - m0 : BM;
  const int G = p.in / 64;
  const int g_lo = (int)((long)kz * G / p.ks), g_hi = (int)((long)(kz + 1) * G / p.ks);

  /* this lane's A row: column col of the tile's union columns */
  const int col = cs * 128 + 32 * wave + i;
  const uint16_t *arow = p.zero_row;
  size_t kstep = 0;
  if (col < C) {
    int mi = 0, off = 0;
    while (mi < p.nmod - 1 && col >= off + TU * p.rpad[mi]) {
      off += TU * p.rpad[mi];
      ++mi;
    }
    const int rp = p.rpad[mi];
    const int u = (col - off) / rp, j = col - off - u * rp;
    const uint16_t *A = p.ap[((size_t)mi * p.mtiles + mt) * p.tu_cap + u];
    if (A) {
      arow = A + (size_t)j * p.in;
      kstep = 1;
    }
  }
  auto aload = [&](int g, u32x4 (&a)[4]) {
    const int gc = g < g_hi ? g : g_hi - 1;
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = aos_gld16(arow + kstep * ((size_t)gc * 64 + 16 * s + 8 * c));
  };

  f32x16 acc[MT];
#pragma unroll
  for (int s = 0; s < MT; ++s) acc[s] = f32x16{};
  if (g_lo < g_hi) {
    Stager<256> st0, st1;
    st0.rows(p.perm, p.in, p.T, m0, tid);
#pragma unroll
    for (int k = 0; k < Stager<256>::CH; ++k) st1.off[k] = st0.off[k];
    u32x4 a0[4], a1[4];
    st0.load(p.x, g_lo);
    st1.load(p.x, g_lo + 1 < g_hi ? g_lo + 1 : g_hi - 1);
    aload(g_lo, a0);
    aload(g_lo + 1, a1);
    st0.store(smem, tid);
    lds_barrier();
    /* group g from LDS buffer (g - g_lo) & 1 with A fragments a; hold (group g + 1) goes to the
     * other buffer, ld receives group g + 2 and a is refilled with group g + 2 after its MFMAs.
     * Every load is unconditional (clamped to the slice), so no branch separates a load from its
     * use and the compiler waits for exactly the loads each step needs. */
    auto step = [&](int g, Stager<256> &hold, Stager<256> &ld, u32x4 (&a)[4]) {
      const unsigned char *tb = smem + ((g - g_lo) & 1) * TILE;
      ld.load(p.x, g + 2 < g_hi ? g + 2 : g_hi - 1);
#pragma unroll
      for (int s = 0; s < MT; ++s) {
        const int r = s * 32 + i;
        u32x4 xv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) xv[k] = *(const u32x4 *)(tb + tile_off(r, 2 * k + c)); /* K 16 k + 8 c */
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[s] = aos_mfma32(xv[k], a[k], acc[s]);
      }
      aload(g + 2, a);
      hold.store(smem + (((g - g_lo) & 1) ^ 1) * TILE, tid);
      lds_barrier();
    };
    int g = g_lo;
    for (; g + 1 < g_hi; g += 2) {
      step(g, st1, st0, a0);
      step(g + 1, st0, st1, a1);
    }
    if (g < g_hi) step(g, st1, st0, a0);
  }

  /* this slice's partial sums, device-coherent (the other slices read them), column-major:
   * registers 4q .. 4q + 3 of a lane hold four consecutive rows of its column, one 16-byte store */
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(p.part + (size_t)mt * p.ks * p.s_stride * BM), (short)0, (int)((size_t)p.ks * p.s_stride * BM * 4),
      0x00020000);
  if (col < C) {
    const int cbase = (kz * p.s_stride + col) * BM;
#pragma unroll
    for (int s = 0; s < MT; ++s)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 v = {acc[s][4 * q], acc[s][4 * q + 1], acc[s][4 * q + 2], acc[s][4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs,
                                               (cbase + s * 32 + 8 * q + 4 * c) * 4, 0, SC1);
      }
  }
  /* meet the other slices of this (tile, column set): the last to arrive resets the count and
   * raises the flag to this launch's generation */
  aos_mem_wait();
  __syncthreads();
  if (tid == 0) {
    const size_t gi = (size_t)mt * p.csets + cs;
    bool ok = true;
    if (aos_arrive(&p.counters[gi]) == (uint32_t)p.ks - 1u) {
      aos_reset(&p.counters[gi]);
      aos_raise(p.flags + gi * 32, p.gen);
    } else {
      ok = aos_wait_gen(p.flags + gi * 32, p.gen);
      if (!ok && p.timeout) __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    met = ok ? 1u : 0u;
  }
  __syncthreads();
  if (!met) return;

  /* this slice's share of the column set (blocks of 4 columns kz, kz + ks, ..., all the rows):
   * SA = bf16(coef * sum of the slices in order) over blocks of 4 rows x 4 columns, the row block
   * fastest across lanes so that each load reads consecutive rows of one column; every slice's
   * loads of a block are in flight before the adds */
  const int nrb = (tn + 3) / 4;
  const int c0 = cs * 128, cn = C - c0 < 128 ? C - c0 : 128;
  const int ncb = cn / 4; /* C is a multiple of 16 */
  const int mycb = ncb > kz ? (ncb - kz + p.ks - 1) / p.ks : 0;
  for (int e = tid; e < mycb * nrb; e += 256) {
    const int r = (e % nrb) * 4, cc = c0 + (kz + (e / nrb) * p.ks) * 4;
    f32x4 sum[4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f},
                    {0.0f, 0.0f, 0.0f, 0.0f}}; /* sum[j]: column cc + j, rows r .. r + 3 */
    for (int k0 = 0; k0 < p.ks; k0 += 4) {
      f32x4 v[4][4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int kk = k0 + k < p.ks ? k0 + k : p.ks - 1;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[k][j] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, ((kk * p.s_stride + cc + j) * BM + r) * 4, 0, SC1));
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k0 + k < p.ks) {
#pragma unroll
          for (int j = 0; j < 4; ++j) sum[j] += v[k][j];
        }
    }
    int mi = 0, off = 0;
    while (mi < p.nmod - 1 && cc >= off + TU * p.rpad[mi]) {
      off += TU * p.rpad[mi];
      ++mi;
    }
    const int u = (cc - off) / p.rpad[mi];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      if (r + e2 >= tn) break;
      const float cf = p.coef[(size_t)(m0 + r + e2) * p.tu_cap + u];
      u32x2 o;
      o.x = (uint32_t)aos_f32_to_bf16(cf * sum[0][e2]) | ((uint32_t)aos_f32_to_bf16(cf * sum[1][e2]) << 16);
      o.y = (uint32_t)aos_f32_to_bf16(cf * sum[2][e2]) | ((uint32_t)aos_f32_to_bf16(cf * sum[3][e2]) << 16);
      *(u32x2 *)(p.SA + (size_t)(m0 + r + e2) * p.s_stride + cc) = o;
    }
  }
}

/* ------------------------------------------------------------------------------------------ */
/* adapter-major shrink                                                                       */
/* ------------------------------------------------------------------------------------------ */

constexpr int AM_NT = 512; /* plan threads */
constexpr int AM_ZB = 8;    /* zeroing workgroups per tile */
constexpr int AM_CB = 8;    /* coefficients each thread has in flight */

/* Workgroup (x, mt) of the tiles with tu >= am_tu. x = 0: counts the tile's users per union slot
 * in LDS, reserves each slot's range of its adapter's list with one atomic add and places the
 * users; the last of these to arrive builds the chunk table and resets the counts. x = 1 ..
 * AM_ZB: zero rows (x - 1) * 128 / AM_ZB .. of the tile's union columns in each SA buffer (the
 * users' entries are overwritten by the shrink). */
__global__ void __launch_bounds__(AM_NT) aos_amplan_kernel(aos_amplan_params p) {
  __shared__ uint32_t lc[AOS_TILE_U_MAX], base[AOS_TILE_U_MAX];
  __shared__ uint32_t cst[AM_NT];
  __shared__ uint32_t last;
  const int tid = threadIdx.x, mt = blockIdx.y;
  const int TU = __builtin_amdgcn_readfirstlane(p.tu[mt]);
  const bool am = p.am_tu > 0 && TU >= p.am_tu;
  const int m0 = mt * BM, tn = p.T - m0 < BM ? p.T - m0 : BM;
  if (blockIdx.x > 0) {
    if (!am) return;
    const int r0 = (blockIdx.x - 1) * BM / AM_ZB, r1 = blockIdx.x * BM / AM_ZB < tn ? blockIdx.x * BM / AM_ZB : tn;
#pragma unroll
    for (int z = 0; z < 2; ++z) {
      if (z >= p.nz) break;
      int C = 0;
      for (int i = 0; i < p.zb[z].nmod; ++i) C += TU * p.zb[z].rpad[i];
      const int c8 = C / 8; /* C is a multiple of 16 */
      uint16_t *SA = p.zb[z].SA;
      const size_t st = (size_t)p.zb[z].s_stride;
      for (int e = tid; e < (r1 - r0) * c8; e += AM_NT) {
        const int r = e / c8, q = e - r * c8;
        *(u32x4 *)(SA + (size_t)(m0 + r0 + r) * st + 8 * q) = u32x4{0u, 0u, 0u, 0u};
      }
    }
    return;
  }
  if (am) {
    const float *cf = p.coef + (size_t)m0 * p.tu_cap;
    const uint16_t *ls = p.list + (size_t)mt * p.tu_cap;
    for (int u = tid; u < TU; u += AM_NT) lc[u] = 0;
    __syncthreads();
    const int ne = tn * TU;
    /* entry e = r * TU + u, AM_CB of a thread's entries loaded before any is used */
    auto coefs = [&](int e0, float (&v)[AM_CB], int (&uu)[AM_CB], int (&rr)[AM_CB]) {
#pragma unroll
      for (int k = 0; k < AM_CB; ++k) {
        const int e = e0 + k * AM_NT + tid;
        rr[k] = e / TU;
        uu[k] = e - rr[k] * TU;
        v[k] = e < ne ? cf[(size_t)rr[k] * p.tu_cap + uu[k]] : 0.0f;
      }
    };
    for (int e0 = 0; e0 < ne; e0 += AM_CB * AM_NT) {
      float v[AM_CB];
      int uu[AM_CB], rr[AM_CB];
      coefs(e0, v, uu, rr);
#pragma unroll
      for (int k = 0; k < AM_CB; ++k)
        if (v[k] != 0.0f) atomicAdd(&lc[uu[k]], 1u);
    }
    __syncthreads();
    for (int u = tid; u < TU; u += AM_NT) {
      base[u] = lc[u] ? __hip_atomic_fetch_add(&p.count[ls[u]], lc[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
      lc[u] = 0;
    }
    __syncthreads();
    for (int e0 = 0; e0 < ne; e0 += AM_CB * AM_NT) {
      float v[AM_CB];
      int uu[AM_CB], rr[AM_CB];
      coefs(e0, v, uu, rr);
#pragma unroll
      for (int k = 0; k < AM_CB; ++k)
        if (v[k] != 0.0f) {
          const uint32_t kk = base[uu[k]] + atomicAdd(&lc[uu[k]], 1u);
          p.users[(size_t)ls[uu[k]] * p.T + kk] = ((uint32_t)(m0 + rr[k]) << 16) | (uint32_t)uu[k];
        }
    }
    if (p.tinfo) { /* each slot's range of its adapter's users, and the slot of each adapter */
      __syncthreads();
      for (int u = tid; u < TU; u += AM_NT) p.tinfo[(size_t)mt * p.tu_cap + u] = (base[u] << 8) | lc[u];
      if (p.xam_tu > 0 && TU >= p.xam_tu) {
        uint16_t *inv = p.inv + (size_t)mt * p.n;
        for (int a = tid; a < p.n; a += AM_NT) inv[a] = 0xffffu;
        __syncthreads();
        for (int u = tid; u < TU; u += AM_NT) inv[ls[u]] = (uint16_t)u;
      }
    }
  }
  /* arrive once this workgroup's atomics and stores are complete */
  aos_mem_wait();
  __syncthreads();
  if (tid == 0) last = aos_arrive(p.done) == gridDim.y - 1u ? 1u : 0u;
  __syncthreads();
  if (!last) return;
  /* the chunk table: thread t takes adapters t * per .. (every count is final) */
  const int per = (p.n + AM_NT - 1) / AM_NT;
  const int a0 = tid * per, a1 = a0 + per < p.n ? a0 + per : p.n;
  uint32_t mine = 0;
  for (int a = a0; a < a1; ++a)
    mine += (__hip_atomic_load(&p.count[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + BM - 1) / BM;
  cst[tid] = mine;
  __syncthreads();
  for (int off = 1; off < AM_NT; off <<= 1) { /* inclusive scan */
    const uint32_t v = tid >= off ? cst[tid - off] : 0u;
    __syncthreads();
    cst[tid] += v;
    __syncthreads();
  }
  uint32_t c = cst[tid] - mine;
  for (int a = a0; a < a1; ++a) {
    const uint32_t n = __hip_atomic_load(&p.count[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t j = 0; j * BM < n; ++j, ++c) {
      const uint32_t nu = n - j * BM < (uint32_t)BM ? n - j * BM : (uint32_t)BM;
      if (c < (uint32_t)p.cb) p.ctab[c] = ((uint32_t)a << 16) | (j << 8) | nu;
    }
    __hip_atomic_store(&p.count[a], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  for (uint32_t e = cst[AM_NT - 1] + tid; e < (uint32_t)p.cb; e += AM_NT) p.ctab[e] = 0u;
  if (tid == 0 && p.xl) { /* the adapter-major expand's tiles, in order */
    uint32_t k = 0;
    for (int t = 0; t < (int)gridDim.y; ++t)
      if (p.xam_tu > 0 && p.tu[t] >= p.xam_tu) p.xl[k++] = (uint32_t)t;
    p.xl[gridDim.y] = k;
  }
  if (tid == 0) aos_reset(p.done);
}

/* Exclusive scan of a[0, n) (n <= 4 * 256) in place by 256 threads, a[n] = the total. */
__device__ __forceinline__ void scan256(uint32_t *a, int n, uint32_t *tmp) {
  const int tid = threadIdx.x;
  uint32_t v[4], s = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = 4 * tid + k < n ? a[4 * tid + k] : 0u;
    s += v[k];
  }
  tmp[tid] = s;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const uint32_t w = tid >= off ? tmp[tid - off] : 0u;
    __syncthreads();
    tmp[tid] += w;
    __syncthreads();
  }
  uint32_t run = tmp[tid] - s;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (4 * tid + k < n) {
      a[4 * tid + k] = run;
      run += v[k];
    }
  if (tid == 255) a[n] = tmp[255];
  __syncthreads();
}

constexpr int XAM_RL = AOS_XAM_RT * BM * 8; /* users a range holds at most */
constexpr int XAM_CT = AOS_XAM_CT;
constexpr uint16_t XAM_SPARE = AOS_XAM_RT * BM; /* the spare LDS row */

/* Range r of the adapter-major expand's tiles: its users in adapter order (tiles in range order
 * within an adapter), their entries in the compact copy, the chunks, and each chunk's local rows
 * padded to 128 with the spare row (one all-spare chunk after the last). */
__global__ void __launch_bounds__(256) aos_amxlist_kernel(aos_amx_params p) {
  constexpr int RT = AOS_XAM_RT;
  __shared__ uint32_t off[AOS_XAM_MAX_N * RT + 1], bas[AOS_XAM_MAX_N * RT + 1], tmp[256], ctl[XAM_CT];
  __shared__ uint16_t lrow[XAM_RL];
  __shared__ uint32_t tl[RT];
  const int tid = threadIdx.x, r = blockIdx.x;
  const int xc = (int)p.xl[p.mtiles];
  const int t0 = r * RT, nt = xc - t0 < RT ? xc - t0 : RT;
  if (nt <= 0) {
    if (tid == 0) p.nch[r] = 0;
    return;
  }
  if (tid < nt) tl[tid] = p.xl[t0 + tid];
  __syncthreads();
  const int ne = p.n * RT; /* entry (a, t): adapter a's users in tile t of the range */
  for (int e = tid; e < ne; e += 256) {
    const int a = e / RT, t = e - a * RT;
    uint32_t c = 0, b = 0;
    if (t < nt) {
      const uint32_t tile = tl[t];
      const uint32_t u = p.inv[(size_t)tile * p.n + a];
      if (u != 0xffffu) {
        const uint32_t w = p.tinfo[(size_t)tile * p.tu_cap + u];
        c = w & 255u;
        b = w >> 8;
      }
    }
    off[e] = c;
    bas[e] = b;
  }
  __syncthreads();
  scan256(off, ne, tmp);
  const uint32_t total = off[ne];
  for (uint32_t k = tid; k < total; k += 256) {
    int lo = 0, hi = ne - 1; /* the last entry starting at or before k */
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (off[mid] <= k) lo = mid;
      else hi = mid - 1;
    }
    const int a = lo / RT, t = lo - a * RT;
    const size_t ui = (size_t)a * p.T + bas[lo] + (k - off[lo]);
    lrow[k] = (uint16_t)(t * BM + ((p.users[ui] >> 16) - tl[t] * BM));
    p.cidx[ui] = (uint32_t)r * XAM_RL + k;
  }
  __syncthreads();
  for (int a = tid; a < p.n; a += 256) bas[a] = (off[(a + 1) * RT] - off[a * RT] + BM - 1) / BM;
  __syncthreads();
  scan256(bas, p.n, tmp);
  const int nch = (int)bas[p.n];
  uint32_t *ct = p.ct + (size_t)r * XAM_CT;
  for (int a = tid; a < p.n; a += 256) {
    const uint32_t s = off[a * RT], len = off[(a + 1) * RT] - s;
    for (uint32_t j = 0; j * BM < len; ++j) {
      const uint32_t nu = len - j * BM < (uint32_t)BM ? len - j * BM : (uint32_t)BM;
      const uint32_t w = ((s + j * BM) << 15) | ((uint32_t)a << 8) | nu;
      ctl[bas[a] + j] = w;
      ct[bas[a] + j] = w;
    }
  }
  if (tid == 0) {
    ctl[nch] = 0u;
    ct[nch] = 0u;
    p.nch[r] = (uint32_t)nch;
  }
  __syncthreads();
  uint16_t *rlp = p.rlp + (size_t)r * XAM_CT * BM;
  for (int e = tid; e < (nch + 1) * BM; e += 256) {
    const uint32_t w = ctl[e >> 7];
    const uint32_t slot = (uint32_t)e & 127u;
    rlp[e] = slot < (w & 255u) ? lrow[(w >> 15) + slot] : XAM_SPARE;
  }
}

/* Workgroup (range r, module m, 32-row block r0), r0 fastest: the range's float32 sums for the
 * block in LDS ([RT * 128 rows + 1 spare][32]); the chunks in order, wave w taking users 32 w .. of
 * each: A operand the users' rows of the compact SA copy, B operand the adapter's B rows r0 * 32 ..
 * in fragment order, one 32 x 32 product (KS = rank / 16 steps), added to the users' rows (distinct
 * within a chunk; a barrier between chunks keeps each row's adds in chunk order, which is adapter
 * order); slots past a chunk's users add into the spare row. Chunk k + XAM_D's loads are issued
 * after chunk k's adds; chunk k + 1's products are formed before the barrier that ends them. The
 * loads are buffer loads whose per-lane offsets never change (the chunk moves the base; an adapter
 * without the module reads through a zero-size range: zeros), all unconditional: a load under a
 * branch makes the compiler wait for every load in flight where the branches join, which took the
 * 4-deep prefetch down to one chunk at a time (1.57 ms for C5's 8 widest tiles). LDS float atomic
 * adds instead of the read-add-writes: 6x slower. Last, each tile's 128 x 32 block stored in
 * accumulator order. */
constexpr int XAM_D = 4;
template <int KS>
__global__ void __launch_bounds__(256, 2) aos_amxexp_kernel(aos_amx_params p) {
  constexpr int RT = AOS_XAM_RT, MT = BM / 32, RP = 16 * KS, CW = 2 * RP;
  extern __shared__ __attribute__((aligned(16))) float accs[]; /* [RT * BM + 1][32] */
  __shared__ uint32_t tl[RT], ctl[XAM_CT];
  __shared__ const uint16_t *bps[AOS_XAM_MAX_N];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, c = lane >> 5;
  const int b = blockIdx.x, r0 = b % p.RB, m = (b / p.RB) & 1, r = b / (2 * p.RB);
  const int xc = __builtin_amdgcn_readfirstlane((int)p.xl[p.mtiles]);
  const int t0 = r * RT, nt = xc - t0 < RT ? xc - t0 : RT;
  if (nt <= 0) return; /* uniform */
  const int nch = __builtin_amdgcn_readfirstlane((int)p.nch[r]);
  for (int e = tid; e < (RT * BM + 1) * 32 / 4; e += 256) ((f32x4 *)accs)[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (tid < nt) tl[tid] = p.xl[t0 + tid];
  for (int a = tid; a < p.n; a += 256) bps[a] = p.Bf[m][a];
  for (int k = tid; k <= nch; k += 256) ctl[k] = p.ct[(size_t)r * XAM_CT + k];
  __syncthreads();
  const uint32_t bbytes = (uint32_t)p.RB * 32 * RP * 2;
  /* per-lane byte offsets: user 32 wave + i's row of the chunk, K piece 8 c; B row r0 * 32 + i */
  const int va = ((wave * 32 + i) * CW + (m ? RP : 0) + 8 * c) * 2;
  const int vb = ((r0 * (RP / 8) + c) * 256 + i * 8) * 2;
  const uint16_t *rlp = p.rlp + (size_t)r * XAM_CT * BM + wave * 32 + 4 * c;
  struct Stage {
    u32x4 av[KS], bv[KS];
    u32x2 lo[4]; /* LDS rows of the 16 accumulator rows 8 q + 4 c + e, e = 0..3 in lo[q] */
  };
  Stage st[XAM_D];
  auto issue = [&](int k, Stage &S) {
    const int kk = k < nch ? k : nch; /* past the last: the all-spare chunk */
    const uint32_t w = ctl[kk];
    const uint32_t s0 = (uint32_t)r * XAM_RL + (w >> 15), a = (w >> 8) & 127u;
    /* the chunk's own rows only: lanes past its users read zeros without a memory access */
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)(p.SAc + (size_t)s0 * CW), (short)0,
                                                                        (int)((w & 255u) * CW * 2), 0x00020000);
    const uint16_t *bb = bps[a];
    /* a wave without users in the chunk (or an adapter without the module) reads zeros */
    const bool wb = bb && (uint32_t)(wave * 32) < (w & 255u);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void *)bb, (short)0, wb ? (int)bbytes : 0, 0x00020000);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      S.av[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, va + 32 * s, 0, 0));
      S.bv[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, vb + 1024 * s, 0, 0));
    }
    const uint16_t *lr = rlp + (size_t)kk * BM;
#pragma unroll
    for (int q = 0; q < 4; ++q) S.lo[q] = *(const __attribute__((address_space(1))) u32x2 *)(lr + 8 * q);
  };
  auto products = [&](const Stage &S) {
    f32x16 d = f32x16{};
#pragma unroll
    for (int s = 0; s < KS; ++s) d = aos_mfma32(S.av[s], S.bv[s], d);
    return d;
  };
  auto add = [&](const f32x16 &d, const Stage &S) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t wd = e < 2 ? S.lo[q].x : S.lo[q].y;
        const uint32_t lr = (wd >> (16 * (e & 1))) & 0xffffu;
        accs[lr * 32 + i] += d[4 * q + e];
      }
  };
  if (nch > 0) {
#pragma unroll
    for (int d = 0; d < XAM_D; ++d) issue(d, st[d]);
    /* every prologue load complete (vmcnt 0; expcnt and lgkmcnt at their maxima): the compiler
     * otherwise merges the prologue's load order into the loop head's and waits there, every
     * round, for all but the last few loads in flight */
    __builtin_amdgcn_s_waitcnt(0x0F70);
    f32x16 dd[2];
    dd[0] = products(st[0]);
    for (int k0 = 0; k0 < nch; k0 += XAM_D) { /* whole rounds: chunks past the last add into the spare row */
#pragma unroll
      for (int d = 0; d < XAM_D; ++d) {
        add(dd[d & 1], st[d]);
        dd[(d + 1) & 1] = products(st[(d + 1) % XAM_D]);
        lds_barrier();
        issue(k0 + d + XAM_D, st[d]);
      }
    }
  }
  lds_barrier();
  for (int t = 0; t < nt; ++t) {
    f32x4 *dst = (f32x4 *)p.xd + (((size_t)m * p.mtiles + tl[t]) * p.RB + r0) * MT * 256;
    for (int w = tid; w < MT * 256; w += 256) {
      const int mt = w >> 8, q = (w >> 6) & 3, l = w & 63;
      const int row = t * BM + mt * 32 + 8 * q + 4 * (l >> 5);
      const float *src = accs + row * 32 + (l & 31);
      dst[w] = f32x4{src[0], src[32], src[64], src[96]};
    }
  }
}

/* Row r's user of a chunk, staged in LDS for the stores: SA row p, its tile's union size, slot u,
 * coefficient. */
struct AmUser {
  uint32_t p, tu, u;
  float cf;
  uint32_t ci; /* row of the compact copy (~0: none) */
};

__device__ __forceinline__ void am_users(const aos_amshrink_params &p, const uint32_t *ul, int nu, AmUser *meta,
                                         int tid) {
  if (tid < nu) {
    const uint32_t w = ul[tid];
    const uint32_t pp = w >> 16, u = w & 0xffffu;
    const uint32_t tu = (uint32_t)p.tu[pp / BM];
    const bool cp = p.SAc && p.xam_tu > 0 && tu >= (uint32_t)p.xam_tu;
    meta[tid] = AmUser{pp, tu, u, p.coef[(size_t)pp * p.tu_cap + u], cp ? p.cidx[ul - p.users + tid] : ~0u};
  }
}

/* Module of adapter column col (modules in order, rpad_i columns each): its index, the column
 * within it and the sum of the rpad of the modules before it. */
__device__ __forceinline__ void am_module(const aos_amshrink_params &p, int col, int &mi, int &j, int &rbefore) {
  mi = 0;
  rbefore = 0;
  while (mi < p.nmod - 1 && col >= rbefore + p.rpad[mi]) {
    rbefore += p.rpad[mi];
    ++mi;
  }
  j = col - rbefore;
}

/* Workgroup of NW waves (K slice kz, chunk c, column set cs of 32 NW adapter columns), kz fastest;
 * wave w takes the 32 columns cs * 32 NW + 32 w .., all the chunk's users (four 32-row sub-tiles):
 * the tile shrink's K loop over the users' gathered rows, staged by all 64 NW threads. Waves
 * without columns only stage rows. Adapters of 64 columns or fewer run 2-wave workgroups, four
 * per CU, so that every wave has matrix work and twice the chunks per CU have loads in flight.
 * (Two waves per 32-column block, each on half the rows, was slower: 343 against 275 us for the
 * rank-64 down shrink at 4096 tokens; both load the block's A rows.) */
template <int NW>
__global__ void __launch_bounds__(64 * NW) aos_amshrink_kernel(aos_amshrink_params p) {
  constexpr int MT = BM / 32, TILE = BM * 128, NT = 64 * NW;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, c = lane >> 5;
  const int kz = blockIdx.x, ch = blockIdx.y, cs = blockIdx.z;
  const uint32_t ct = __builtin_amdgcn_readfirstlane(p.ctab[ch]);
  const int nu = (int)(ct & 255u);
  if (nu == 0) return;
  const int a = (int)(ct >> 16), jc = (int)((ct >> 8) & 255u);
  const uint32_t *ul = p.users + (size_t)a * p.T + jc * BM;
  int CW = 0;
  for (int m = 0; m < p.nmod; ++m) CW += p.rpad[m];
  const int G = p.in / 64;
  const int g_lo = (int)((long)kz * G / p.ks), g_hi = (int)((long)(kz + 1) * G / p.ks);

  const int col = cs * 32 * NW + 32 * wave + i;
  const bool wact = cs * 32 * NW + 32 * wave < CW; /* wave-uniform: the wave has columns */
  int mi = 0, jj = 0, rbefore = 0;
  const uint16_t *arow = p.zero_row;
  size_t kstep = 0;
  if (col < CW) {
    am_module(p, col, mi, jj, rbefore);
    const uint16_t *A = p.A[mi][a];
    if (A) {
      arow = A + (size_t)jj * p.in;
      kstep = 1;
    }
  }
  auto aload = [&](int g, u32x4 (&av)[4]) {
    const int gc = g < g_hi ? g : g_hi - 1;
#pragma unroll
    for (int s = 0; s < 4; ++s) av[s] = aos_gld16(arow + kstep * ((size_t)gc * 64 + 16 * s + 8 * c));
  };

  f32x16 acc[MT];
#pragma unroll
  for (int s = 0; s < MT; ++s) acc[s] = f32x16{};
  if (g_lo < g_hi) {
    Stager<NT> st0, st1;
#pragma unroll
    for (int k = 0; k < Stager<NT>::CH; ++k) {
      const int idx = tid + k * NT;
      const int r = idx >> 3, chk = idx & 7;
      const int pp = (int)(ul[r < nu ? r : nu - 1] >> 16);
      const int tok = p.perm ? (int)p.perm[pp] : pp;
      st0.off[k] = tok * p.in + chk * 8;
      st1.off[k] = st0.off[k];
    }
    u32x4 a0[4], a1[4];
    st0.load(p.x, g_lo);
    st1.load(p.x, g_lo + 1 < g_hi ? g_lo + 1 : g_hi - 1);
    aload(g_lo, a0);
    aload(g_lo + 1, a1);
    st0.store(smem, tid);
    lds_barrier();
    auto step = [&](int g, Stager<NT> &hold, Stager<NT> &ld, u32x4 (&av)[4]) {
      const unsigned char *tb = smem + ((g - g_lo) & 1) * TILE;
      ld.load(p.x, g + 2 < g_hi ? g + 2 : g_hi - 1);
      if (wact) {
#pragma unroll
        for (int s = 0; s < MT; ++s) {
          const int r = s * 32 + i;
          u32x4 xv[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) xv[k] = *(const u32x4 *)(tb + tile_off(r, 2 * k + c));
#pragma unroll
          for (int k = 0; k < 4; ++k) acc[s] = aos_mfma32(xv[k], av[k], acc[s]);
        }
      }
      aload(g + 2, av);
      hold.store(smem + (((g - g_lo) & 1) ^ 1) * TILE, tid);
      lds_barrier();
    };
    int g = g_lo;
    for (; g + 1 < g_hi; g += 2) {
      step(g, st1, st0, a0);
      step(g + 1, st0, st1, a1);
    }
    if (g < g_hi) step(g, st1, st0, a0);
  }

  if (p.ks > 1) {
    /* this slice's partial sums, [row][128 columns] */
    if (col < CW) {
      float *dst = p.part + (((size_t)kz * p.cb + ch) * p.csets + cs) * BM * 128 + (col - cs * 32 * NW);
#pragma unroll
      for (int s = 0; s < MT; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = s * 32 + 8 * q + 4 * c + e;
            if (r < nu) dst[(size_t)r * 128] = acc[s][4 * q + e];
          }
    }
    return;
  }
  /* one slice: SA directly (the tile buffers are free past the K loop's last barrier) */
  AmUser *meta = (AmUser *)smem;
  __syncthreads();
  am_users(p, ul, nu, meta, tid);
  __syncthreads();
  if (col < CW) {
    const int rp = p.rpad[mi];
#pragma unroll
    for (int s = 0; s < MT; ++s)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = s * 32 + 8 * q + 4 * c + e;
          if (r < nu) {
            const AmUser m = meta[r];
            const uint16_t v = aos_f32_to_bf16(m.cf * acc[s][4 * q + e]);
            p.SA[(size_t)m.p * p.s_stride + m.tu * rbefore + m.u * rp + jj] = v;
            if (m.ci != ~0u) p.SAc[(size_t)m.ci * CW + col] = v;
          }
        }
  }
}

/* Workgroup (chunk c, column set cs): sums the slices' partials in slice order, four columns of
 * one row per thread step, and stores SA = bf16(coef * sum). */
__global__ void __launch_bounds__(256) aos_amreduce_kernel(aos_amshrink_params p) {
  __shared__ AmUser meta[BM];
  const int tid = threadIdx.x, ch = blockIdx.x, cs = blockIdx.y;
  const uint32_t ct = __builtin_amdgcn_readfirstlane(p.ctab[ch]);
  const int nu = (int)(ct & 255u);
  if (nu == 0) return;
  const int a = (int)(ct >> 16), jc = (int)((ct >> 8) & 255u);
  am_users(p, p.users + (size_t)a * p.T + jc * BM, nu, meta, tid);
  __syncthreads();
  int CW = 0;
  for (int m = 0; m < p.nmod; ++m) CW += p.rpad[m];
  const int cn = CW - cs * p.setw < p.setw ? CW - cs * p.setw : p.setw;
  const int ncg = cn / 4; /* rpad_i are multiples of 16: a group of 4 columns lies in one module */
  const size_t slab = (size_t)p.cb * p.csets * BM * 128;
  const float *src = p.part + ((size_t)ch * p.csets + cs) * BM * 128;
  for (int e = tid; e < nu * ncg; e += 256) {
    const int r = e / ncg, cg = e - r * ncg;
    const float *s0 = src + (size_t)r * 128 + cg * 4;
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < p.ks; k0 += 4) {
      f32x4 v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int kk = k0 + k < p.ks ? k0 + k : p.ks - 1;
        v[k] = *(const f32x4 *)(s0 + (size_t)kk * slab);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k0 + k < p.ks) sum += v[k];
    }
    int mi, jj, rbefore;
    am_module(p, cs * p.setw + cg * 4, mi, jj, rbefore);
    const AmUser m = meta[r];
    u32x2 o;
    o.x = (uint32_t)aos_f32_to_bf16(m.cf * sum[0]) | ((uint32_t)aos_f32_to_bf16(m.cf * sum[1]) << 16);
    o.y = (uint32_t)aos_f32_to_bf16(m.cf * sum[2]) | ((uint32_t)aos_f32_to_bf16(m.cf * sum[3]) << 16);
    *(u32x2 *)(p.SA + (size_t)m.p * p.s_stride + m.tu * rbefore + m.u * p.rpad[mi] + jj) = o;
    if (m.ci != ~0u) *(u32x2 *)(p.SAc + (size_t)m.ci * CW + cs * p.setw + cg * 4) = o;
  }
}

/* ------------------------------------------------------------------------------------------ */
/* int4 GEMM + LoRA expand (+ SwiGLU)                                                          */
/* ------------------------------------------------------------------------------------------ */

/* Expand K steps: the LoRA expand of a token tile runs as extra K steps of 64 union columns after
 * the weight groups: module 0's ceil(TU * rpad0 / 64) steps, then module 1's (SwiGLU). The token
 * operand is the tile's SA columns (coefficient-scaled shrink), the weight operand the union
 * adapters' B rows (bf16). LDS after the token tiles: 16 bytes of flags (word 0: the stream-K
 * owner's "every partial arrived"), then up to LBP B pointers per module (loaded at kernel start
 * while the tile union is small enough). The GEMM kernels declare no static LDS: their dynamic
 * area then starts at LDS address 0, where the token-tile DMA (M0-based) and the reads agree. */
constexpr int LBP = 256;
__host__ __device__ constexpr int gemm_aux() { return 16 + 2 * LBP * 8; }

/* Workgroup b of a grid of mb token tiles x nb weight blocks -> (token tile, weight block).
 * Workgroup b runs on XCD b % 8. With a multiple of 8 token tiles each XCD takes its own token
 * tiles against every weight block (its L2 keeps those token rows while the weights stream):
 * XCD x the tiles x, x + 8, x + 16, ..., so that a run of consecutive tiles with large adapter
 * unions (the grouped order puts the tokens of rare adapter sets last) spreads over the XCDs
 * instead of landing on one; otherwise each XCD takes a contiguous range of tiles (token tile
 * fastest), so a weight block's token tiles share its L2. */
__device__ __forceinline__ void gemm_tile_of(int b, int mb, int nb, int &mbi, int &nbk) {
  if (mb % 8 == 0) {
    const int mpx = mb / 8, k = b >> 3;
    mbi = (k % mpx) * 8 + (b & 7);
    nbk = k / mpx;
  } else {
    const int nt = mb * nb;
    int tile = b;
    if (nt % 8 == 0) tile = (b & 7) * (nt / 8) + (b >> 3);
    mbi = tile % mb;
    nbk = tile / mb;
  }
}

/* The expand steps of one token tile (WV waves, NM modules). Each lane's B fragment word w of a
 * step holds union columns k = 64 j + koff[w] .. +7 of the lane's weight row:
 * B_{list[u]}[row][k - u * rpad .. +7] with u = k / rpad (read from the fragment-order copy, where
 * the 32 rows of a wave's word are contiguous), zeros past the union or for an adapter
 * without the module (rpad is a multiple of 16, so 8 columns never straddle two slots). Words
 * w and w + 1 share a slot when NW / NP = 2 (koff 16-aligned for w even). */
template <int WV, int NM, int NW, int NP>
struct Expand {
  static constexpr int TILE = BM * 128;
  const aos_gemm_params &p;
  unsigned char *smem;
  const uint16_t **lbp;
  const uint16_t *const *bpt[2];
  int wave, lane, m0, mbi, row, TU, n0, nls, off[2], rp[2];
  bool bp_lds;
  /* parameters the steps read, held in registers: a read of the kernel's arguments after an
   * asm statement with a memory clobber (the waits, the barriers) is a scalar load again, and its
   * wait also waits for the LDS reads in flight */
  const uint16_t *zero;
  int sa_stride, nbs;

  /* row: the lane's weight row (of every module) */
  __device__ Expand(const aos_gemm_params &p_, unsigned char *smem_, int ntile, int wave_, int lane_, int m0_,
                    int mbi_, int row_)
      : p(p_), smem(smem_), wave(wave_), lane(lane_), m0(m0_), mbi(mbi_), row(row_) {
    zero = p.zero;
    sa_stride = p.sa_stride;
    nbs = p.nbs;
    lbp = (const uint16_t **)(smem + ntile * TILE + 16);
    TU = (p.tu && (p.rpad0 | (NM == 2 ? p.rpad1 : 0))) ? __builtin_amdgcn_readfirstlane(p.tu[mbi]) : 0;
    rp[0] = p.rpad0;
    rp[1] = NM == 2 ? p.rpad1 : 0;
    int before = 0;
    for (int i = 0; i < p.sa_mod_before; ++i) before += TU * p.rpad_before[i];
    off[0] = before;
    off[1] = before + TU * rp[0];
    n0 = rp[0] ? (TU * rp[0] + 63) >> 6 : 0;
    nls = n0 + (rp[1] ? (TU * rp[1] + 63) >> 6 : 0);
#pragma unroll
    for (int m = 0; m < 2; ++m) bpt[m] = p.bp + ((size_t)(p.mod0 + m) * p.mtiles + mbi) * p.tu_cap;
    bp_lds = TU <= LBP;
  }

  /* At kernel start: the union's B pointers go straight to LDS; their loads complete during the
   * K loop. */
  __device__ void prefetch() {
    if (nls == 0 || !bp_lds) return;
    constexpr int NT = 64 * WV;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      if (!rp[m]) continue;
      const __amdgpu_buffer_rsrc_t rb =
          __builtin_amdgcn_make_buffer_rsrc((void *)bpt[m], (short)0, TU * 8, 0x00020000);
      for (int d0 = wave * 64; d0 < 2 * TU; d0 += NT)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb, (__attribute__((address_space(3))) void *)((uint32_t *)(lbp + m * LBP) + d0), 4,
            (d0 + lane) * 4, 0, 0, 0);
    }
  }

  __device__ __forceinline__ void step_of(int l, int &m, int &j) const {
    l = l < nls ? l : nls - 1;
    m = l < n0 ? 0 : 1;
    j = l - (m ? n0 : 0);
  }

  /* Runs the nls steps. With the union's B pointers in LDS: pipelined over the NT token-tile
   * stages, as the weight groups are: step l's token tile (its SA columns, through a buffer resource
   * over the tile's rows; columns past the union read as zeros) goes straight from memory to stage
   * l % NT, NT - 1 steps ahead of its use, its B fragments to a register ring NT - 1 deep, and each
   * step waits only for its own loads (a counted vmcnt: steps past the last re-load the last
   * step's operands, so that the count holds to the end), one pipeline per module. mma1(mc, tile,
   * bv) adds one step of module mc (a std::integral_constant). Otherwise in chunks of LC steps within one module with one wait per chunk, the next
   * chunk's B pointers loading meanwhile: mma(m, n, bv) adds the chunk's n steps of module m (token
   * tile q at smem + q * TILE). */
  template <int LC, int NT, class Mma, class Mma1>
  __device__ void run(const int (&koff)[NW], Mma &&mma, Mma1 &&mma1) {
    if (nls == 0) return;
    if (p.nbs && threadIdx.x == 0) { /* SA comes from this launch's shrink workgroups */
      if (!aos_wait_gen(p.sa_lines + (size_t)mbi * 32, p.gen) && p.timeout)
        __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier(); /* the prefetched pointers, the tile's SA line, and every wave past the K loop's
                    * last LDS reads */
    const int rows = p.T - m0 < BM ? p.T - m0 : BM;
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.SA + (size_t)m0 * p.sa_stride), (short)0, rows * p.sa_stride * 2, 0x00020000);
    auto load_ptrs = [&](int l, const uint16_t *(&pr)[NP]) {
      int m, j;
      step_of(l, m, j);
#pragma unroll
      for (int h = 0; h < NP; ++h) {
        int u = (64 * j + koff[h * (NW / NP)]) / rp[m];
        u = u < TU ? u : TU - 1;
        /* two explicit loads (LDS, global) and a select of the value: a select of the two
         * addresses would make one generic load */
        const uint16_t *from_lds =
            (const uint16_t *)((const __attribute__((address_space(3))) uint64_t *)lbp)[m * LBP + (u < LBP ? u : 0)];
        pr[h] = bp_lds ? from_lds : aos_gld_ptr(bpt[m] + u);
      }
    };
    auto load_frags = [&](int l, const uint16_t *const (&pr)[NP], u32x4 (&bv)[NW]) {
      int m, j;
      step_of(l, m, j);
      const int r = rp[m];
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const uint16_t *b = pr[w / (NW / NP)];
        const int k = 64 * j + koff[w];
        const int u = k / r;
        /* B in fragment order: the 8 columns of 32 consecutive rows are 512 contiguous bytes */
        const uint16_t *src =
            (u < TU && b) ? b + ((size_t)(row >> 5) * (r >> 3) + ((k - u * r) >> 3)) * 256 + (row & 31) * 8 : zero;
        bv[w] = aos_gld16(src);
      }
    };
    /* token tile of step l into LDS region q: BM / 8 blocks of 8 rows (1 KB), lane l of a block
     * writing bytes 16 l, i.e. row 8 b + l / 8, slot l % 8, which holds chunk slot ^ ((r >> 1) & 7) */
    auto dma_tile = [&](int q, int l) {
      int m, j;
      step_of(l, m, j);
      const int cb = (off[m] + 64 * j) * 2, lim = (off[m] + TU * rp[m]) * 2, rb = sa_stride * 2;
#pragma unroll
      for (int k = 0; k < BM / 8 / WV; ++k) {
        const int bk = k * WV + wave;
        const int r = bk * 8 + (lane >> 3);
        const int ch = (lane & 7) ^ ((r >> 1) & 7);
        const int rr = r < rows ? r : rows - 1;
        const int col = cb + ch * 16;
        const int vo = col < lim ? rr * rb + col : (int)0x80000000;
        /* SA stored in this launch (by a workgroup maybe on another XCD): device-coherent (sc1) */
        if (nbs)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rsa, (__attribute__((address_space(3))) void *)(smem + q * TILE + bk * 1024), 16, vo, 0, 0, SC1);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rsa, (__attribute__((address_space(3))) void *)(smem + q * TILE + bk * 1024), 16, vo, 0, 0, 0);
      }
    };
    if constexpr (NT >= 3) if (bp_lds) {
      constexpr int VMS = BM / 8 / WV + NW; /* memory instructions a wave issues per step */
      /* one pipeline per module (its steps lo .. hi - 1), the module a constant in each */
      auto pipe = [&](auto mc, int lo, int hi) {
        if (lo >= hi) return;
        u32x4 bq[NT - 1][NW];
        const uint16_t *pq[NP];
#pragma unroll
        for (int k = 0; k < NT - 1; ++k) {
          dma_tile(k, lo + k);
          load_ptrs(lo + k, pq);
          load_frags(lo + k, pq, bq[k]);
        }
        for (int base = 0; base < hi - lo; base += NT - 1) {
#pragma unroll
          for (int d = 0; d < NT - 1; ++d) {
            const int k = base + d;
            if (k < hi - lo) {
              /* step k's tile and fragments are in (this wave's loads, then every wave's after
               * the barrier); every wave is past its reads of step k - 1's stage, refilled next */
              asm volatile("s_waitcnt vmcnt(%0)" ::"n"(VMS * (NT - 2)) : "memory");
              lds_barrier();
              const int kn = k + NT - 1;
              dma_tile(kn % NT, lo + kn);
              load_ptrs(lo + kn, pq);
              mma1(mc, smem + (k % NT) * TILE, bq[d]);
              load_frags(lo + kn, pq, bq[d]);
            }
          }
        }
        /* the loads past the last step land before the LDS is used again */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
      };
      pipe(std::integral_constant<int, 0>{}, 0, n0);
      if (NM > 1) pipe(std::integral_constant<int, 1>{}, n0, nls);
      return;
    }
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

/* Single-matrix kernel (and SwiGLU) on v_mfma_f32_32x32x16_bf16.
 * SW: SwiGLU (gate and up rows of one 32-row block per wave) or a single matrix (one 32-row
 * block per wave); D: weight ring depth (divides the group count); DB: token tile loads two groups
 * ahead (two register stages); APF: next sub-tile's LDS fragments loaded before the current
 * MFMAs; WV: waves per workgroup; OCC: waves per SIMD the registers are sized for; LC: expand
 * steps per chunk (their token tiles occupy LC LDS regions); NS: 0, or the token tiles go straight
 * from memory to an NS-stage LDS ring, NS - 1 groups ahead of their use (no staging registers). */
template <int NS, int LC>
__host__ __device__ constexpr int gemm_ntile() { return NS > (LC > 2 ? LC : 2) ? NS : (LC > 2 ? LC : 2); }

/* Group gx of a token tile straight to LDS (the DMA of the NS-stage ring): the wave's n (<= 4)
 * blocks of 8 rows, block k at stage + (k * wv + wave) * 1024; v[k] is the lane's byte offset in x
 * of its chunk in group 0. A device function of its own, not a template: the buffer resource type
 * exists only on the device, and the kernel's lambdas are compiled for the host as well. */
__device__ __forceinline__ void tile_dma(const uint16_t *x, int T, int in, unsigned char *stage, int wave, int wv,
                                         int n, int v0, int v1, int v2, int v3, int gx) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, T * in * 2, 0x00020000);
  const int v[4] = {v0, v1, v2, v3};
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (k < n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void *)(stage + (k * wv + wave) * 1024), 16, v[k], gx * 128, 0, 0);
}

/* Wait until at most n of this wave's memory instructions are outstanding (n a constant). */
#define AOS_VM_WAIT_LE(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")

/* Shrink workgroup sb of token tile mbi (a GEMM launch's first workgroups): for module
 * m = sb % nmg of the nmg modules the launch's expand consumes (SwiGLU: gate, up), S = x . A^T over
 * the tile's union columns c = 32 WV (sb / nmg) + 32 w + i (wave w, lane i % 32), with the token
 * tiles through the same NS-stage LDS ring as the GEMM workgroups and the A rows (bf16) as the
 * weight operand through a 4-deep register ring; then SA[p][off_m + c] = bf16(coef[p][u] * S)
 * with u = c / rpad_m, stored device-coherently, and an arrival on the tile's counter: the last of
 * the tile's nbs workgroups raises its line. A workgroup whose columns are all past the tile's
 * union only arrives. Column c reads union slot u = c / rpad, row c - u * rpad of its A (zeros for
 * an adapter without the module). */
template <int WV, int NS>
__device__ __forceinline__ void tile_shrink_rows(const aos_gemm_params &p, unsigned char *smem, int mbi, int sb,
                                                 int nmg, int wave, int lane) {
  constexpr int MT = BM / 32, TILE = BM * 128, DMA_N = BM / 8 / WV, D = 4;
  const int i = lane & 31, c = lane >> 5;
  const int m0 = mbi * BM, G = p.w0.G, in = p.w0.in;
  const int tn = p.T - m0 < BM ? p.T - m0 : BM;
  const int TU = __builtin_amdgcn_readfirstlane(p.tu[mbi]);
  const int m = sb % nmg, cb = sb / nmg;
  const int rp = m == 0 ? p.rpad0 : p.rpad1;
  int off = m == 0 ? 0 : TU * p.rpad0;
  for (int k = 0; k < p.sa_mod_before; ++k) off += TU * p.rpad_before[k];
  const int C = TU * rp;
  const int col = cb * 32 * WV + 32 * wave + i;
  if (cb * 32 * WV < C) { /* uniform */
    const uint16_t *arow = p.zero;
    size_t kst = 0;
    if (col < C) {
      const int u = col / rp, j = col - u * rp;
      const uint16_t *A = aos_gld_ptr(p.ap + ((size_t)(p.mod0 + m) * p.mtiles + mbi) * p.tu_cap + u);
      if (A) {
        arow = A + (size_t)j * in;
        kst = 1;
      }
    }
    /* word s of lane (i, c): K elements 32 c + 8 s .. +7 of group g (the GEMM's fragment layout) */
    auto bload = [&](int g, u32x4 (&b)[4]) {
      const int gc = g < G ? g : G - 1;
#pragma unroll
      for (int s = 0; s < 4; ++s) b[s] = aos_gld16(arow + kst * ((size_t)gc * 64 + 32 * c + 8 * s));
    };
    int voff[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < DMA_N; ++k) {
      const int r = (k * WV + wave) * 8 + (lane >> 3);
      const int ch = (lane & 7) ^ ((r >> 1) & 7);
      const int ps = m0 + r < p.T ? m0 + r : p.T - 1;
      const int tok = p.in_perm ? (int)p.in_perm[ps] : ps;
      voff[k] = (tok * in + ch * 8) * 2;
    }
    auto dma = [&](int stage, int gx) {
      tile_dma(p.x, p.T, in, smem + stage * TILE, wave, WV, DMA_N, voff[0], voff[1], voff[2], voff[3],
               gx < G ? gx : G - 1);
    };
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) dma(s, s);
    u32x4 b[D][4];
#pragma unroll
    for (int d = 0; d < D; ++d) bload(d, b[d]);
    /* the prologue's tiles are complete: the counted wait below covers the later ones */
    AOS_VM_WAIT_LE(0);
    /* memory instructions per group: the DMA of a tile, then the A rows of the group D ahead. At
     * the top of group g >= NS - 1 the DMA of tile g was issued NS - 1 groups earlier and followed
     * by that group's A loads and NS - 2 full groups: at most VM_AFTER outstanding means it is
     * complete */
    constexpr int VM_AFTER = 4 + (NS - 2) * (DMA_N + 4);
    f32x16 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x16{};
    /* group g: tile g is in LDS once each wave's DMA of it is complete and all have passed the
     * barrier, which also puts every wave past its reads of the stage the next DMA refills */
    auto grp = [&](int g, u32x4 (&bb)[4]) {
      AOS_VM_WAIT_LE(VM_AFTER);
      ring_barrier();
      dma((g + NS - 1) % NS, g + NS - 1);
      const unsigned char *tb = smem + (g % NS) * TILE;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 a[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = *(const u32x4 *)(tb + tile_off(mt * 32 + i, 4 * c + s));
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[mt] = aos_mfma32(a[s], bb[s], acc[mt]);
      }
      bload(g + D, bb);
    };
    for (int g = 0; g < G; g += D) {
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (g + d < G) grp(g + d, b[d]);
    }
    aos_mem_wait(); /* the rings' trailing loads (past the last group) land before the workgroup ends */
    if (col < C) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(p.sa_out + (size_t)m0 * p.sa_stride), (short)0, tn * p.sa_stride * 2, 0x00020000);
      const int u = col / rp;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = mt * 32 + aos_acc_m(v, lane);
          if (r >= tn) continue;
          const float cf = p.coef[(size_t)(m0 + r) * p.tu_cap + u];
          __builtin_amdgcn_raw_buffer_store_b16(aos_f32_to_bf16(cf * acc[mt][v]), rs,
                                                (r * p.sa_stride + off + col) * 2, 0, SC1);
        }
    }
  }
  aos_mem_wait();
  __syncthreads();
  if (threadIdx.x == 0 && aos_arrive(p.sa_ctr + mbi) == (uint32_t)p.nbs - 1u) {
    aos_reset(p.sa_ctr + mbi);
    aos_raise(p.sa_lines + (size_t)mbi * 32, p.gen);
  }
}

/* Roles of a piece [ga, gb) of a task's K groups: the whole task; the owner of a task split over
 * workgroups (it holds group 0, adds the other pieces' partial sums, then runs the expand and the
 * epilogue); a partial piece (its sums go to the workspace for the owner). */
enum { GEMM_WHOLE = 0, GEMM_OWNER = 1, GEMM_PART = 2 };

/* Stream-K: the task's pieces after the owner's, which hold its partial sums, and where they go. */
struct SkCtx {
  uint32_t v;          /* this workgroup's slot (its place in the launch's iteration order) */
  uint32_t v_first;    /* owner: first contributing slot (v + 1) */
  uint32_t v_last;     /* owner: last contributing slot */
};

/* One task (token tile mbi, weight block nbk) over K groups [ga, gb). */
template <bool SW, int D, bool DBT, bool APF, int WV, int OCC, int LC, int NS>
__device__ __forceinline__ void gemm_task(const aos_gemm_params &p, unsigned char *smem, int mbi, int nbk, int ga,
                                          int gb, int role, const SkCtx &sk) {
  constexpr int MT = BM / 32;
  constexpr int TILE = BM * 128;
  constexpr int NT = 64 * WV;
  constexpr int NTILE = gemm_ntile<NS, LC>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, c = lane >> 5;
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
  const int glast = gb - 1; /* groups past the piece are clamped to its last (never read) */

  f32x16 acc0[MT], acc1[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc0[mt] = f32x16{};
    acc1[mt] = f32x16{};
  }

  /* prologue: weight ring D groups deep (slot d holds group ga + d, ga + d + D, ...), first
   * token tile */
  u32x4 wq0[D], wq1[D];
  uint32_t ws0[D], ws1[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int gd = ga + d < gb ? ga + d : glast;
    wq0[d] = q0[(size_t)gd * 64];
    ws0[d] = s0p[(size_t)gd * 32];
    if (SW) {
      wq1[d] = q1[(size_t)gd * 64];
      ws1[d] = s1p[(size_t)gd * 32];
    }
  }
  /* Token tiles, NS == 0: LDS holds groups g and g + 1 (double buffer); registers hold the loads
   * in flight. With D even, two register stages let the loads run two groups ahead of their LDS
   * store. NS > 0: tile g goes straight to LDS stage g % NS: block k of 8 rows (1 KB) by wave
   * k % WV, lane l writing bytes 16 l (row 8 k + l / 8, slot l % 8, which holds chunk
   * slot ^ ((row >> 1) & 7): the layout tile_off reads). */
  constexpr bool DB = NS == 0 && DBT && (D % 2) == 0;
  constexpr int DMA_N = BM / 8 / WV; /* 1 KB blocks per wave per tile */
  static_assert(NS == 0 || DMA_N <= 4, "tile DMA: at most 4 blocks per wave");
  Stager<NT> st0, st1;
  int voff[4] = {0, 0, 0, 0};
  const uint16_t *const xg = p.x; /* in registers: see Expand */
  const int Tg = p.T;
  auto dma = [&](int stage, int gx) {
    /* tiles past the piece's last group repeat it and are never read */
    tile_dma(xg, Tg, in, smem + stage * TILE, wave, WV, DMA_N, voff[0], voff[1], voff[2], voff[3],
             gx < gb ? gx : glast);
  };
  if (NS) {
#pragma unroll
    for (int k = 0; k < DMA_N; ++k) {
      const int r = (k * WV + wave) * 8 + (lane >> 3);
      const int ch = (lane & 7) ^ ((r >> 1) & 7);
      const int ps = m0 + r < p.T ? m0 + r : p.T - 1;
      const int tok = p.in_perm ? (int)p.in_perm[ps] : ps;
      voff[k] = (tok * in + ch * 8) * 2;
    }
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) dma((ga + s) % (NS ? NS : 1), ga + s);
  } else {
    st0.rows(p.in_perm, in, p.T, m0, tid);
    st0.load(p.x, ga);
    if (DB) {
#pragma unroll
      for (int k = 0; k < Stager<NT>::CH; ++k) st1.off[k] = st0.off[k];
    }
  }
  const bool expand = role != GEMM_PART;
  Expand<WV, SW ? 2 : 1, 4, 2> ex(p, smem, NTILE, wave, lane, m0, mbi, row);
  /* a tile whose expand ran in the expand launch: its sums are added in the epilogue */
  const bool xe = SW && p.xd && ex.TU * (p.rpad0 > p.rpad1 ? p.rpad0 : p.rpad1) >= p.xe_cols;
  if (xe) ex.nls = 0;
  if (expand) ex.prefetch();
  if (!NS) {
    st0.store(smem + (ga & 1) * TILE, tid);
    lds_barrier();
  }

  /* token tile of weight group gx (clamped: the tiles staged past the piece are not read) */
  auto stage = [&](Stager<NT> &st, const int gx) { st.load(p.x, gx < gb ? gx : glast); };
  if (DB) stage(st1, ga + 1);
  /* NS > 0: memory instructions a wave issues per group (the tile's DMA, then the ring refill);
   * waiting until no more than VM_AFTER are outstanding completes the DMA issued NS - 1 groups
   * earlier (at least that many were issued after it) */
  constexpr int VM_AFTER = NS >= 2 ? (DMA_N + (SW ? 4 : 2)) * (NS - 2) : 0;

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
    const int gc = gn < gb ? gn : glast;
    wq0[d] = q0[(size_t)gc * 64];
    ws0[d] = s0p[(size_t)gc * 32];
    if (SW) {
      wq1[d] = q1[(size_t)gc * 64];
      ws1[d] = s1p[(size_t)gc * 32];
    }
  };

  /* one K group: ld receives group g + 2 (g + 1 without DB), sto holds group g + 1 */
  auto group = [&](const int g, const int d, Stager<NT> &ld, Stager<NT> &sto) {
    if (NS) { /* tile g is in LDS once this wave's DMA of it completes and every wave has waited;
               * the piece's first group waits for every load (fewer than VM_AFTER may follow its
               * tile's DMA there) */
      if (g == ga)
        AOS_VM_WAIT_LE(0);
      else
        AOS_VM_WAIT_LE(VM_AFTER);
      lds_barrier(); /* also: every wave is past its reads of the stage refilled next */
      dma((g + NS - 1) % (NS ? NS : 1), g + NS - 1);
    }
    const unsigned char *tb = smem + (NS ? (g % (NS ? NS : 1)) : (g & 1)) * TILE;
    /* token fragments of the first sub-tile: their LDS latency overlaps the dequantisation */
    u32x4 a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = *(const u32x4 *)(tb + tile_off(i, 4 * c + s));
    if (!NS) stage(ld, g + (DB ? 2 : 1));
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
    if (!NS) {
      sto.store(smem + ((g & 1) ^ 1) * TILE, tid);
      lds_barrier();
    }
  };

  for (int g0 = ga; g0 < gb; g0 += D) {
    if (DB) {
#pragma unroll
      for (int d = 0; d < D; d += 2) {
        if (g0 + d < gb) group(g0 + d, d, st0, st1);
        if (g0 + d + 1 < gb) group(g0 + d + 1, d + 1, st1, st0);
      }
    } else {
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (g0 + d < gb) group(g0 + d, d, st0, st0);
    }
  }
  constexpr int NMAT = SW ? 2 : 1;
  if (role != GEMM_WHOLE) {
    /* the pieces meet through the workspace: slot v holds [WV waves][NMAT][MT][4 quads][64 lanes]
     * 16-byte words, stored and loaded device-coherently (the slots' workgroups sit on other XCDs) */
    constexpr int PW = NMAT * MT * 4; /* 16-byte words per lane per wave */
    const size_t slot_words = (size_t)WV * PW * 64;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.sk_part, (short)0, 0x7fffffff, 0x00020000);
    if (role == GEMM_PART) {
      const uint32_t base = (uint32_t)(sk.v * slot_words + (size_t)wave * PW * 64 + lane) * 16u;
#pragma unroll
      for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x16 &a = m ? acc1[mt] : acc0[mt];
            f32x4 w4 = {a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, w4), rs,
                                                   base + (uint32_t)(((m * MT + mt) * 4 + q) * 64 * 16), 0, SC1);
          }
      aos_mem_wait();
      __syncthreads();
      if (tid == 0) aos_raise(p.sk_lines + (size_t)sk.v * 32, p.gen);
      return;
    }
    /* owner: the other pieces' sums, in slot order, added to this piece's */
    volatile uint32_t *sk_ok = (volatile uint32_t *)(smem + NTILE * TILE); /* aux word 0 */
    if (tid == 0) {
      bool ok = true;
      for (uint32_t u = sk.v_first; u <= sk.v_last && ok; ++u) ok = aos_wait_gen(p.sk_lines + (size_t)u * 32, p.gen);
      if (!ok && p.timeout) __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      *sk_ok = ok ? 1u : 0u;
    }
    __syncthreads();
    if (*sk_ok) {
      for (uint32_t u = sk.v_first; u <= sk.v_last; ++u) {
        const uint32_t base = (uint32_t)(u * slot_words + (size_t)wave * PW * 64 + lane) * 16u;
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
          /* one matrix's words in flight together, then added; through __builtin_bit_cast: this
           * compiler turns an ext_vector initialised straight from the builtin's result into
           * element 0 for every element (one dword load) */
          f32x4 w4[MT][4];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              w4[mt][q] = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                             rs, base + (uint32_t)(((m * MT + mt) * 4 + q) * 64 * 16), 0, SC1));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            f32x16 &a = m ? acc1[mt] : acc0[mt];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              a[4 * q] += w4[mt][q].x;
              a[4 * q + 1] += w4[mt][q].y;
              a[4 * q + 2] += w4[mt][q].z;
              a[4 * q + 3] += w4[mt][q].w;
            }
          }
        }
      }
    }
  }

  /* LoRA expand over the tile union: word s of lane (i, c) covers step columns 32 c + 8 s .. +7 */
  {
    const int koff[4] = {32 * c, 32 * c + 8, 32 * c + 16, 32 * c + 24};
    auto mma_into = [&](int n, const u32x4 (&bv)[LC][4], f32x16 (&acc)[MT]) {
#pragma unroll
      for (int q = 0; q < LC; ++q) {
        if (q >= n) continue;
        const unsigned char *tb = smem + q * TILE;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          u32x4 a[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) a[mt] = *(const u32x4 *)(tb + tile_off(mt * 32 + i, 4 * c + s));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = aos_mfma32(a[mt], bv[q][s], acc[mt]);
        }
      }
    };
    auto mma_step = [&](const unsigned char *tb, const u32x4 (&bv)[4], f32x16 (&acc)[MT]) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 a[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) a[mt] = *(const u32x4 *)(tb + tile_off(mt * 32 + i, 4 * c + s));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = aos_mfma32(a[mt], bv[s], acc[mt]);
      }
    };
    ex.template run<LC, (SW ? 0 : NTILE)>(
        koff,
        [&](int m, int n, const u32x4 (&bv)[LC][4]) {
          if (!SW || m == 0)
            mma_into(n, bv, acc0);
          else
            mma_into(n, bv, acc1);
        },
        [&](auto mc, const unsigned char *tb, const u32x4 (&bv)[4]) {
          if constexpr (!SW || decltype(mc)::value == 0)
            mma_step(tb, bv, acc0);
          else
            mma_step(tb, bv, acc1);
        });
  }

  /* epilogue: sorted row m0 + r goes to output row out_perm[m0 + r] (or m0 + r) */
  if (!live) return;
  if (SW && xe) { /* the expand launch's gate and up sums, in accumulator order */
    const size_t plane = (size_t)p.mtiles * RB * MT * 256; /* f32x4 words per module */
    const f32x4 *d0 = (const f32x4 *)p.xd + ((size_t)mbi * RB + r0) * MT * 256 + lane;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 g4[4], u4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        g4[q] = d0[(mt * 4 + q) * 64];
        u4[q] = d0[plane + (mt * 4 + q) * 64];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc0[mt][4 * q + e] += g4[q][e];
          acc1[mt][4 * q + e] += u4[q][e];
        }
    }
  }
  const int out = p.w0.out;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int ps = m0 + mt * 32 + aos_acc_m(v, lane);
      if (ps >= p.T) continue;
      const int tok = p.out_perm ? (int)p.out_perm[ps] : ps;
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

template <bool SW, int D, bool DBT, bool APF, int WV, int OCC, int LC, int NS = 0>
__global__ void __launch_bounds__(64 * WV, OCC) aos_gemm_kernel(aos_gemm_params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  /* The launch's first mb * nbs workgroups are shrink workgroups (tile fastest): dispatched before
   * every GEMM workgroup, which waits for them only after its K loop, so none waits on a
   * workgroup that cannot start. */
  const int nsh = p.mb * p.nbs;
  if (NS > 0 && (int)blockIdx.x < nsh) { /* uniform */
    tile_shrink_rows<WV, (NS > 0 ? NS : 2)>(p, smem, blockIdx.x % p.mb, blockIdx.x / p.mb, SW ? 2 : 1, wave, lane);
    return;
  }
  int mbi, nbk;
  gemm_tile_of(blockIdx.x - nsh, p.mb, p.nb, mbi, nbk);
  gemm_task<SW, D, DBT, APF, WV, OCC, LC, NS>(p, smem, mbi, nbk, 0, p.w0.G, GEMM_WHOLE, SkCtx{0u, 0u, 0u});
}

/* Stream-K form of the same GEMM: sk_nwg workgroups (as many as the device holds at once) share
 * the launch's mb * nb tasks x G groups evenly, in an order where a task's groups are consecutive
 * and the tasks run token tile fastest; the slots of one XCD (workgroup w runs on XCD w % 8) take
 * consecutive ranges, so each XCD streams its own share of the weights. A workgroup's range cuts
 * at most its first and last tasks: it hands the first one's sums on (partial) when the task
 * started in an earlier slot, and owns its last one when that continues in later slots (the
 * partial pieces of a range run first, so the owner, which finishes its range with that task,
 * rarely waits). */
template <bool SW, int D, bool DBT, bool APF, int WV, int OCC, int LC, int NS>
__global__ void __launch_bounds__(64 * WV, OCC) aos_gemm_sk_kernel(aos_gemm_params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  static_assert(NS > 0, "stream-K needs the LDS-DMA token tiles");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int nsh = p.mb * p.nbs;
  if ((int)blockIdx.x < nsh) { /* uniform */
    tile_shrink_rows<WV, NS>(p, smem, blockIdx.x % p.mb, blockIdx.x / p.mb, SW ? 2 : 1, wave, lane);
    return;
  }
  const uint32_t nw = (uint32_t)p.sk_nwg, w = blockIdx.x - nsh;
  const uint32_t v = nw % 8 == 0 ? (w & 7u) * (nw / 8) + (w >> 3) : w;
  const uint32_t G = (uint32_t)p.w0.G, total = (uint32_t)(p.mb * p.nb) * G; /* the host keeps total * nw < 2^32 */
  auto slot_lo = [&](uint32_t s) { return s * total / nw; };
  auto slot_of = [&](uint32_t it) { return ((it + 1) * nw - 1) / total; };
  const uint32_t lo = slot_lo(v), hi = slot_lo(v + 1);
  for (uint32_t it = lo; it < hi;) {
    const uint32_t t = it / G, ga = it - t * G;
    const uint32_t gb = hi - it < G - ga ? ga + (hi - it) : G;
    int role = GEMM_WHOLE;
    SkCtx sk{v, v + 1, v};
    if (ga > 0) {
      role = GEMM_PART;
    } else if (gb < G) {
      role = GEMM_OWNER;
      sk.v_last = slot_of(t * G + G - 1);
    }
    if (it > lo) { /* the previous piece's loads (LDS DMA included) are complete before reuse */
      aos_mem_wait();
      __syncthreads();
    }
    gemm_task<SW, D, DBT, APF, WV, OCC, LC, NS>(p, smem, (int)(t % (uint32_t)p.mb), (int)(t / (uint32_t)p.mb), (int)ga,
                                                (int)gb, role, sk);
    it += gb - ga;
  }
}

/* The expand launch of a SwiGLU GEMM (aos_xexp_params): workgroup (module m, token tile mbi,
 * block nbk of XW * 32 rows), the tiles mapped to XCDs as the GEMM's plain grid maps them. Each
 * wave expands its 32 rows of module m over the tile's union with the pipelined expand (token tiles
 * through an LDS ring, B fragments in a register ring) into one accumulator set and stores it in
 * accumulator order. Tiles the GEMM expands itself (tu * rmax < xe_cols) exit at once. Shape: 4-wave
 * workgroups with a 3-stage ring (52 KB of LDS, 162 VGPRs), three per CU; 8-wave workgroups with 4
 * stages (one per CU) and 4-wave ones with 4 stages (two per CU) measured 17% slower on the 32B-shaped
 * stress prefill: the steps wait on their loads, and more resident waves cover more of it. */
constexpr int XW = 4;  /* waves per expand workgroup */
constexpr int XNT = 3; /* LDS ring stages */
__global__ void __launch_bounds__(64 * XW, 3) aos_xexp_kernel(aos_xexp_params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int MT = BM / 32;
  constexpr int TILE = BM * 128;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 31, c = lane >> 5;
  const aos_gemm_params &g0 = p.g[0];
  const int mb = g0.mb, nb = g0.nb, RB = g0.w0.RB;
  const int m = (int)blockIdx.x / (mb * nb);
  int mbi, nbk;
  gemm_tile_of((int)blockIdx.x - m * mb * nb, mb, nb, mbi, nbk);
  const int TU = __builtin_amdgcn_readfirstlane(g0.tu[mbi]);
  if (TU * p.rmax < p.xe_cols) return; /* uniform: the GEMM expands this tile */
  if (p.xam_tu > 0 && TU >= p.xam_tu) return; /* the adapter-major expand's tile */
  const aos_gemm_params &q = p.g[m];
  const int rb = nbk * XW + wave;
  const bool live = rb < RB;
  const int r0 = live ? rb : RB - 1;
  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x16{};
  Expand<XW, 1, 4, 2> ex(q, smem, XNT, wave, lane, mbi * BM, mbi, r0 * 32 + i);
  ex.prefetch();
  const int koff[4] = {32 * c, 32 * c + 8, 32 * c + 16, 32 * c + 24};
  auto mma_step = [&](const unsigned char *tb, const u32x4 (&bv)[4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 a[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) a[mt] = *(const u32x4 *)(tb + tile_off(mt * 32 + i, 4 * c + s));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = aos_mfma32(a[mt], bv[s], acc[mt]);
    }
  };
  ex.template run<XNT, XNT>(
      koff,
      [&](int, int n, const u32x4 (&bv)[XNT][4]) {
#pragma unroll
        for (int k = 0; k < XNT; ++k)
          if (k < n) mma_step(smem + k * TILE, bv[k]);
      },
      [&](auto, const unsigned char *tb, const u32x4 (&bv)[4]) { mma_step(tb, bv); });
  if (!live) return;
  f32x4 *d = (f32x4 *)p.xd + (((size_t)m * g0.mtiles + mbi) * RB + r0) * MT * 256 + lane;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int k = 0; k < 4; ++k)
      d[(mt * 4 + k) * 64] = f32x4{acc[mt][4 * k], acc[mt][4 * k + 1], acc[mt][4 * k + 2], acc[mt][4 * k + 3]};
}

}  // namespace

extern "C" int aos_launch_xexp(const aos_xexp_params *p, const aos_launch_ctx *ctx) {
  aos_xexp_params q = *p;
  const aos_gemm_params &g = q.g[0];
  if (!q.xd || q.xe_cols < 1 || q.rmax < 1 || !g.tu || !g.bp || !g.SA || g.T < 1 || g.T > AOS_PREFILL_MAX_T ||
      g.w0.RB < 1 || q.g[1].w0.RB != g.w0.RB || g.mtiles != (g.T + BM - 1) / BM)
    return (int)hipErrorInvalidValue;
  for (int m = 0; m < 2; ++m) {
    q.g[m].mb = g.mtiles;
    q.g[m].nb = (g.w0.RB + XW - 1) / XW;
    q.g[m].nbs = 0;
  }
  const size_t lds = (size_t)XNT * BM * 128 + gemm_aux();
  AOS_LAUNCH(ctx, aos_xexp_kernel, dim3(2 * q.g[0].mb * q.g[0].nb), dim3(64 * XW), lds, q);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_gplan(const aos_gplan_params *p, const aos_launch_ctx *ctx) {
  const int mtiles = (p->T + BM - 1) / BM;
  if (p->T < 1 || p->T > AOS_PREFILL_MAX_T || p->n > AOS_MAX_ADAPTERS || p->nmod < 0 || p->nmod > 3)
    return (int)hipErrorInvalidValue;
  const int ucap = p->n < AOS_TILE_U_MAX ? p->n : AOS_TILE_U_MAX;
  if (p->tu_cap < ucap || p->tu_cap < 1) return (int)hipErrorInvalidValue;
  AOS_LAUNCH(ctx, aos_gplan_kernel, dim3(mtiles), dim3(GP_NT), GP_LDS, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_tshrink(const aos_tshrink_params *p, const aos_launch_ctx *ctx) {
  if (p->T < 1 || p->T > AOS_PREFILL_MAX_T || p->nmod < 1 || p->nmod > 3 || p->ks < 1 || p->csets < 1 ||
      p->mtiles != (p->T + BM - 1) / BM || p->in % 64 || p->s_stride % 4)
    return (int)hipErrorInvalidValue;
  int cols = 0;
  for (int i = 0; i < p->nmod; ++i) {
    if (p->rpad[i] < 0 || p->rpad[i] % 16) return (int)hipErrorInvalidValue;
    cols += p->tu_cap * p->rpad[i];
  }
  if (cols > p->s_stride || (cols + 127) / 128 > p->csets) return (int)hipErrorInvalidValue;
  if (!p->counters || !p->flags || !p->gen) return (int)hipErrorInvalidValue;
  dim3 grid(p->ks, p->csets, p->mtiles);
  AOS_LAUNCH(ctx, aos_tshrink_kernel, grid, dim3(256), 2 * BM * 128, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_amplan(const aos_amplan_params *p, const aos_launch_ctx *ctx) {
  if (p->T < 1 || p->T > AOS_PREFILL_MAX_T || p->n < 1 || p->n > AOS_AM_MAX_N || p->am_tu < 1 || p->tu_cap < 1 ||
      p->tu_cap > AOS_TILE_U_MAX || p->cb < (8 * p->T + BM - 1) / BM + p->n || p->cb > 65535 || !p->count ||
      !p->done || !p->ctab || !p->users || !p->tu || !p->list || !p->coef || p->nz < 0 || p->nz > 2)
    return (int)hipErrorInvalidValue;
  for (int z = 0; z < p->nz; ++z) {
    const aos_am_zero &zb = p->zb[z];
    if (!zb.SA || zb.nmod < 1 || zb.nmod > 3 || zb.s_stride % 8) return (int)hipErrorInvalidValue;
    int cols = 0;
    for (int i = 0; i < zb.nmod; ++i) {
      if (zb.rpad[i] < 0 || zb.rpad[i] % 16) return (int)hipErrorInvalidValue;
      cols += p->tu_cap * zb.rpad[i];
    }
    if (cols > zb.s_stride) return (int)hipErrorInvalidValue;
  }
  AOS_LAUNCH(ctx, aos_amplan_kernel, dim3(1 + AM_ZB, (p->T + BM - 1) / BM), dim3(AM_NT), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_amx(const aos_amx_params *p, const aos_launch_ctx *ctx) {
  if (p->T < 1 || p->T > AOS_PREFILL_MAX_T || p->n < 1 || p->n > AOS_XAM_MAX_N || p->tu_cap < p->n ||
      p->mtiles != (p->T + BM - 1) / BM || p->RB < 1 || !p->tu || !p->tinfo || !p->inv || !p->xl || !p->users ||
      !p->rlp || !p->ct || !p->nch || !p->cidx)
    return (int)hipErrorInvalidValue;
  const int ranges = (p->mtiles + AOS_XAM_RT - 1) / AOS_XAM_RT;
  if (p->list) {
    AOS_LAUNCH(ctx, aos_amxlist_kernel, dim3(ranges), dim3(256), 0, *p);
    return (int)hipGetLastError();
  }
  const int rp = p->rpad[0];
  if (rp < 16 || rp > 64 || rp % 16 || p->rpad[1] != rp || !p->Bf[0] || !p->Bf[1] || !p->SAc || !p->xd)
    return (int)hipErrorInvalidValue;
  const size_t lds = (size_t)(AOS_XAM_RT * BM + 1) * 32 * 4;
  const void *fn[4] = {(const void *)aos_amxexp_kernel<1>, (const void *)aos_amxexp_kernel<2>,
                       (const void *)aos_amxexp_kernel<3>, (const void *)aos_amxexp_kernel<4>};
  /* dynamic LDS above 64 KiB must be allowed once per device and kernel */
  static uint64_t allowed[4] = {0, 0, 0, 0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return (int)hipErrorInvalidValue;
  const int ks = rp / 16;
  if (!(allowed[ks - 1] >> dev & 1u)) {
    const hipError_t e = hipFuncSetAttribute(fn[ks - 1], hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    allowed[ks - 1] |= 1ull << dev;
  }
  const dim3 grid(ranges * 2 * p->RB), block(256);
  if (ks == 1) AOS_LAUNCH(ctx, aos_amxexp_kernel<1>, grid, block, lds, *p);
  else if (ks == 2) AOS_LAUNCH(ctx, aos_amxexp_kernel<2>, grid, block, lds, *p);
  else if (ks == 3) AOS_LAUNCH(ctx, aos_amxexp_kernel<3>, grid, block, lds, *p);
  else AOS_LAUNCH(ctx, aos_amxexp_kernel<4>, grid, block, lds, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_amshrink(const aos_amshrink_params *p, const aos_launch_ctx *ctx) {
  if (p->T < 1 || p->T > AOS_PREFILL_MAX_T || p->nmod < 1 || p->nmod > 3 || p->ks < 1 || p->cb < 1 ||
      p->cb > 65535 || p->in % 64 || p->in < 64 * p->ks || !p->ctab || !p->users || !p->tu || !p->coef || !p->SA ||
      !p->zero_row || (p->ks > 1 && !p->part))
    return (int)hipErrorInvalidValue;
  int cols = 0;
  for (int i = 0; i < p->nmod; ++i) {
    if (p->rpad[i] < 16 || p->rpad[i] % 16 || !p->A[i]) return (int)hipErrorInvalidValue;
    cols += p->rpad[i];
  }
  if ((p->setw != 64 && p->setw != 128) || (p->setw == 64 && cols > 64) || p->csets != (cols + p->setw - 1) / p->setw ||
      p->s_stride % 8)
    return (int)hipErrorInvalidValue;
  if (p->reduce) {
    if (p->ks < 2) return (int)hipErrorInvalidValue;
    AOS_LAUNCH(ctx, aos_amreduce_kernel, dim3(p->cb, p->csets), dim3(256), 0, *p);
  } else {
    if (p->setw == 64)
      AOS_LAUNCH(ctx, aos_amshrink_kernel<2>, dim3(p->ks, p->cb, p->csets), dim3(128), 2 * BM * 128, *p);
    else
      AOS_LAUNCH(ctx, aos_amshrink_kernel<4>, dim3(p->ks, p->cb, p->csets), dim3(256), 2 * BM * 128, *p);
  }
  return (int)hipGetLastError();
}

/* Kernel shapes (measured on the 7B-shaped layer at 2048 tokens): 128-token tiles at two waves
 * per SIMD, so that one wave's dequantisation overlaps the other's matrix-core work; SwiGLU with
 * a shallow ring and single staging in 4-wave workgroups (two per CU), the single-matrix kernel
 * with the deep pipeline in 8-wave workgroups. */
template <bool SW, int D, bool DBT, bool APF, int WV, int OCC, int LC, int NS>
static int launch_gemm_cfg(const aos_gemm_params *p, const aos_launch_ctx *ctx) {
  constexpr int NTILE = gemm_ntile<NS, LC>();
  aos_gemm_params q = *p;
  q.mb = (q.T + BM - 1) / BM;
  q.nb = (q.w0.RB + WV - 1) / WV;
  /* shrink workgroups: one module, 32 columns per wave (they use the LDS ring: NS > 0) */
  q.nbs = q.s_cols > 0 ? (SW ? 2 : 1) * ((q.s_cols + 32 * WV - 1) / (32 * WV)) : 0;
  if (q.nbs && NS == 0) return (int)hipErrorInvalidValue;
  const size_t lds = (size_t)NTILE * BM * 128 + gemm_aux();
  const dim3 grid(q.mb * (q.nbs + q.nb)), block(64 * WV);
  const int G = q.w0.G;
  if (q.sk_nwg > 0) {
    if (NS == 0 || !q.sk_part || !q.sk_lines || !q.gen ||
        (uint64_t)q.mb * q.nb * G * (uint64_t)q.sk_nwg >= (1ull << 32))
      return (int)hipErrorInvalidValue;
    const dim3 skg(q.mb * q.nbs + q.sk_nwg);
    if (G % D == 0)
      AOS_LAUNCH(ctx, (aos_gemm_sk_kernel<SW, D, DBT, APF, WV, OCC, LC, (NS > 0 ? NS : 2)>), skg, block, lds, q);
    else if (G % 2 == 0)
      AOS_LAUNCH(ctx, (aos_gemm_sk_kernel<SW, 2, DBT, APF, WV, OCC, LC, (NS > 0 ? NS : 2)>), skg, block, lds, q);
    else
      AOS_LAUNCH(ctx, (aos_gemm_sk_kernel<SW, 1, DBT, APF, WV, OCC, LC, (NS > 0 ? NS : 2)>), skg, block, lds, q);
    return (int)hipGetLastError();
  }
  if (G % D == 0)
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, D, DBT, APF, WV, OCC, LC, NS>), grid, block, lds, q);
  else if (G % 2 == 0)
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, 2, DBT, APF, WV, OCC, LC, NS>), grid, block, lds, q);
  else
    AOS_LAUNCH(ctx, (aos_gemm_kernel<SW, 1, DBT, APF, WV, OCC, LC, NS>), grid, block, lds, q);
  return (int)hipGetLastError();
}

#ifndef AOS_GEMM_NS_SW
#define AOS_GEMM_NS_SW 4 /* token-tile LDS stages, SwiGLU GEMM (0: register staging) */
#endif
#ifndef AOS_GEMM_NS_ONE
#define AOS_GEMM_NS_ONE 4 /* ... single-matrix GEMM */
#endif

/* Whether a GEMM's shrink workgroups (s_cols columns per module at the widest union) fit in the
 * idle slots of its grid's last round on the current device: then the launch takes no longer with
 * them. Workgroups resident per CU: the waves the kernel's registers allow, and its LDS. */
template <bool SW, int WV, int OCC, int LC, int NS>
static int shrink_fits_cfg(int T, int RB, int s_cols) {
  if (NS == 0 || s_cols <= 0) return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus < 1)
    return 0;
  const size_t lds = (size_t)gemm_ntile<NS, LC>() * BM * 128 + gemm_aux();
  int per_cu = 4 * OCC / WV;
  const int by_lds = (int)(((size_t)160 << 10) / lds);
  if (by_lds < per_cu) per_cu = by_lds;
  if (per_cu < 1) per_cu = 1;
  const long slots = (long)cus * per_cu;
  const long n = (long)((T + BM - 1) / BM) * ((RB + WV - 1) / WV);
  const long slack = (n + slots - 1) / slots * slots - n;
  const long nsh = (long)((T + BM - 1) / BM) * (SW ? 2 : 1) * ((s_cols + 32 * WV - 1) / (32 * WV));
  return nsh <= slack ? 1 : 0;
}

extern "C" int aos_gemm_shrink_fits(int T, int RB, int s_cols, int swiglu) {
  if (swiglu) return shrink_fits_cfg<true, 4, 2, 2, AOS_GEMM_NS_SW>(T, RB, s_cols);
  return shrink_fits_cfg<false, 8, 2, 4, AOS_GEMM_NS_ONE>(T, RB, s_cols);
}

/* Workgroups of one kernel shape resident at once on the current device (registers and LDS). */
template <bool SW, int D, bool DBT, bool APF, int WV, int OCC, int LC, int NS>
static int sk_slots_cfg() {
  int dev = 0, cus = 0, per_cu = 0;
  const size_t lds = (size_t)gemm_ntile<NS, LC>() * BM * 128 + gemm_aux();
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus < 1)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, aos_gemm_sk_kernel<SW, D, DBT, APF, WV, OCC, LC, NS>,
                                                   64 * WV, lds) != hipSuccess || per_cu < 1)
    return 0;
  return cus * per_cu;
}

extern "C" int aos_gemm_sk_slots(int swiglu) {
  if (swiglu) return sk_slots_cfg<true, 2, false, false, 4, 2, 2, AOS_GEMM_NS_SW>();
  return sk_slots_cfg<false, 4, true, true, 8, 2, 4, AOS_GEMM_NS_ONE>();
}

extern "C" int aos_gemm_sk_slot_floats(int swiglu) { return (swiglu ? 4 * 2 : 8) * (BM / 32) * 16 * 64; }

extern "C" int aos_launch_gemm(const aos_gemm_params *p, int swiglu, const aos_launch_ctx *ctx) {
  if (p->T < 1 || p->T > AOS_PREFILL_MAX_T || p->mtiles != (p->T + BM - 1) / BM || (p->sa_mod_before < 0) ||
      p->sa_mod_before > 2 || p->rpad0 % 16 || p->rpad1 % 16 || (swiglu && (!p->w1.qt || p->w1.RB != p->w0.RB)))
    return (int)hipErrorInvalidValue;
  if (p->s_cols < 0 || (p->s_cols > 0 && (!p->ap || !p->coef || !p->sa_out || p->sa_out != p->SA || !p->sa_ctr ||
                                          !p->sa_lines || !p->gen || !p->tu || p->s_cols > p->tu_cap * 1024)))
    return (int)hipErrorInvalidValue;
  if (swiglu) return launch_gemm_cfg<true, 2, false, false, 4, 2, 2, AOS_GEMM_NS_SW>(p, ctx);
  return launch_gemm_cfg<false, 4, true, true, 8, 2, 4, AOS_GEMM_NS_ONE>(p, ctx);
}

AOS_DEFINE_SPIN_SETTER(aos_spin_setter_gemm)
