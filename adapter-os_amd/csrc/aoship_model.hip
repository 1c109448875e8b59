/*
 * aoship_model.hip — the parts of a decoder step around the adapter-augmented projections, as in
 * the MLX fused forward (mlx_model_forward_with_cache_and_lora,
 * crates/adapteros-lora-mlx-ffi/src/mlx_cpp_wrapper_real.cpp:3339-3527):
 *
 *   embedding lookup          take(embed, ids) with 4-bit rows dequantised (…real.cpp:3421-3432)
 *   residual add + RMSNorm    x * (w / sqrt(mean(x^2) + eps)) (…real.cpp:3384-3390), float32, the
 *                             residual stream kept in float32 (MLX promotes to float32 after RoPE)
 *   RoPE + bias + KV cache    the fused forward's rotation (…real.cpp:3249-3279): halves
 *                             [x1, x2] -> [x1 cos - x2 sin, x1 sin + x2 cos] with
 *                             inv_freq_i = 1 / theta^(-2i / hd), angle = position * inv_freq_i;
 *                             K and V appended to a bf16 cache laid out [kv head][position][hd]
 *   attention                 causal scaled dot-product attention over the cache, GQA by head
 *                             group (…real.cpp:3282-3327): one wave per (split of positions,
 *                             head, token) with an online softmax in float32, then a fixed-order
 *                             merge of the splits
 *
 * Every reduction has a fixed order, so results are bit-identical run to run.
 */
#include "aoship_device.h"
#include "aoship_internal.h"
#include <hip/hip_ext.h>

namespace {

/* ---- embedding -------------------------------------------------------------------------------- */

/* One thread per 8 elements of a row (one packed word, or 16 bytes of bfloat16), so every load of
 * the launch is in flight at once. */
__global__ void __launch_bounds__(256) aos_embed_kernel(aos_embed_params p) {
  const int t = blockIdx.y, g = blockIdx.x * 256 + threadIdx.x;
  if (8 * g >= p.H) return;
  const int id = p.ids[t];
  float4 *dst = (float4 *)(p.hidden + (size_t)t * p.H + 8 * g);
  if (id < 0 || id >= p.vocab) {
    dst[0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    dst[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (g == 0 && p.status) p.status[0] = 1;
    return;
  }
  float v[8];
  if (p.q4) {
    const uint32_t w = p.q4[(size_t)id * (p.H / 8) + g];
    const size_t gi = (size_t)id * (p.H / 64) + (g >> 3);
    const float s = aos_f16_to_f32(p.s16[gi]);
    const float b = p.b16 ? aos_f16_to_f32(p.b16[gi]) : 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = s * (float)((w >> (4 * e)) & 15u) + b; /* low nibble first */
  } else {
    const u32x4 r = *(const u32x4 *)(p.bf16 + (size_t)id * p.H + 8 * g);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = __builtin_bit_cast(float, w[e] << 16);
      v[2 * e + 1] = __builtin_bit_cast(float, w[e] & 0xffff0000u);
    }
  }
  dst[0] = make_float4(v[0], v[1], v[2], v[3]);
  dst[1] = make_float4(v[4], v[5], v[6], v[7]);
}

/* ---- residual add + RMSNorm ------------------------------------------------------------------- */

/* One workgroup of 1024 threads per token; each thread holds up to NORM_J runs of 4 elements
 * (H <= 16384), loaded together before any arithmetic. The sum of squares is formed per thread
 * in element order, across each wave by a butterfly and across the 16 waves in wave order. */
constexpr int NORM_J = 4;

__global__ void __launch_bounds__(1024) aos_norm_kernel(aos_norm_params p) {
  __shared__ float red[16];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, H = p.H;
  float *x = p.hidden + (size_t)t * H;
  const uint16_t *a = p.add ? p.add + (size_t)t * H : nullptr;
  float4 xv[NORM_J], wv[NORM_J];
  u32x2 av[NORM_J];
#pragma unroll
  for (int j = 0; j < NORM_J; ++j) {
    const int e = 4 * (tid + 1024 * j);
    if (e < H) {
      xv[j] = *(const float4 *)(x + e);
      wv[j] = *(const float4 *)(p.w + e);
      if (a) av[j] = *(const u32x2 *)(a + e);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NORM_J; ++j) {
    const int e = 4 * (tid + 1024 * j);
    if (e < H) {
      if (a) {
        xv[j].x = xv[j].x + __builtin_bit_cast(float, av[j].x << 16);
        xv[j].y = xv[j].y + __builtin_bit_cast(float, av[j].x & 0xffff0000u);
        xv[j].z = xv[j].z + __builtin_bit_cast(float, av[j].y << 16);
        xv[j].w = xv[j].w + __builtin_bit_cast(float, av[j].y & 0xffff0000u);
        *(float4 *)(x + e) = xv[j];
      }
      ss += xv[j].x * xv[j].x;
      ss += xv[j].y * xv[j].y;
      ss += xv[j].z * xv[j].z;
      ss += xv[j].w * xv[j].w;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss = ss + aos_shfl_f(ss, lane ^ o);
  if (lane == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) tot += red[w];
  const float mean = tot / (float)H;
  const float d = sqrtf(mean + p.eps);
  uint16_t *o = p.out + (size_t)t * H;
#pragma unroll
  for (int j = 0; j < NORM_J; ++j) {
    const int e = 4 * (tid + 1024 * j);
    if (e < H) {
      u32x2 r;
      r.x = (uint32_t)aos_f32_to_bf16(xv[j].x * (wv[j].x / d)) | ((uint32_t)aos_f32_to_bf16(xv[j].y * (wv[j].y / d)) << 16);
      r.y = (uint32_t)aos_f32_to_bf16(xv[j].z * (wv[j].z / d)) | ((uint32_t)aos_f32_to_bf16(xv[j].w * (wv[j].w / d)) << 16);
      *(u32x2 *)(o + e) = r;
    }
  }
}

/* ---- RoPE, biases, KV cache append ---------------------------------------------------------- */

/* One thread per rotated pair of q or k, or per element of v. */
__global__ void __launch_bounds__(256) aos_rope_kernel(aos_rope_params p) {
  const int t = blockIdx.y, half = p.hd / 2;
  const int pos = p.offset + t;
  const float fpos = (float)pos;
  const int nq = p.nh * half, nk = p.nkv * half, nv = p.nkv * p.hd;
  const int w = blockIdx.x * 256 + threadIdx.x;
  if (w >= nq + nk + nv) return;
  if (w < nq + nk) {
    const bool isq = w < nq;
    const int idx = isq ? w : w - nq;
    const int h = idx / half, i = idx - h * half;
    const int width = (isq ? p.nh : p.nkv) * p.hd;
    const uint16_t *src = (isq ? p.q : p.k) + (size_t)t * width + (size_t)h * p.hd;
    const float *bias = isq ? p.bq : p.bk;
    float x1 = aos_bf16_to_f32(src[i]), x2 = aos_bf16_to_f32(src[i + half]);
    if (bias) {
      x1 = x1 + bias[h * p.hd + i];
      x2 = x2 + bias[h * p.hd + i + half];
    }
    const float ang = fpos * p.inv_freq[i];
    const float c = cosf(ang), s = sinf(ang);
    const float r1 = x1 * c - x2 * s, r2 = x1 * s + x2 * c;
    if (isq) {
      float *dst = p.qr + ((size_t)t * p.nh + h) * p.hd;
      dst[i] = r1;
      dst[i + half] = r2;
    } else {
      uint16_t *dst = p.kc + ((size_t)h * p.max_seq + pos) * p.hd;
      dst[i] = aos_f32_to_bf16(r1);
      dst[i + half] = aos_f32_to_bf16(r2);
    }
  } else {
    const int idx = w - nq - nk;
    const int h = idx / p.hd, d = idx - h * p.hd;
    float v = aos_bf16_to_f32(p.v[(size_t)t * nv + idx]);
    if (p.bv) v = v + p.bv[idx];
    p.vc[((size_t)h * p.max_seq + pos) * p.hd + d] = aos_f32_to_bf16(v);
  }
}

/* ---- attention ---------------------------------------------------------------------------------- */

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, aos_shfl_f(v, (int)(threadIdx.x ^ o)));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = v + aos_shfl_f(v, (int)(threadIdx.x ^ o));
  return v;
}

/* One wave: positions [split * chunk, min(+chunk, visible)) of token t for head h, in blocks of
 * 64. Phase 1 puts one position on each lane: its key row (hd <= 64 * DPL) is loaded whole, then
 * the score q . k is formed in order over d. Phase 2 puts one or two 32-bit words of the value row
 * (two dimensions each) on each lane and adds p . v over the block's positions in order. A
 * block's key rows and its first PB value rows are loaded before anything waits on memory (the
 * query is staged into LDS behind them), so a block costs about one memory round trip. */
constexpr int ATTN_MAX_SPLITS = 1024;
constexpr int MERGE_B = 16;

/* RoPE of one pair (x1, x2) = (x[i], x[i + hd/2]) at position pos, as the separate RoPE kernel
 * computes it. */
__device__ __forceinline__ void rope_pair(float x1, float x2, float fpos, float invf, float &r1, float &r2) {
  const float ang = fpos * invf;
  const float c = cosf(ang), s = sinf(ang);
  r1 = x1 * c - x2 * s;
  r2 = x1 * s + x2 * c;
}

template <int DPL>
__device__ void attn_merge(const aos_attn_params &p, int h, int t, int lane, float *fs, float *lf);

template <int DPL>
__global__ void __launch_bounds__(64) aos_attn_kernel(aos_attn_params p) {
  constexpr int NC = 8 * DPL;            /* 16-byte chunks of the longest key row */
  constexpr int NW = (DPL + 1) / 2;      /* value words per lane */
  constexpr int PB = DPL > 2 ? 32 : 64;  /* value rows loaded per batch */
  __shared__ float qs[AOS_ATTN_MAX_HD];
  __shared__ float ps[64];
  __shared__ __attribute__((aligned(16))) uint32_t kcur[AOS_ATTN_MAX_HD / 2]; /* current key, bf16 pairs */
  __shared__ uint32_t vcur[AOS_ATTN_MAX_HD / 2];                             /* current value */
  const int split = blockIdx.x, h = blockIdx.y, t = blockIdx.z, lane = threadIdx.x;
  const int hd = p.hd, hw = hd / 2, kvh = h / (p.nh / p.nkv);
  const int visible = p.offset + t + 1;
  const int beg = split * p.chunk;
  const int end = min(beg + p.chunk, visible);
  const float *q = p.q + ((size_t)t * p.nh + h) * hd;
  /* rope_fused: this token's own key and value are formed here, not read from the cache */
  const int cur = p.offset + t;
  const bool has_cur = p.rope_fused && beg <= cur && cur < end;
  const uint16_t *kbase = p.kc + (size_t)kvh * p.max_seq * hd;
  const uint32_t *vbase = (const uint32_t *)(p.vc + (size_t)kvh * p.max_seq * hd);
  float m = -__builtin_inff(), l = 0.0f, acc[2 * NW];
#pragma unroll
  for (int j = 0; j < 2 * NW; ++j) acc[j] = 0.0f;
  int wi[NW];
#pragma unroll
  for (int jw = 0; jw < NW; ++jw) {
    const int w = lane + 64 * jw;
    wi[jw] = w < hw ? w : 0;
  }
  /* rope_fused: the token's query pairs (and, in the split holding its position, its key pairs
   * and value words) with their biases and frequencies are loaded first, so that they share the
   * memory round trip of the first block's key and value rows; pair w = lane + 64 jw */
  float cq1[NW], cq2[NW], cf[NW], ck1[NW], ck2[NW], cv0[NW], cv1[NW];
  if (p.rope_fused) {
    const uint16_t *qb = p.qb + (size_t)h * hd;
    const uint16_t *kb = p.kb + (size_t)kvh * hd;
    const uint32_t *vb = (const uint32_t *)(p.vb + (size_t)kvh * hd);
#pragma unroll
    for (int jw = 0; jw < NW; ++jw) {
      const int w = wi[jw];
      cq1[jw] = aos_bf16_to_f32(qb[w]);
      cq2[jw] = aos_bf16_to_f32(qb[w + hw]);
      if (p.bq) {
        cq1[jw] = cq1[jw] + p.bq[h * hd + w];
        cq2[jw] = cq2[jw] + p.bq[h * hd + w + hw];
      }
      cf[jw] = p.inv_freq[w];
      ck1[jw] = ck2[jw] = cv0[jw] = cv1[jw] = 0.0f;
      if (has_cur) {
        ck1[jw] = aos_bf16_to_f32(kb[w]);
        ck2[jw] = aos_bf16_to_f32(kb[w + hw]);
        if (p.bk) {
          ck1[jw] = ck1[jw] + p.bk[kvh * hd + w];
          ck2[jw] = ck2[jw] + p.bk[kvh * hd + w + hw];
        }
        const uint32_t pr = vb[w];
        cv0[jw] = __builtin_bit_cast(float, pr << 16);
        cv1[jw] = __builtin_bit_cast(float, pr & 0xffff0000u);
        if (p.bv) {
          cv0[jw] = cv0[jw] + p.bv[kvh * hd + 2 * w];
          cv1[jw] = cv1[jw] + p.bv[kvh * hd + 2 * w + 1];
        }
      }
    }
  }
  for (int base = beg; base < end; base += 64) {
    const int pos = base + lane;
    const bool valid = pos < end;
    const int n = min(64, end - base);
    u32x4 kv[NC];
    {
      const u32x4 *kr = (const u32x4 *)(kbase + (size_t)(valid ? pos : base) * hd);
#pragma unroll
      for (int c = 0; c < NC; ++c) kv[c] = c < hd / 8 ? kr[c] : kv[0];
    }
    uint32_t vv[PB][NW];
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int jj = u < n ? u : n - 1;
#pragma unroll
      for (int jw = 0; jw < NW; ++jw) vv[u][jw] = vbase[(size_t)(base + jj) * hw + wi[jw]];
    }
    if (base == beg) {
      if (p.rope_fused) {
        const float fpos = (float)cur;
        /* the key and value as the cache holds them (bf16); the first head of the group
         * appends them */
        const bool writer = has_cur && h % (p.nh / p.nkv) == 0;
        uint16_t *kdst = p.kc + ((size_t)kvh * p.max_seq + cur) * hd;
        uint32_t *vdst = (uint32_t *)(p.vc + ((size_t)kvh * p.max_seq + cur) * hd);
#pragma unroll
        for (int jw = 0; jw < NW; ++jw) {
          const int i = lane + 64 * jw;
          if (i < hw) {
            rope_pair(cq1[jw], cq2[jw], fpos, cf[jw], qs[i], qs[i + hw]);
            if (has_cur) {
              float r1, r2;
              rope_pair(ck1[jw], ck2[jw], fpos, cf[jw], r1, r2);
              const uint16_t b1 = aos_f32_to_bf16(r1), b2 = aos_f32_to_bf16(r2);
              ((uint16_t *)kcur)[i] = b1;
              ((uint16_t *)kcur)[i + hw] = b2;
              const uint32_t o = (uint32_t)aos_f32_to_bf16(cv0[jw]) | ((uint32_t)aos_f32_to_bf16(cv1[jw]) << 16);
              vcur[i] = o;
              if (writer) {
                kdst[i] = b1;
                kdst[i + hw] = b2;
                vdst[i] = o;
              }
            }
          }
        }
      } else {
        for (int d = lane; d < hd; d += 64) qs[d] = q[d];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
    if (has_cur && pos == cur) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (c < hd / 8) kv[c] = ((const u32x4 *)kcur)[c];
    }
    float s = -__builtin_inff();
    {
      float dot = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (c < hd / 8) {
          const uint32_t wv[4] = {kv[c].x, kv[c].y, kv[c].z, kv[c].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dot = dot + qs[8 * c + 2 * e] * __builtin_bit_cast(float, wv[e] << 16);
            dot = dot + qs[8 * c + 2 * e + 1] * __builtin_bit_cast(float, wv[e] & 0xffff0000u);
          }
        }
      }
      if (valid) s = dot * p.scale;
    }
    const float mc = wave_max(s);
    const float mn = fmaxf(m, mc);
    const float alpha = expf(m - mn);
    const float pv = valid ? expf(s - mn) : 0.0f;
    l = l * alpha + wave_sum(pv);
    ps[lane] = pv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
    for (int j = 0; j < 2 * NW; ++j) acc[j] = acc[j] * alpha;
    for (int j0 = 0; j0 < n; j0 += PB) {
      if (j0 > 0) {
#pragma unroll
        for (int u = 0; u < PB; ++u) {
          const int jj = j0 + u < n ? j0 + u : n - 1;
#pragma unroll
          for (int jw = 0; jw < NW; ++jw) vv[u][jw] = vbase[(size_t)(base + jj) * hw + wi[jw]];
        }
      }
      if (has_cur && cur >= base + j0 && cur < base + j0 + PB) { /* uniform */
        const int uc = cur - base - j0;
#pragma unroll
        for (int u = 0; u < PB; ++u)
          if (u == uc) {
#pragma unroll
            for (int jw = 0; jw < NW; ++jw) vv[u][jw] = vcur[wi[jw]];
          }
      }
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        if (j0 + u < n) {
          const float pj = ps[j0 + u];
#pragma unroll
          for (int jw = 0; jw < NW; ++jw) {
            acc[2 * jw] = acc[2 * jw] + pj * __builtin_bit_cast(float, vv[u][jw] << 16);
            acc[2 * jw + 1] = acc[2 * jw + 1] + pj * __builtin_bit_cast(float, vv[u][jw] & 0xffff0000u);
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    m = mn;
  }
  if (p.splits == 1) {
    uint32_t *o = (uint32_t *)(p.out + (size_t)t * p.nh * hd + (size_t)h * hd);
#pragma unroll
    for (int jw = 0; jw < NW; ++jw) {
      const int w = lane + 64 * jw;
      if (w < hw)
        o[w] = (uint32_t)aos_f32_to_bf16(acc[2 * jw] / l) | ((uint32_t)aos_f32_to_bf16(acc[2 * jw + 1] / l) << 16);
    }
    return;
  }
  float *pp = p.part + (((size_t)t * p.nh + h) * p.splits + split) * (hd + 2);
  if (!p.counters) {
#pragma unroll
    for (int jw = 0; jw < NW; ++jw) {
      const int w = lane + 64 * jw;
      if (w < hw) {
        pp[2 * w] = acc[2 * jw];
        pp[2 * w + 1] = acc[2 * jw + 1];
      }
    }
    if (lane == 0) {
      pp[hd] = m;
      pp[hd + 1] = l;
    }
    return;
  }
  /* device-scope stores, then the arrival count; the last split of (token, head) merges */
#pragma unroll
  for (int jw = 0; jw < NW; ++jw) {
    const int w = lane + 64 * jw;
    if (w < hw) {
      aos_publish(pp + 2 * w, acc[2 * jw]);
      aos_publish(pp + 2 * w + 1, acc[2 * jw + 1]);
    }
  }
  if (lane == 0) {
    aos_publish(pp + hd, m);
    aos_publish(pp + hd + 1, l);
  }
  uint32_t *ctr = p.counters + (size_t)t * p.nh + h;
  uint32_t old = 0;
  if (lane == 0) old = aos_arrive(ctr);
  old = aos_shfl(old, 0);
  if (old != (uint32_t)p.splits - 1u) return;
  if (lane == 0) aos_reset(ctr);
  __shared__ float fs[1024], lf[1024];
  attn_merge<DPL>(p, h, t, lane, fs, lf);
}

/* Merge of the splits of (head, token), in split order. A split past the visible positions has
 * max -inf and sum 0 and adds nothing. The splits' maxima and sums are read one split per lane;
 * the partial outputs 16 splits at a time. */

template <int DPL>
__device__ void attn_merge(const aos_attn_params &p, int h, int t, int lane, float *fs, float *lf) {
  const int hd = p.hd, S = p.splits;
  const bool co = p.counters != nullptr; /* partials of this launch: device-scope loads */
  auto ld = [&](const float *a) { return co ? aos_collect(a) : *a; };
  const float *pp = p.part + ((size_t)t * p.nh + h) * S * (hd + 2);
  float mloc = -__builtin_inff();
  for (int s = lane; s < S; s += 64) mloc = fmaxf(mloc, ld(pp + (size_t)s * (hd + 2) + hd));
  const float M = wave_max(mloc);
  for (int s = lane; s < S; s += 64) {
    const float ms = ld(pp + (size_t)s * (hd + 2) + hd), ls = ld(pp + (size_t)s * (hd + 2) + hd + 1);
    const bool live = ls > 0.0f;
    const float f = live ? expf(ms - M) : 0.0f;
    fs[s] = f;
    lf[s] = live ? ls * f : 0.0f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  float L = 0.0f, acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.0f;
  int di[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    di[j] = d < hd ? d : 0;
  }
  for (int s0 = 0; s0 < S; s0 += MERGE_B) {
    float qv[MERGE_B][DPL];
#pragma unroll
    for (int u = 0; u < MERGE_B; ++u) {
      const int s = s0 + u < S ? s0 + u : S - 1;
#pragma unroll
      for (int j = 0; j < DPL; ++j) qv[u][j] = ld(pp + (size_t)s * (hd + 2) + di[j]);
    }
#pragma unroll
    for (int u = 0; u < MERGE_B; ++u) {
      if (s0 + u < S && fs[s0 + u] != 0.0f) {
        const float f = fs[s0 + u];
        L = L + lf[s0 + u];
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = acc[j] + qv[u][j] * f;
      }
    }
  }
  uint16_t *o = p.out + (size_t)t * p.nh * hd + (size_t)h * hd;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    if (d < hd) o[d] = aos_f32_to_bf16(acc[j] / L);
  }
}

template <int DPL>
__global__ void __launch_bounds__(64) aos_attn_merge_kernel(aos_attn_params p) {
  __shared__ float fs[ATTN_MAX_SPLITS], lf[ATTN_MAX_SPLITS];
  attn_merge<DPL>(p, blockIdx.x, blockIdx.y, threadIdx.x, fs, lf);
}

template <int DPL>
int launch_attn(const aos_attn_params *p, const aos_launch_ctx *ctx) {
  AOS_LAUNCH(ctx, aos_attn_kernel<DPL>, dim3(p->splits, p->nh, p->T), dim3(64), 0, *p);
  if (p->splits > 1 && !p->counters) AOS_LAUNCH(ctx, aos_attn_merge_kernel<DPL>, dim3(p->nh, p->T), dim3(64), 0, *p);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int aos_launch_embed(const aos_embed_params *p, const aos_launch_ctx *ctx) {
  if (p->H % 64) return (int)hipErrorInvalidValue;
  AOS_LAUNCH(ctx, aos_embed_kernel, dim3((p->H / 8 + 255) / 256, p->T), dim3(256), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_norm(const aos_norm_params *p, const aos_launch_ctx *ctx) {
  if (p->H % 64 || p->H > 4 * 1024 * NORM_J) return (int)hipErrorInvalidValue;
  AOS_LAUNCH(ctx, aos_norm_kernel, dim3(p->T), dim3(1024), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_rope(const aos_rope_params *p, const aos_launch_ctx *ctx) {
  const int items = p->nh * (p->hd / 2) + p->nkv * (p->hd / 2) + p->nkv * p->hd;
  AOS_LAUNCH(ctx, aos_rope_kernel, dim3((items + 255) / 256, p->T), dim3(256), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_attention(const aos_attn_params *p, const aos_launch_ctx *ctx) {
  if (p->hd % 8 || p->hd > AOS_ATTN_MAX_HD || p->splits < 1 || p->splits > ATTN_MAX_SPLITS || p->chunk % 64)
    return (int)hipErrorInvalidValue;
  if (p->rope_fused && (p->T != 1 || !p->qb || !p->kb || !p->vb || !p->inv_freq)) return (int)hipErrorInvalidValue;
  if (p->hd <= 64) return launch_attn<1>(p, ctx);
  if (p->hd <= 128) return launch_attn<2>(p, ctx);
  return launch_attn<4>(p, ctx);
}

AOS_DEFINE_SPIN_SETTER(aos_spin_setter_model)
