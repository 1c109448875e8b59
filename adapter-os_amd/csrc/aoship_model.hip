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

__global__ void __launch_bounds__(256) aos_embed_kernel(aos_embed_params p) {
  const int t = blockIdx.x;
  const int id = p.ids[t];
  float *dst = p.hidden + (size_t)t * p.H;
  if (id < 0 || id >= p.vocab) {
    for (int e = threadIdx.x; e < p.H; e += blockDim.x) dst[e] = 0.0f;
    if (threadIdx.x == 0 && p.status) p.status[0] = 1;
    return;
  }
  if (p.q4) {
    const uint32_t *row = p.q4 + (size_t)id * (p.H / 8);
    const uint16_t *sr = p.s16 + (size_t)id * (p.H / 64);
    const uint16_t *br = p.b16 ? p.b16 + (size_t)id * (p.H / 64) : nullptr;
    for (int e = threadIdx.x; e < p.H; e += blockDim.x) {
      const uint32_t q = (row[e >> 3] >> (4 * (e & 7))) & 15u; /* low nibble first */
      const float s = aos_f16_to_f32(sr[e >> 6]);
      const float b = br ? aos_f16_to_f32(br[e >> 6]) : 0.0f;
      dst[e] = s * (float)q + b;
    }
  } else {
    const uint16_t *row = p.bf16 + (size_t)id * p.H;
    for (int e = threadIdx.x; e < p.H; e += blockDim.x) dst[e] = aos_bf16_to_f32(row[e]);
  }
}

/* ---- residual add + RMSNorm ------------------------------------------------------------------- */

__global__ void __launch_bounds__(256) aos_norm_kernel(aos_norm_params p) {
  __shared__ float red[256];
  const int t = blockIdx.x, tid = threadIdx.x;
  float *x = p.hidden + (size_t)t * p.H;
  const uint16_t *a = p.add ? p.add + (size_t)t * p.H : nullptr;
  float ss = 0.0f;
  for (int e = tid; e < p.H; e += 256) {
    float v = x[e];
    if (a) {
      v = v + aos_bf16_to_f32(a[e]);
      x[e] = v;
    }
    ss += v * v;
  }
  red[tid] = ss;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) { /* fixed-order tree */
    if (tid < w) red[tid] = red[tid] + red[tid + w];
    __syncthreads();
  }
  const float mean = red[0] / (float)p.H;
  const float d = sqrtf(mean + p.eps);
  uint16_t *o = p.out + (size_t)t * p.H;
  for (int e = tid; e < p.H; e += 256) o[e] = aos_f32_to_bf16(x[e] * (p.w[e] / d));
}

/* ---- RoPE, biases, KV cache append ---------------------------------------------------------- */

__global__ void __launch_bounds__(256) aos_rope_kernel(aos_rope_params p) {
  const int t = blockIdx.x, half = p.hd / 2;
  const int pos = p.offset + t;
  const float fpos = (float)pos;
  const int nq = p.nh * half, nk = p.nkv * half, nv = p.nkv * p.hd;
  for (int w = threadIdx.x; w < nq + nk + nv; w += blockDim.x) {
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

/* One wave: positions [split * chunk, min(+chunk, visible)) of token t for head h. Phase 1 puts
 * one position on each lane (its score, q . k in order over d), phase 2 one or more dimensions on
 * each lane (acc += p . v over the 64 positions in order). */
template <int DPL>
__global__ void __launch_bounds__(64) aos_attn_kernel(aos_attn_params p) {
  __shared__ float qs[AOS_ATTN_MAX_HD];
  __shared__ float ps[64];
  const int split = blockIdx.x, h = blockIdx.y, t = blockIdx.z, lane = threadIdx.x;
  const int hd = p.hd, kvh = h / (p.nh / p.nkv);
  const int visible = p.offset + t + 1;
  const int beg = split * p.chunk;
  const int end = min(beg + p.chunk, visible);
  const float *q = p.q + ((size_t)t * p.nh + h) * hd;
  for (int d = lane; d < hd; d += 64) qs[d] = q[d];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  const uint16_t *kbase = p.kc + (size_t)kvh * p.max_seq * hd;
  const uint16_t *vbase = p.vc + (size_t)kvh * p.max_seq * hd;
  float m = -__builtin_inff(), l = 0.0f, acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.0f;
  for (int base = beg; base < end; base += 64) {
    const int pos = base + lane;
    const bool valid = pos < end;
    float s = -__builtin_inff();
    if (valid) {
      const u32x4 *kr = (const u32x4 *)(kbase + (size_t)pos * hd);
      float dot = 0.0f;
      for (int c = 0; c < hd / 8; ++c) {
        const u32x4 w = kr[c];
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dot = dot + qs[8 * c + 2 * e] * __builtin_bit_cast(float, wv[e] << 16);
          dot = dot + qs[8 * c + 2 * e + 1] * __builtin_bit_cast(float, wv[e] & 0xffff0000u);
        }
      }
      s = dot * p.scale;
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
    const int n = min(64, end - base);
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int d = lane + 64 * j;
      float a = acc[j] * alpha;
      if (d < hd)
        for (int jj = 0; jj < n; ++jj) a = a + ps[jj] * aos_bf16_to_f32(vbase[(size_t)(base + jj) * hd + d]);
      acc[j] = a;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    m = mn;
  }
  if (p.splits == 1) {
    uint16_t *o = p.out + (size_t)t * p.nh * hd + (size_t)h * hd;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int d = lane + 64 * j;
      if (d < hd) o[d] = aos_f32_to_bf16(acc[j] / l);
    }
    return;
  }
  float *pp = p.part + (((size_t)t * p.nh + h) * p.splits + split) * (hd + 2);
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    if (d < hd) pp[d] = acc[j];
  }
  if (lane == 0) {
    pp[hd] = m;
    pp[hd + 1] = l;
  }
}

/* Merge of the splits of (head, token), in split order. A split past the visible positions has
 * max -inf and sum 0 and adds nothing. */
template <int DPL>
__global__ void __launch_bounds__(64) aos_attn_merge_kernel(aos_attn_params p) {
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x, hd = p.hd;
  const float *pp = p.part + ((size_t)t * p.nh + h) * p.splits * (hd + 2);
  float M = -__builtin_inff();
  for (int s = 0; s < p.splits; ++s) M = fmaxf(M, pp[(size_t)s * (hd + 2) + hd]);
  float L = 0.0f, acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.0f;
  for (int s = 0; s < p.splits; ++s) {
    const float *q = pp + (size_t)s * (hd + 2);
    const float ms = q[hd], ls = q[hd + 1];
    if (!(ls > 0.0f)) continue;
    const float f = expf(ms - M);
    L = L + ls * f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int d = lane + 64 * j;
      if (d < hd) acc[j] = acc[j] + q[d] * f;
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
int launch_attn(const aos_attn_params *p, const aos_launch_ctx *ctx) {
  AOS_LAUNCH(ctx, aos_attn_kernel<DPL>, dim3(p->splits, p->nh, p->T), dim3(64), 0, *p);
  if (p->splits > 1) AOS_LAUNCH(ctx, aos_attn_merge_kernel<DPL>, dim3(p->nh, p->T), dim3(64), 0, *p);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int aos_launch_embed(const aos_embed_params *p, const aos_launch_ctx *ctx) {
  AOS_LAUNCH(ctx, aos_embed_kernel, dim3(p->T), dim3(256), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_norm(const aos_norm_params *p, const aos_launch_ctx *ctx) {
  AOS_LAUNCH(ctx, aos_norm_kernel, dim3(p->T), dim3(256), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_rope(const aos_rope_params *p, const aos_launch_ctx *ctx) {
  AOS_LAUNCH(ctx, aos_rope_kernel, dim3(p->T), dim3(256), 0, *p);
  return (int)hipGetLastError();
}

extern "C" int aos_launch_attention(const aos_attn_params *p, const aos_launch_ctx *ctx) {
  if (p->hd <= 64) return launch_attn<1>(p, ctx);
  if (p->hd <= 128) return launch_attn<2>(p, ctx);
  return launch_attn<4>(p, ctx);
}
