/*
 * aoship_mlp1.hip — the decode MLP of one token in one launch, the down matrix held in LDS.
 *
 * Computes the SwiGLU MLP with LoRA on gate/up/down (mlx_cpp_wrapper_real.cpp:3509-3527, the
 * adapter deltas of apply_lora :3394-3419 over the ring as prepare_lora_for_ring selects them,
 * crates/adapteros-lora-mlx-ffi/src/backend.rs:398-428), optionally after routing the token from
 * its router features (crates/adapteros-lora-router/src/router.rs:1567-1952, the plain router).
 *
 * Why one launch: at one token the layer is a stream of int4 weights (gate and up, then down)
 * with a chain of dependent memory round trips after each stream (the LoRA expand, the h shrink,
 * the split sums). With one launch per matrix the down weights start streaming only after the
 * gate/up launch has ended. Here the down matrix is loaded into LDS while gate and up stream: two
 * workgroups per CU, 8 waves each, hold 1/nwg of the down units each (about 65 KiB at the
 * Qwen2.5-7B shape), so when h is complete the down product runs from LDS.
 *
 * Roles (aos_mlp1_params in aoship_internal.h describes the exchange buffers):
 *  - waves 0-3 ("G waves") stream an even share of the gate/up units, 16-byte loads per lane,
 *    a register ring 3 units deep, dequantised with the bf16 128 + q trick into
 *    v_mfma_f32_32x32x16_bf16 with the token as M (aoship_gemv.h, apply_group). A wave's share
 *    spans at most two row blocks; the wave holding a row block's last unit (its owner) sums the
 *    partials handed on by the waves before it, in order, adds the LoRA expand of gate and up
 *    (formed ahead by a D wave), applies SwiGLU, publishes h and forms the row block's part of
 *    the down shrink (hpart).
 *    Designated G waves that own nothing then sum hpart over the row blocks, one column each.
 *  - waves 4-7 ("D waves") first do producer work if they have any (a router prior per wave,
 *    the routing itself in the wave of the last prior; the x shrink, a 32-column tile over a K
 *    piece per wave, the last piece of a tile summing it; the rest the gate/up LoRA expand of
 *    row blocks, which needs only S and the ring), then load their down units into LDS
 *    (buffer_load ... lds), wait for the h groups they multiply, stage them in LDS and compute
 *    their partial sums; the owner of a down row block sums them with the LoRA expand and writes
 *    y.
 * Waiting waves poll little: a D wave first polls one word per (h group, producing owner) before
 * it loads all of its h words, since thousands of waves polling every word starve the streaming
 * waves of memory bandwidth. Unit indices are 32-bit (no 64-bit divisions in the kernel).
 * Every hand-over is a 64-bit word (payload | generation << 32), stored device-coherently and read
 * with device-coherent loads until its stamp equals this launch's generation; waits are bounded
 * (the spin limit of aoship_device.h): a wave that gives up sets the timeout word and skips what
 * it waited for. All reductions run in a fixed order, so results are identical run to run.
 *
 * Residency: every workgroup of the launch waits for data that other workgroups produce, so the
 * launch relies on all nwg = 2 x CUs workgroups being resident at once: the LDS size lets at most
 * two share a CU, and the host checks the registers (4 waves per SIMD) and that nothing else
 * shares the device's queue (one stream, in order). A wait that gives up ends the launch with the
 * timeout reported, never a hang.
 */
#include <hip/hip_ext.h>

#include "aoship_device.h"
#include "aoship_gemv.h"
#include "aoship_internal.h"
#include "aoship_route.h"

namespace {

constexpr int RD = 3; /* gate/up units in flight per G wave */

__device__ __forceinline__ void tag_store(uint64_t *p, uint32_t v, uint32_t gen) {
  __hip_atomic_store(p, ((uint64_t)gen << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t tag_load(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float fbits(uint32_t v) { return __builtin_bit_cast(float, v); }
__device__ __forceinline__ uint32_t ubits(float v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ void set_timeout(const aos_mlp1_params &p, int lane) {
  if (lane == 0 && p.timeout) __hip_atomic_store(p.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

/* A barrier of the workgroup's four G waves over LDS: each adds 1 to the LDS counter *ctr after
 * its LDS stores and waits (bounded) until it reaches target. Only LDS is ordered, so the waves'
 * outstanding global loads are not waited for. */
__device__ __forceinline__ void g_sync(const aos_mlp1_params &p, uint32_t *ctr, uint32_t target, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if (lane == 0) atomicAdd(ctr, 1u);
  const uint32_t limit = aos_spin_limit();
  uint32_t spins = 0;
  while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    if (spins++ >= limit) {
      set_timeout(p, lane);
      break;
    }
    __builtin_amdgcn_s_sleep(0);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* Loads N tagged words per lane (word k of this lane at addr(k), which must be a valid address
 * for every k and lane) until the stamps of the words with need(k) of every lane equal gen; the
 * payloads go to val. Returns false (uniformly) when it gave up. */
template <int N, int SLEEP = 2, class Addr, class Need>
__device__ __forceinline__ bool wait_tagged_if(Addr addr, Need need, uint32_t gen, uint32_t (&val)[N]) {
  const uint32_t limit = aos_spin_limit();
  uint32_t spins = 0;
  while (true) {
    if (spins++ >= limit) {
      aos_compiler_barrier();
      return false;
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const uint64_t w = tag_load(addr(k));
      ok = ok && (!need(k) || (uint32_t)(w >> 32) == gen);
      val[k] = (uint32_t)w;
    }
    if (__ballot(!ok) == 0ull) break;
    __builtin_amdgcn_s_sleep(SLEEP);
  }
  aos_compiler_barrier();
  return true;
}

/* wait_tagged_if for words that many waves wait for at once: after a failed check only word 0 of
 * the lanes with sent (which must need it) is polled until it is ready, then all words are checked
 * again, so the waiting waves load a few words per poll instead of N per lane. */
template <int N, int SLEEP = 2, class Addr, class Need>
__device__ __forceinline__ bool wait_tagged_sent(Addr addr, Need need, bool sent, uint32_t gen, uint32_t (&val)[N]) {
  const uint32_t limit = aos_spin_limit();
  uint32_t spins = 0;
  while (true) {
    if (spins++ >= limit) {
      aos_compiler_barrier();
      return false;
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const uint64_t w = tag_load(addr(k));
      ok = ok && (!need(k) || (uint32_t)(w >> 32) == gen);
      val[k] = (uint32_t)w;
    }
    if (__ballot(!ok) == 0ull) break;
    while (true) {
      __builtin_amdgcn_s_sleep(SLEEP);
      if (spins++ >= limit) {
        aos_compiler_barrier();
        return false;
      }
      const bool sok = !sent || (uint32_t)(tag_load(addr(0)) >> 32) == gen;
      if (__ballot(!sok) == 0ull) break;
    }
  }
  aos_compiler_barrier();
  return true;
}

/* wait_tagged_if for the words k < cnt. */
template <int N, int SLEEP = 2, class Addr>
__device__ __forceinline__ bool wait_tagged(Addr addr, int cnt, uint32_t gen, uint32_t (&val)[N]) {
  return wait_tagged_if<N, SLEEP>(addr, [&](int k) { return k < cnt; }, gen, val);
}

/* Waits, polling one word per lane, until the stamp of word addr (lanes with want) equals gen;
 * false (uniformly) when it gave up. Used before a wait_tagged over many words written by few
 * producers: one sentinel word per producer is polled instead of every word, which keeps waiting
 * waves from flooding the memory path the streaming waves use. */
__device__ __forceinline__ bool wait_sentinel(const uint64_t *addr, bool want, uint32_t gen) {
  const uint32_t limit = aos_spin_limit();
  uint32_t spins = 0;
  while (true) {
    if (spins++ >= limit) {
      aos_compiler_barrier();
      return false;
    }
    const bool ok = !want || (uint32_t)(tag_load(addr) >> 32) == gen;
    if (__ballot(!ok) == 0ull) break;
    __builtin_amdgcn_s_sleep(8);
  }
  aos_compiler_barrier();
  return true;
}

/* The union of the ring's adapters (prepare_lora_for_ring: slot < top_k, q > 0, a bound adapter of
 * the table), in ascending adapter index, with coef[u] = sum over the slots naming list[u] of
 * scale * (q / 32767), in slot order (the plan's arithmetic). rw: the ring's ten words (uniform);
 * bnd / scl: lane a holds adapter a's bound flag and scale. */
struct RingUnion {
  int U;
  int la;    /* lane u < U: the adapter of union slot u */
  float lcf; /* lane u < U: its coefficient */
  __device__ int a(int u) const { return (int)aos_shfl((uint32_t)la, u); }
  __device__ float cf(int u) const { return aos_shfl_f(lcf, u); }
};

__device__ __forceinline__ RingUnion ring_union(const uint32_t (&rw)[10], int n, uint32_t bnd, float scl, int lane) {
  RingUnion r;
  r.la = 0;
  r.lcf = 0.0f;
  const int top = (int)rw[0];
  uint64_t mask = 0;
  int idx[8], q[8];
  bool ok[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    idx[s] = (int)((rw[2 + (s >> 1)] >> (16 * (s & 1))) & 0xffffu);
    q[s] = (int)(int16_t)((rw[6 + (s >> 1)] >> (16 * (s & 1))) & 0xffffu);
    const int a = idx[s] < n ? idx[s] : 0;
    const uint32_t b = aos_shfl(bnd, a);
    ok[s] = s < top && q[s] > 0 && idx[s] < n && b != 0u;
    if (ok[s]) mask |= 1ull << idx[s];
  }
  r.U = __builtin_popcountll(mask);
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int a = mask ? __builtin_ctzll(mask) : 0;
    mask &= mask ? mask - 1ull : 0ull;
    const float sc = aos_shfl_f(scl, a);
    float c = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (ok[s] && idx[s] == a) c += sc * ((float)q[s] / 32767.0f);
    if (lane == u && u < r.U) {
      r.la = a;
      r.lcf = c;
    }
  }
  return r;
}

/* The ring's ten words, uniform: loaded from the input ring, or (routed in this launch) from the
 * tagged copy the routing wave publishes. */
__device__ __forceinline__ bool load_ring(const aos_mlp1_params &p, int lane, uint32_t (&rw)[10]) {
  uint32_t v[1] = {0u};
  bool ok = true;
  if (p.route) {
    ok = wait_tagged_sent<1>([&](int) { return p.ringt + (lane < 10 ? lane : 0); }, [&](int) { return lane < 10; },
                             lane == 0, p.gen, v);
    if (lane >= 10) v[0] = 0u;
  } else if (lane < 10) {
    v[0] = ((const uint32_t *)p.ring_in)[lane];
  }
#pragma unroll
  for (int w = 0; w < 10; ++w) rw[w] = __builtin_amdgcn_readlane(v[0], w);
  return ok;
}

/* Row pointer of adapter a in table T (lane a holds it): uniform. */
__device__ __forceinline__ const uint16_t *tab_ptr(uint64_t lane_ptr, int a) {
  return (const uint16_t *)aos_shfl64(lane_ptr, a);
}

/* The expand of one module adds coef * S . B over the union's rank rows for the 32 rows at row0:
 * steps (u, j0) in order, four per batch. A batch's 64 S words (4 steps x the token's 16 values)
 * are loaded one per lane (lane 16 k + 8 c + e: step k, values j0 + 8 c + e), tagged and waited
 * for, scaled by the step's coefficient, rounded to bf16, paired, and gathered into the A operands
 * of lanes 0 and 32 with shuffles; the B fragments of the batch load with them. S of union slot
 * u, rank row j is at sbase + a(u) * rpad + j for the x shrink's per-adapter S (by_adapter), at
 * sbase + u * rpad + j for S_h (by union column). */
struct ExpMod {
  uint64_t bptr_lane; /* lane a: adapter a's B (row-major [rows][rpad]) */
  int rpad;
  const uint64_t *sbase;
  bool by_adapter;
  __device__ int nst(const RingUnion &ru) const { return rpad ? ru.U * (rpad >> 4) : 0; }
};

/* The B fragments of batch s0 (steps s0 .. s0 + 3; past nst the last step is reloaded). */
__device__ __forceinline__ void exp_b(const aos_mlp1_params &p, const RingUnion &ru, const ExpMod &m, int row0,
                                      int s0, int nst, int lane, u32x4 (&bf)[4]) {
  const int i = lane & 31, c = lane >> 5;
  const int per = m.rpad >> 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int st = s0 + k < nst ? s0 + k : (nst > 0 ? nst - 1 : 0);
    const int u = per ? st / per : 0, j0 = (st - u * per) * 16;
    const int a = ru.a(u);
    const uint16_t *B = nst > 0 ? tab_ptr(m.bptr_lane, a) : nullptr;
    bf[k] = aos_gld16(B ? B + (size_t)(row0 + i) * m.rpad + j0 + 8 * c : p.zero_row);
  }
}

/* This lane's S word of batch s0 (a valid address always); need: the word belongs to a step of
 * the batch; u: the word's union slot. */
__device__ __forceinline__ const uint64_t *exp_s(const RingUnion &ru, const ExpMod &m, int s0, int nst, int lane,
                                                 bool &need, int &u) {
  const int per = m.rpad >> 4;
  const int k = lane >> 4, hc = (lane >> 3) & 1, e = lane & 7;
  need = s0 + k < nst;
  const int st = need ? s0 + k : s0;
  u = per ? st / per : 0;
  const int j0 = (st - u * per) * 16;
  const int a = ru.a(u);
  return m.sbase + (m.by_adapter ? (size_t)a * m.rpad : (size_t)u * m.rpad) + j0 + 8 * hc + e;
}

/* The MFMAs of batch s0 given this lane's S word (nb steps valid). */
__device__ __forceinline__ void exp_mfma(const RingUnion &ru, uint32_t sword, int u, int nb, int lane,
                                         const u32x4 (&bf)[4], f32x16 &f) {
  const int i = lane & 31, c = lane >> 5;
  const float val = ru.cf(u) * fbits(sword);
  const uint32_t h16 = aos_f32_to_bf16(val);
  const uint32_t nxt = aos_shfl(h16, lane ^ 1);
  const uint32_t packed = h16 | (nxt << 16); /* valid in even lanes: values e, e + 1 */
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int src = 16 * kk + 8 * c;
    u32x4 av;
    av.x = aos_shfl(packed, src);
    av.y = aos_shfl(packed, src + 2);
    av.z = aos_shfl(packed, src + 4);
    av.w = aos_shfl(packed, src + 6);
    if (i != 0) av = u32x4{0u, 0u, 0u, 0u};
    if (kk < nb) {
      f = aos_mfma32(av, bf[kk], f);
      aos_mfma_done(f, av, bf[kk]);
    }
  }
}

/* The expand of one module into f. Returns false when a wait gave up. */
__device__ __forceinline__ bool expand_module(const aos_mlp1_params &p, const RingUnion &ru, const ExpMod &m, int row0,
                                              int lane, f32x16 &f) {
  const int nst = m.nst(ru);
  for (int s0 = 0; s0 < nst; s0 += 4) {
    u32x4 bf[4];
    exp_b(p, ru, m, row0, s0, nst, lane, bf);
    bool need;
    int u;
    const uint64_t *sp = exp_s(ru, m, s0, nst, lane, need, u);
    uint32_t v[1];
    if (!wait_tagged_sent<1>([&](int) { return sp; }, [&](int) { return need; }, need && (lane & 15) == 0, p.gen, v))
      return false;
    exp_mfma(ru, v[0], u, nst - s0 < 4 ? nst - s0 : 4, lane, bf, f);
  }
  return true;
}

/* The expands of two modules (gate and up), their batches loaded and waited for together. */
__device__ __forceinline__ bool expand_pair(const aos_mlp1_params &p, const RingUnion &ru, const ExpMod &m0,
                                            const ExpMod &m1, int row0, int lane, f32x16 &f0, f32x16 &f1) {
  const int n0 = m0.nst(ru), n1 = m1.nst(ru);
  const int nmax = n0 > n1 ? n0 : n1;
  for (int s0 = 0; s0 < nmax; s0 += 4) {
    u32x4 b0[4], b1[4];
    exp_b(p, ru, m0, row0, s0, n0, lane, b0);
    exp_b(p, ru, m1, row0, s0, n1, lane, b1);
    bool need0, need1;
    int u0, u1;
    const uint64_t *sp0 = exp_s(ru, m0, s0, n0, lane, need0, u0);
    const uint64_t *sp1 = exp_s(ru, m1, s0, n1, lane, need1, u1);
    uint32_t v[2];
    if (!wait_tagged_sent<2>([&](int k) { return k ? sp1 : sp0; }, [&](int k) { return k ? need1 : need0; },
                             need0 && (lane & 15) == 0, p.gen, v))
      return false;
    if (s0 < n0) exp_mfma(ru, v[0], u0, n0 - s0 < 4 ? n0 - s0 : 4, lane, b0, f0);
    if (s0 < n1) exp_mfma(ru, v[1], u1, n1 - s0 < 4 ? n1 - s0 : 4, lane, b1, f1);
  }
  return true;
}

/* Even shares of U units over NW waves: wave w holds [w U / NW, (w + 1) U / NW). Unit indices and
 * these products stay in 32 bits (the host keeps U NW below 2^32): a 64-bit division is a long
 * software sequence on this GPU, and these run on the critical path. */
__device__ __forceinline__ uint32_t share_lo(uint32_t w, uint32_t NW, uint32_t U) { return w * U / NW; }

/* The wave holding unit u0 among NW waves sharing U units evenly. */
__device__ __forceinline__ uint32_t wave_of_unit(uint32_t u0, uint32_t NW, uint32_t U) { return ((u0 + 1) * NW - 1) / U; }

/* ---- G waves ---- */

struct GRing {
  u32x4 wa[RD], wb[RD];
  uint32_t sa[RD], sb[RD];
};

__device__ __forceinline__ void g_unit_load(const aos_mlp1_params &p, uint32_t u, int lane, u32x4 &wa, u32x4 &wb,
                                            uint32_t &sa, uint32_t &sb) {
  const int i = lane & 31;
  wa = ((const u32x4 *)p.wg.qt)[(size_t)u * 64 + lane];
  wb = ((const u32x4 *)p.wu.qt)[(size_t)u * 64 + lane];
  sa = p.wg.sb[(size_t)u * 32 + i];
  sb = p.wu.sb[(size_t)u * 32 + i];
}

/* The LoRA expand of gate and up for the 32 rows of gate/up row block rb, published in ex (lanes
 * 0-31: gate, 32-63: up): run ahead of the row block's owner by a wave with nothing else to do
 * before h is ready. */
__device__ __forceinline__ void d_expand(const aos_mlp1_params &p, uint32_t rb, int lane) {
  const int i = lane & 31;
  uint32_t rw[10];
  bool ok = load_ring(p, lane, rw);
  const int n = p.n;
  uint32_t bnd = 0;
  float scl = 0.0f;
  uint64_t pbg = 0, pbu = 0;
  if (lane < n) {
    bnd = p.bound[lane];
    scl = p.scale[lane];
    if (p.tg.rpad) pbg = (uint64_t)p.tg.B[lane];
    if (p.tu.rpad) pbu = (uint64_t)p.tu.B[lane];
  }
  const RingUnion ru = ring_union(rw, n, bnd, scl, lane);
  f32x16 f0 = {}, f1 = {};
  const ExpMod mg{pbg, p.tg.rpad, p.sx, true}, mu{pbu, p.tu.rpad, p.sx + (size_t)n * p.tg.rpad, true};
  ok = ok && expand_pair(p, ru, mg, mu, (int)rb * 32, lane, f0, f1);
  if (!ok) {
    set_timeout(p, lane);
    return;
  }
  const float e0 = f0[0], e1 = f1[0];
  aos_mfma_hold(f0);
  aos_mfma_hold(f1);
  if (lane < 32) {
    tag_store(p.ex + (size_t)rb * 64 + i, ubits(e0), p.gen);
    tag_store(p.ex + (size_t)rb * 64 + 32 + i, ubits(e1), p.gen);
  }
}

/* One 32-column block cb of the h shrink for gate/up row block rb: the A_down fragments (lane
 * (i, c): column cb * 32 + i, rows rb * 32 + 8 c .. + 7 and + 16 .. + 23). */
__device__ __forceinline__ void hshrink_frag(const aos_mlp1_params &p, const RingUnion &ru, uint64_t pad, int cols,
                                             uint32_t rb, int cb, int lane, u32x4 &b0, u32x4 &b1) {
  const int i = lane & 31, c = lane >> 5;
  const int rpd = p.td.rpad;
  const int col = cb * 32 + i;
  const int u = col / rpd, j = col - u * rpd;
  const int a = ru.a(u);
  const uint16_t *A = tab_ptr(pad, a);
  const uint16_t *arow = (col < cols && A) ? A + (size_t)j * p.wd.in + rb * 32 + 8 * c : p.zero_row;
  const int step = (col < cols && A) ? 16 : 0;
  b0 = aos_gld16(arow);
  b1 = aos_gld16(arow + step);
}

/* The owner's epilogue of gate/up row block rb: the handed-on partials with the row block's
 * expand (ex), SwiGLU, h and hpart. own0 / own1: this wave's partial of the row block (gate / up,
 * lanes 0-31). The first two column blocks of A_down load before the waits. */
__device__ __forceinline__ void g_owner(const aos_mlp1_params &p, uint32_t rb, uint32_t gw, float own0, float own1,
                                        int lane) {
  const int i = lane & 31, c = lane >> 5;
  const uint32_t G = p.wg.G;
  const uint32_t U = (uint32_t)p.wg.RB * G, NGW = 4u * p.nwg;
  const uint32_t wf = wave_of_unit(rb * G, NGW, U);
  const int nc = (int)(gw - wf);
  /* the ring, the adapters' flags and A_down row pointers */
  uint32_t rw[10];
  bool ok = load_ring(p, lane, rw);
  const int n = p.n;
  uint32_t bnd = 0;
  uint64_t pad = 0;
  if (lane < n) {
    bnd = p.bound[lane];
    if (p.td.rpad) pad = (uint64_t)p.td.A[lane];
  }
  const RingUnion ru = ring_union(rw, n, bnd, 0.0f, lane);
  const int cols = ru.U * p.td.rpad;
  u32x4 pb[4];
  if (cols > 0) {
    hshrink_frag(p, ru, pad, cols, rb, 0, lane, pb[0], pb[1]);
    hshrink_frag(p, ru, pad, cols, rb, 1, lane, pb[2], pb[3]);
  }
  /* the partials handed on, in wave order (lane i < 32 sums row i of gate and of up), with the
   * expand words of row i (words 16 and 17 of the first batch) */
  float sg = 0.0f, su = 0.0f, eg = 0.0f, eu = 0.0f;
  for (int k0 = 0; ok && (k0 == 0 || k0 < nc); k0 += 8) {
    uint32_t v[18];
    const int cnt = nc - k0 < 8 ? nc - k0 : 8;
    const bool first = k0 == 0;
    ok = wait_tagged_if<18>(
        [&](int k) {
          return k < 16 ? p.gpart + (size_t)(wf + k0 + ((k >> 1) < cnt ? (k >> 1) : 0)) * 64 + 32 * (k & 1) + i
                        : p.ex + (size_t)rb * 64 + 32 * (k & 1) + i;
        },
        [&](int k) { return lane < 32 && (k < 16 ? (k >> 1) < cnt : first); }, p.gen, v);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < cnt) {
        sg += fbits(v[2 * k]);
        su += fbits(v[2 * k + 1]);
      }
    if (first) {
      eg = fbits(v[16]);
      eu = fbits(v[17]);
    }
  }
  if (!ok) {
    set_timeout(p, lane);
    return;
  }
  sg += own0;
  su += own1;
  const float gt = sg + eg;
  const float up = su + eu;
  const float sig = 1.0f / (1.0f + expf(-gt));
  const uint16_t hb = aos_f32_to_bf16((gt * sig) * up);
  if (lane < 32) tag_store(p.htag + rb * 32 + i, hb, p.gen);
  /* this row block's part of the down shrink: hpart[rb][col] = sum over its 32 rows of
   * h[row] A_down(col)[row], col = u * rpad_d + j over the union */
  if (cols == 0) return;
  /* the token's h rows as the A operand: lane (i, c) of step k2 takes rows 16 k2 + 8 c .. + 7 */
  u32x4 ha[2];
  const uint32_t hv = hb;
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    uint32_t r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = aos_shfl(hv, 16 * k2 + 8 * c + e);
    ha[k2].x = i == 0 ? (r[0] | r[1] << 16) : 0u;
    ha[k2].y = i == 0 ? (r[2] | r[3] << 16) : 0u;
    ha[k2].z = i == 0 ? (r[4] | r[5] << 16) : 0u;
    ha[k2].w = i == 0 ? (r[6] | r[7] << 16) : 0u;
  }
  for (int cb = 0; cb * 32 < cols; ++cb) {
    u32x4 b0, b1;
    if (cb < 2) {
      b0 = cb == 0 ? pb[0] : pb[2];
      b1 = cb == 0 ? pb[1] : pb[3];
    } else {
      hshrink_frag(p, ru, pad, cols, rb, cb, lane, b0, b1);
    }
    f32x16 acc = {};
    acc = aos_mfma32(ha[0], b0, acc);
    acc = aos_mfma32(ha[1], b1, acc);
    const int col = cb * 32 + i;
    if (lane < 32 && col < cols) tag_store(p.hpart + rb * p.hc + col, ubits(acc[0]), p.gen);
    aos_mfma_done(acc, ha[0], b0);
    aos_mfma_done(acc, ha[1], b1);
  }
}

/* S_h[col] = sum over the gate/up row blocks of hpart[rb][col], lane l taking rb = l, l + 64, ...
 * in order, then a xor butterfly. */
__device__ __forceinline__ void g_hsum(const aos_mlp1_params &p, int col, int lane) {
  uint32_t rw[10];
  if (!load_ring(p, lane, rw)) {
    set_timeout(p, lane);
    return;
  }
  uint32_t bnd = lane < p.n ? (uint32_t)p.bound[lane] : 0u;
  const RingUnion ru = ring_union(rw, p.n, bnd, 0.0f, lane);
  if (col >= ru.U * p.td.rpad) return;
  const int RB = p.wg.RB;
  float s = 0.0f;
  for (int r0 = 0; r0 < RB; r0 += 64 * 12) {
    uint32_t v[12];
    const int rem = (RB - r0 - lane + 63) / 64;
    const int cnt = rem < 0 ? 0 : (rem > 12 ? 12 : rem);
    if (!wait_tagged<12, 8>(
            [&](int k) { return p.hpart + (size_t)(k < cnt ? r0 + lane + 64 * k : 0) * p.hc + col; }, cnt, p.gen, v)) {
      set_timeout(p, lane);
      return;
    }
#pragma unroll
    for (int k = 0; k < 12; ++k)
      if (k < cnt) s += fbits(v[k]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s = s + aos_shfl_f(s, lane ^ o);
  if (lane == 0) tag_store(p.sh + col, ubits(s), p.gen);
}

/* ---- D waves ---- */

/* Router prior of adapter a (one wave): the dot product of the token's features with router
 * weight row a, in the order of route_features_block (lane l sums elements 256 k + 4 l + e with
 * fused multiply-adds, then a xor butterfly); published tagged. The wave of the last adapter then
 * collects every prior, routes the token (route_one) and publishes the ring's words. */
__device__ __forceinline__ void d_route(const aos_mlp1_params &p, int a, int lane) {
  const aos_route_params &rp = p.rp;
  __shared__ float prl[AOS_MLP1_MAXN];
  /* the order of route_features_block's dot products: lane l sums elements 256 k + 4 l + e (k
   * ascending, e = 0..3) with fused multiply-adds, then the d % 256 tail, then a xor butterfly;
   * the features come from memory, eight 256-element chunks loaded at a time */
  const int nk = rp.d >> 8, tail = rp.d & 255;
  const float *wr = rp.router_w + (size_t)a * rp.d;
  const float4 *w4 = (const float4 *)wr, *f4 = (const float4 *)rp.features;
  float acc = 0.0f;
  for (int k0 = 0; k0 < nk; k0 += 8) {
    float4 wv[8], fv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = k0 + j < nk ? k0 + j : nk - 1;
      wv[j] = w4[k * 64 + lane];
      fv[j] = f4[k * 64 + lane];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (k0 + j < nk) {
        acc = fmaf(wv[j].x, fv[j].x, acc);
        acc = fmaf(wv[j].y, fv[j].y, acc);
        acc = fmaf(wv[j].z, fv[j].z, acc);
        acc = fmaf(wv[j].w, fv[j].w, acc);
      }
    }
  }
  if (4 * lane < tail) {
    const float4 fv = f4[nk * 64 + lane], wt = w4[nk * 64 + lane];
    acc = fmaf(wt.x, fv.x, acc);
    acc = fmaf(wt.y, fv.y, acc);
    acc = fmaf(wt.z, fv.z, acc);
    acc = fmaf(wt.w, fv.w, acc);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc = acc + aos_shfl_f(acc, lane ^ o);
  const float v = acc;
  if (lane == 0) {
    tag_store(p.pri + a, ubits(v), p.gen);
    if (rp.priors_out) rp.priors_out[a] = v;
  }
  if (a != rp.n - 1) return;
  RouteMeta meta = route_meta<false>(rp, lane);
  uint32_t pv[1];
  if (!wait_tagged<1>([&](int) { return p.pri + (lane < rp.n ? lane : 0); }, lane < rp.n ? 1 : 0, p.gen, pv)) {
    set_timeout(p, lane);
    return;
  }
  if (lane < rp.n) prl[lane] = fbits(pv[0]);
  wave_lds_sync();
  route_one<true, false>(rp, prl, 0, lane, &meta);
  aos_mem_wait();
  if (lane < 10) {
    const uint32_t w = __hip_atomic_load((const uint32_t *)rp.rings + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    tag_store(p.ringt + lane, w, p.gen);
  }
}

/* x shrink piece q: tile q / x_ks (32 columns of gate's n * rpad_g, then of up's), K piece
 * q % x_ks; S partials for the token go out tagged, and the wave of a tile's last piece sums the
 * pieces in order into sx. x comes from memory (this runs before x is staged in LDS). */
__device__ __forceinline__ void d_xshrink(const aos_mlp1_params &p, int q, int lane) {
  const int i = lane & 31, c = lane >> 5;
  const int tile = q / p.x_ks, kp = q - tile * p.x_ks;
  const bool up = tile >= p.x_tiles_g;
  const uint16_t *const *tabA = up ? p.tu.A : p.tg.A;
  const int rpad = up ? p.tu.rpad : p.tg.rpad;
  const int ncol = p.n * rpad;
  const int col = (up ? tile - p.x_tiles_g : tile) * 32 + i;
  const int G = p.wg.G, in = p.wg.in;
  const int a = col / (rpad ? rpad : 1), j = col - a * rpad;
  const uint16_t *A = col < ncol ? tabA[a] : nullptr;
  const uint16_t *arow = A ? A + (size_t)j * in + 32 * c : p.zero_row;
  const int gstep = A ? 64 : 0, sstep = A ? 8 : 0;
  const int g0 = kp * G / p.x_ks, g1 = (kp + 1) * G / p.x_ks;
  f32x16 acc = {};
  /* the token's x as the A operand (lanes 0 and 32; the rest zero), loaded with the A rows */
  const uint16_t *xrow = i == 0 ? p.x + 32 * c : p.zero_row;
  const int xstep = i == 0 ? 64 : 0, xs8 = i == 0 ? 8 : 0;
  for (int g = g0; g < g1; g += 2) {
    u32x4 w[2][4], xv[2][4];
#pragma unroll
    for (int gg = 0; gg < 2; ++gg)
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int ge = g + gg < g1 ? g + gg : g1 - 1;
        w[gg][st] = aos_gld16(arow + (size_t)ge * gstep + sstep * st);
        xv[gg][st] = aos_gld16(xrow + (size_t)ge * xstep + xs8 * st);
      }
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      if (g + gg >= g1) continue;
      u32x4 xa[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        xa[st] = xv[gg][st];
        acc = aos_mfma32(xa[st], w[gg][st], acc);
      }
#pragma unroll
      for (int st = 0; st < 4; ++st) aos_mfma_done(acc, xa[st], w[gg][st]);
    }
  }
  uint64_t *sp = p.spart + (size_t)tile * p.x_ks * 32;
  const float mine = acc[0];
  aos_mfma_hold(acc);
  if (lane < 32) tag_store(sp + (size_t)kp * 32 + i, ubits(mine), p.gen);
  if (kp != p.x_ks - 1) return;
  /* the pieces handed on: lanes 0-31 sum the first half in order, lanes 32-63 the rest (the same
   * columns), then first half + second half + this wave's own */
  const int np = p.x_ks - 1, half = (np + 1) / 2;
  const int m0 = c ? half : 0, mc = c ? np - half : half;
  float s = 0.0f;
  for (int k0 = 0; k0 < half; k0 += 16) {
    uint32_t v[16];
    int cnt = mc - k0;
    cnt = cnt < 0 ? 0 : (cnt > 16 ? 16 : cnt);
    if (!wait_tagged<16>([&](int k) { return sp + (size_t)(m0 + k0 + (k < cnt ? k : 0)) * 32 + i; }, cnt, p.gen, v)) {
      set_timeout(p, lane);
      return;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k)
      if (k < cnt) s += fbits(v[k]);
  }
  const float second = aos_shfl_f(s, (i + 32) & 63);
  s = (s + second) + mine;
  if (lane < 32 && col < ncol) tag_store(p.sx + (up ? (size_t)p.n * p.tg.rpad : 0) + col, ubits(s), p.gen);
}

/* The owner's epilogue of down row block rb: the partials handed on, its own, the LoRA expand of
 * S_h, y. */
__device__ __forceinline__ void d_owner(const aos_mlp1_params &p, uint32_t rb, int dw, float own, int lane) {
  const int i = lane & 31;
  const uint32_t Gd = p.wd.G;
  const uint32_t UD = (uint32_t)p.wd.RB * Gd;
  /* the D wave holding the row block's first unit: its workgroup, then its share within it */
  const uint32_t u0 = rb * Gd;
  const uint32_t wgf = wave_of_unit(u0, p.nwg, UD);
  const uint32_t dlo = share_lo(wgf, p.nwg, UD), nd = share_lo(wgf + 1, p.nwg, UD) - dlo;
  int kf = 3;
  while (kf > 0 && dlo + (uint32_t)kf * nd / 4 > u0) --kf;
  const int wf = (int)wgf * 4 + kf;
  const int nc = (int)(dw - wf);
  uint32_t rw[10];
  bool ok = load_ring(p, lane, rw);
  const int n = p.n;
  uint32_t bnd = 0;
  float scl = 0.0f;
  uint64_t pbd = 0;
  if (lane < n) {
    bnd = p.bound[lane];
    scl = p.scale[lane];
    if (p.td.rpad) pbd = (uint64_t)p.td.B[lane];
  }
  /* the partials handed on: lanes 0-31 sum the first half of the waves, lanes 32-63 the rest (the
   * same rows), each in wave order, then first half + second half + this wave's own */
  const int half = (nc + 1) / 2;
  const int c = lane >> 5;
  const int mw0 = wf + (c ? half : 0);
  const int mcnt = c ? nc - half : half;
  float sum = 0.0f;
  for (int k0 = 0; k0 < half && ok; k0 += 12) {
    uint32_t v[12];
    int cnt = mcnt - k0;
    cnt = cnt < 0 ? 0 : (cnt > 12 ? 12 : cnt);
    ok = wait_tagged<12>([&](int k) { return p.dpart + (size_t)(mw0 + k0 + (k < cnt ? k : 0)) * 32 + i; }, cnt, p.gen,
                         v);
#pragma unroll
    for (int k = 0; k < 12; ++k)
      if (k < cnt) sum += fbits(v[k]);
  }
  if (!ok) {
    set_timeout(p, lane);
    return;
  }
  const float second = aos_shfl_f(sum, (i + 32) & 63);
  sum = (sum + second) + own;
  const RingUnion ru = ring_union(rw, n, bnd, scl, lane);
  f32x16 f = {};
  const ExpMod md{pbd, p.td.rpad, p.sh, false};
  if (!expand_module(p, ru, md, (int)rb * 32, lane, f)) {
    set_timeout(p, lane);
    return;
  }
  const float yv = sum + f[0];
  aos_mfma_hold(f);
  if (lane < 32) p.y[rb * 32 + i] = aos_f32_to_bf16(yv);
}

template <int MAXDU>
__device__ __forceinline__ void d_main(const aos_mlp1_params &p, int wgi, int k, int lane, unsigned char *smem,
                                       uint32_t *x_done) {
  const int i = lane & 31, c = lane >> 5;
  const int dw = wgi * 4 + k;
  /* producer work first: its loads would otherwise queue behind this wave's LDS loads */
  const int nr = p.route ? p.rp.n : 0;
  const int rw4 = (nr + 3) / 4 * 4; /* D waves taken by the router */
  /* the host leaves at least RB_gate waves after the producers: one gate/up row block's expand each */
  const int nprod = rw4 + (p.x_tiles_g + p.x_tiles_u) * p.x_ks;
  if (dw < nr) {
    d_route(p, dw, lane);
  } else if (dw >= rw4 && dw < nprod) {
    d_xshrink(p, dw - rw4, lane);
  } else if (dw >= nprod && dw - nprod < p.wg.RB) {
    d_expand(p, (uint32_t)(dw - nprod), lane);
  }
  if (lane == 0) atomicAdd(x_done, 1u); /* this wave is done with the staged x */

  /* this wave's down units: its share of the workgroup's, which the G wave of the same index
   * loads into LDS */
  const uint32_t Gd = p.wd.G;
  const uint32_t UD = (uint32_t)p.wd.RB * Gd;
  const uint32_t dlo = share_lo(wgi, p.nwg, UD), nd = share_lo(wgi + 1, p.nwg, UD) - dlo;
  const uint32_t lo = dlo + (uint32_t)k * nd / 4, hi = dlo + (uint32_t)(k + 1) * nd / 4;
  const int nu = (int)(hi - lo);
  /* unit lo + j: group g0 + j (wrapping once at most: nu <= Gd), LDS slot lo - dlo + j (the
   * workgroup's units are consecutive and at most Gd, so their groups are distinct) */
  const uint32_t rb0 = lo / Gd;
  const int g0 = (int)(lo - rb0 * Gd), s0 = (int)(lo - dlo);
  auto grp = [&](int j) { const int g = g0 + j; return g >= (int)Gd ? g - (int)Gd : g; };
  uint32_t sbv[MAXDU];
#pragma unroll
  for (int j = 0; j < MAXDU; ++j) sbv[j] = j < nu ? p.wd.sb[(size_t)(lo + j) * 32 + i] : 0u;

  /* h for this wave's groups (tagged), once h is complete there */
  static_assert(2 * MAXDU <= 64, "one sentinel lane per (unit, half)");
  uint32_t hv[MAXDU];
  /* first one word per (group, owner): lane 2j + s polls the first word of unit j's half s (the
   * gate/up row block 2g + s writes the 32 words of that half with one store) */
  const int sj = lane >> 1;
  const bool sok = wait_sentinel(p.htag + (size_t)grp(sj < nu ? sj : 0) * 64 + 32 * (lane & 1), sj < nu, p.gen);
  const bool hok = sok && wait_tagged<MAXDU>(
      [&](int j) { return p.htag + (size_t)grp(j < nu ? j : 0) * 64 + lane; }, nu, p.gen, hv);
  if (!hok) set_timeout(p, lane);
  /* wait until every wave of the workgroup is done with the staged x and the G waves' loads of the
   * down units have landed in LDS, then stage h in x's place: unit j's group at slot s0 + j, bf16
   * at 128 + slot * 128, the two 32-element half sums after the workgroup's slots (lane 2j + c
   * sums half c of unit j, in element order) */
  {
    const uint32_t limit = aos_spin_limit();
    uint32_t spins = 0;
    while (__hip_atomic_load(x_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 8u) {
      if (spins++ >= limit) {
        set_timeout(p, lane);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  }
  uint16_t *hl = (uint16_t *)(smem + 128);
  float *hs = (float *)(smem + 128 + (size_t)p.d_units_max * 128);
#pragma unroll
  for (int j = 0; j < MAXDU; ++j)
    if (j < nu) hl[(s0 + j) * 64 + lane] = (uint16_t)(hok ? hv[j] : 0u);
  wave_lds_sync();
  if (sj < nu) {
    const u32x4 *src = (const u32x4 *)(smem + 128 + (size_t)(s0 + sj) * 128 + 64 * (lane & 1));
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 v = src[q];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
        s += __builtin_bit_cast(float, w << 16);
        s += __builtin_bit_cast(float, w & 0xffff0000u);
      }
    }
    hs[(s0 + sj) * 2 + (lane & 1)] = s;
  }
  wave_lds_sync();

  /* the partial sums of this wave's units: at most two row blocks */
  const uint32_t qmask = aos_q4_mask(), qexp = aos_q4_exp();
  const uint32_t b = (rb0 + 1) * Gd < hi ? (rb0 + 1) * Gd : hi;
  const int jb = (int)(b - lo);
  float acc = 0.0f, accA = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXDU; ++j) {
    if (j >= nu) continue;
    if (j == jb) {
      accA = acc;
      acc = 0.0f;
    }
    const int slot = s0 + j;
    const u32x4 w = *(const u32x4 *)(smem + p.doff + slot * 1024 + lane * 16);
    const int abase = i == 0 ? 128 + slot * 128 + 64 * c : 0;
    f32x16 t = {};
    u32x4 av[4], bv[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      av[st] = *(const u32x4 *)(smem + abase + 16 * st);
      bv[st] = aos_q4_magic(w[st], qmask, qexp);
      t = aos_mfma32(av[st], bv[st], t);
    }
    const float s = aos_f16_to_f32(sbv[j] & 0xffffu), bb = aos_f16_to_f32(sbv[j] >> 16);
    const float bp = fmaf(-128.0f, s, bb);
    const float sx = hs[slot * 2] + hs[slot * 2 + 1];
    acc = fmaf(s, t[0], fmaf(bp, sx, acc));
#pragma unroll
    for (int st = 0; st < 4; ++st) aos_mfma_done(t, av[st], bv[st]);
  }
  if (nu == 0) { /* an empty share hands on zero (owners count every wave between them) */
    if (lane < 32) tag_store(p.dpart + (size_t)dw * 32 + i, 0u, p.gen);
    return;
  }
  const bool crossing = jb < nu;
  const float p0 = crossing ? accA : acc;
  const bool owned0 = b == (rb0 + 1) * Gd;
  /* hand on the piece this wave does not own (at most one) */
  if (crossing || !owned0) {
    const float hand = crossing ? acc : p0;
    if (lane < 32) tag_store(p.dpart + (size_t)dw * 32 + i, ubits(hand), p.gen);
  }
  if (owned0) d_owner(p, rb0, dw, p0, lane);
}

__device__ __forceinline__ bool g_owns(uint32_t gw, uint32_t NGW, uint32_t U, uint32_t G) {
  const uint32_t lo = share_lo(gw, NGW, U), hi = share_lo(gw + 1, NGW, U);
  if (hi <= lo) return false;
  const uint32_t rb0 = lo / G;
  const uint32_t b = (rb0 + 1) * G < hi ? (rb0 + 1) * G : hi;
  return b == (rb0 + 1) * G;
}

__global__ void __launch_bounds__(512, 4) aos_mlp1_kernel(aos_mlp1_params p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ uint32_t x_done, x_staged;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wgi = blockIdx.x;
  const int i = lane & 31, c = lane >> 5;
  const uint32_t G = p.wg.G;
  const uint32_t U = (uint32_t)p.wg.RB * G, NGW = 4u * p.nwg;
  const uint32_t gw = (uint32_t)wgi * 4 + (wave & 3);
  const uint32_t lo = share_lo(gw, NGW, U), hi = share_lo(gw + 1, NGW, U);
  const int n = wave < 4 ? (int)(hi - lo) : 0;

  /* the LDS counters and the zero block, before any wave uses them; then the D waves go their own
   * way (they read x from memory, so they never wait for its staging) */
  if (tid == 0) {
    x_done = 0u;
    x_staged = 0u;
  }
  if (tid < 32) ((uint32_t *)smem)[tid] = 0u;
  aos_gemv::lds_barrier();
  if (wave >= 4) {
    d_main<AOS_MLP1_MAX_DU>(p, wgi, wave - 4, lane, smem, &x_done);
    return;
  }

  /* G waves: x first (the LDS stores below wait for these loads only), then prime the ring (units
   * past the share reload the last one; an empty share reloads unit lo, which exists) */
  const int nx = G * 8;
  u32x4 xv0 = {}, xv1 = {};
  if (tid < nx) xv0 = ((const u32x4 *)p.x)[tid];
  if (tid + 256 < nx) xv1 = ((const u32x4 *)p.x)[tid + 256];
  GRing r;
#pragma unroll
  for (int d = 0; d < RD; ++d) {
    const uint32_t u = d < n ? lo + d : (n > 0 ? hi - 1 : lo);
    g_unit_load(p, u, lane, r.wa[d], r.wb[d], r.sa[d], r.sb[d]);
  }
  /* x -> LDS, then the group half sums, each step closed by the four G waves' LDS counter */
  for (int idx = tid + 512; idx < nx; idx += 256) *(u32x4 *)(smem + 128 + idx * 16) = ((const u32x4 *)p.x)[idx];
  if (tid < nx) *(u32x4 *)(smem + 128 + tid * 16) = xv0;
  if (tid + 256 < nx) *(u32x4 *)(smem + 128 + (tid + 256) * 16) = xv1;
  g_sync(p, &x_staged, 4u, lane);
  float *xs = (float *)(smem + 128 + (size_t)G * 128);
  for (int idx = tid; idx < (int)G * 2; idx += 256) {
    const u32x4 *src = (const u32x4 *)(smem + 128 + idx * 64);
    const u32x4 v0 = src[0], v1 = src[1], v2 = src[2], v3 = src[3];
    const uint32_t w[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                            v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
    float s = 0.0f; /* the 32 elements in order */
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s += __builtin_bit_cast(float, w[e] << 16);
      s += __builtin_bit_cast(float, w[e] & 0xffff0000u);
    }
    xs[idx] = s;
  }
  g_sync(p, &x_staged, 8u, lane);

  /* G waves: stream the share, at most two row blocks (pieces split at unit b) */
  const uint32_t qmask = aos_q4_mask(), qexp = aos_q4_exp();
  const uint32_t rb0 = lo / G;
  const uint32_t b = (rb0 + 1) * G < hi ? (rb0 + 1) * G : hi;
  const int jb = (int)(b - lo);
  const int g0 = (int)(lo - rb0 * G);
  const int xbase = i == 0 ? 128 + 64 * c : 0, xmult = i == 0 ? 128 : 0;
  /* the down units of the workgroup's D wave with this wave's index go into LDS from here, one
   * per gate/up unit streamed (buffer_load ... lds), so the down bytes flow with the gate/up
   * stream on every CU instead of arriving as one burst */
  const uint32_t Gd = p.wd.G, UD = (uint32_t)p.wd.RB * Gd;
  const uint32_t dlo = share_lo(wgi, p.nwg, UD), nd = share_lo(wgi + 1, p.nwg, UD) - dlo;
  const uint32_t mlo = dlo + (uint32_t)wave * nd / 4;
  const int m = (int)(dlo + (uint32_t)(wave + 1) * nd / 4 - mlo);
  const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)p.wd.qt, (short)0, (int)((size_t)UD * 1024 < 0x7fffffff ? (size_t)UD * 1024 : 0x7fffffff), 0x00020000);
  auto dma = [&](int j) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        drs, (__attribute__((address_space(3))) void *)(smem + p.doff + (mlo - dlo + j) * 1024), 16,
        (int)(((mlo + j) * 64 + lane) * 16), 0, 0, 0);
  };
  float acc0[1] = {0.0f}, acc1[1] = {0.0f}, a0A = 0.0f, a1A = 0.0f;
  for (int base = 0; base < n; base += RD) {
#pragma unroll
    for (int d = 0; d < RD; ++d) {
      const int j = base + d;
      if (j < n) {
        if (j == jb) {
          a0A = acc0[0];
          a1A = acc1[0];
          acc0[0] = 0.0f;
          acc1[0] = 0.0f;
        }
        int gl = g0 + j;
        gl = gl >= (int)G ? gl - (int)G : gl;
        f32x16 t0 = {}, t1 = {};
        u32x4 a[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) a[st] = *(const u32x4 *)(smem + xbase + (size_t)gl * xmult + 16 * st);
        u32x4 bg[4], bu[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          bg[st] = aos_q4_magic(r.wa[d][st], qmask, qexp);
          bu[st] = aos_q4_magic(r.wb[d][st], qmask, qexp);
          t0 = aos_mfma32(a[st], bg[st], t0);
          t1 = aos_mfma32(a[st], bu[st], t1);
        }
        aos_gemv::apply_group<1>(t0, r.sa[d], xs, G, gl, 1, lane, acc0);
        aos_gemv::apply_group<1>(t1, r.sb[d], xs, G, gl, 1, lane, acc1);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          aos_mfma_done(t0, a[st], bg[st]);
          aos_mfma_done(t1, a[st], bu[st]);
        }
      }
      const int jn = j + RD < n ? j + RD : n - 1;
      g_unit_load(p, lo + (jn > 0 ? jn : 0), lane, r.wa[d], r.wb[d], r.sa[d], r.sb[d]);
      if (j < m) dma(j);
    }
  }
  for (int j = n; j < m; ++j) dma(j);
  if (n > 0) {
    const bool crossing = jb < n;
    const float p0g = crossing ? a0A : acc0[0], p0u = crossing ? a1A : acc1[0];
    const bool owned0 = b == (rb0 + 1) * G;
    if (crossing || !owned0) {
      const float hg = crossing ? acc0[0] : p0g, hu = crossing ? acc1[0] : p0u;
      if (lane < 32) {
        tag_store(p.gpart + (size_t)gw * 64 + i, ubits(hg), p.gen);
        tag_store(p.gpart + (size_t)gw * 64 + 32 + i, ubits(hu), p.gen);
      }
    }
    if (owned0) g_owner(p, rb0, gw, p0g, p0u, lane);
  } else { /* an empty share hands on zero (owners count every wave between them) */
    tag_store(p.gpart + (size_t)gw * 64 + lane, 0u, p.gen);
  }
  /* this wave's down units are in LDS (and it is long done with the staged x): tell the D waves */
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if (lane == 0) atomicAdd(&x_done, 1u);
  /* S_h column wgi (when the h shrink has that many columns): the last G wave of the workgroup
   * that owns no row block */
  if (wgi < p.hc) {
    int summer = -1;
    for (int k = 3; k >= 0 && summer < 0; --k)
      if (!g_owns((uint32_t)wgi * 4 + k, NGW, U, G)) summer = k;
    if (summer == wave) g_hsum(p, wgi, lane);
  }
}

}  // namespace

extern "C" int aos_launch_mlp1(const aos_mlp1_params *p, const aos_launch_ctx *ctx) {
  if (!p->gen || p->nwg < 1 || p->lds_bytes > AOS_MLP1_LDS_MAX || p->n > AOS_MLP1_MAXN)
    return (int)hipErrorInvalidValue;
  /* dynamic LDS above 64 KiB must be allowed once per device */
  static uint64_t allowed = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return (int)hipErrorInvalidValue;
  if (!(allowed >> dev & 1u)) {
    const hipError_t e =
        hipFuncSetAttribute((const void *)aos_mlp1_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, AOS_MLP1_LDS_MAX);
    if (e != hipSuccess) return (int)e;
    allowed |= 1ull << dev;
  }
  AOS_LAUNCH(ctx, aos_mlp1_kernel, dim3(p->nwg), dim3(512), (size_t)p->lds_bytes, *p);
  return (int)hipGetLastError();
}

AOS_DEFINE_SPIN_SETTER(aos_spin_setter_mlp1)
