/*
 * aoship_device.h — device-side types and helpers shared by the gfx950 kernels.
 *
 * Matrix-core fragments use v_mfma_f32_32x32x16_bf16. For an MFMA step, lane l = i + 32 c
 * (i in 0..31, c in 0..1) supplies 8 consecutive K elements for row/column i, half c. The
 * accumulator holds C[m][n] with n = l % 32 and m = 8 (v / 4) + 4 (l / 32) + v % 4 for
 * register v in 0..15.
 */
#ifndef AOSHIP_DEVICE_H
#define AOSHIP_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aoship_internal.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define AOS_WAVE 64

__device__ __forceinline__ f32x16 aos_mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

/* MFMA register lifetimes. An MFMA reads its A and B operands and writes all 16 result registers
 * some cycles after it issues, later still when other waves' MFMAs occupy the SIMD's matrix core.
 * The compiler (ROCm 7.2, gfx950) does not always allow for that: measured in the one-token MLP
 * launch, (1) a VALU write into a result register of an in-flight 32x32x16 MFMA that the kernel
 * never reads (at one token only register 0 of the 16 holds a token) was overwritten by the MFMA's
 * write-back, and (2) a VALU write into the A operand registers of the MFMA issued just before it
 * reached that MFMA; both gave deterministic wrong outputs only when other waves issued MFMAs on the
 * same SIMD, and correct ones when the same code ran alone. The rule kept here: the registers of an
 * MFMA's operands and of its whole result stay reserved until an instruction has read the result
 * (which waits for the MFMA to complete). aos_mfma_hold(t), placed after the instructions that
 * consume t, reads t[0] and passes all 16 registers to an empty asm statement; aos_mfma_done(t, a,
 * b) does the same and keeps the operands a and b as well. Result holds cost no registers and are
 * used wherever fewer than 16 result registers are read. Operand holds are used in the one-token
 * MLP launch, where (2) was measured; in the streaming GEMV and shrink loops they would keep 32-48
 * more registers live (three waves per SIMD to two, the 7B gate/up GEMV 25 to 34 us), and those
 * kernels' outputs are checked run to run and against the oracle by the GPU tests instead. */
__device__ __forceinline__ void aos_mfma_hold(const f32x16 &t) {
  float u = t[0];
  asm volatile("" : "+v"(u) : "v"(t));
}

__device__ __forceinline__ void aos_mfma_done(const f32x16 &t, const u32x4 &a, const u32x4 &b) {
  float u = t[0];
  asm volatile("" : "+v"(u) : "v"(t), "v"(a), "v"(b));
}

/* Token (row of the MFMA M dimension) held by accumulator register v in lane l. */
__device__ __forceinline__ int aos_acc_m(int v, int lane) {
  return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

__device__ __forceinline__ float aos_bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}

/* float32 -> bfloat16, round to nearest even (NaN kept quiet). */
__device__ __forceinline__ uint16_t aos_f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float aos_f16_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

/* Four packed bfloat16 pairs (128 + q) from one nibble-shuffled weight word: register p holds
 * (q[2p], q[2p+1]) of the original MLX word as bf16 values 128 + q (exact). One shift and one
 * v_and_or_b32 per register; the mask lives in an SGPR and the exponent pattern in a VGPR
 * (gfx950's VOP3 encoding takes no literal operands). */
__device__ __forceinline__ uint32_t aos_and_or(uint32_t a, uint32_t smask, uint32_t vmagic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(smask), "v"(vmagic));
  return r;
}

__device__ __forceinline__ u32x4 aos_q4_magic(uint32_t w, uint32_t smask, uint32_t vmagic) {
  u32x4 r;
  r.x = aos_and_or(w, smask, vmagic);
  r.y = aos_and_or(w >> 4, smask, vmagic);
  r.z = aos_and_or(w >> 8, smask, vmagic);
  r.w = aos_and_or(w >> 12, smask, vmagic);
  return r;
}

/* Uniform (SGPR) copies of the extraction constants. */
__device__ __forceinline__ uint32_t aos_q4_mask() { return __builtin_amdgcn_readfirstlane(0x000F000Fu); }
__device__ __forceinline__ uint32_t aos_q4_exp() { return 0x43004300u; }

/* 16-byte load through the global address space. Pointers read from tables (adapter rows, the
 * union's B pointers) are otherwise generic, and a generic (flat) load counts against the LDS
 * counter as well: every later wait for an LDS access would then also wait for it. */
__device__ __forceinline__ u32x4 aos_gld16(const void *p) {
  return *(const __attribute__((address_space(1))) u32x4 *)p;
}

/* A pointer stored in global memory (a table), loaded through the global address space. */
__device__ __forceinline__ const uint16_t *aos_gld_ptr(const void *p) {
  return (const uint16_t *)*(const __attribute__((address_space(1))) uint64_t *)p;
}

__device__ __forceinline__ uint32_t aos_shfl(uint32_t v, int src_lane) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane << 2, (int)v);
}

__device__ __forceinline__ float aos_shfl_f(float v, int src_lane) {
  return __builtin_bit_cast(float, aos_shfl(__builtin_bit_cast(uint32_t, v), src_lane));
}

__device__ __forceinline__ uint64_t aos_shfl64(uint64_t v, int src_lane) {
  uint32_t lo = aos_shfl((uint32_t)v, src_lane);
  uint32_t hi = aos_shfl((uint32_t)(v >> 32), src_lane);
  return ((uint64_t)hi << 32) | lo;
}

/* Cross-workgroup hand-over without cache flushes.
 *
 * Payload: every value another workgroup reads is stored with aos_publish (an agent-scope
 * relaxed atomic store, global_store with sc1: it is written through the XCD's L2 to the
 * device-coherent level) and read with aos_collect (agent-scope relaxed atomic load, sc1: it is
 * not served from a possibly stale line of another XCD's L2).
 *
 * Ordering: the producing wave waits until its payload stores are acknowledged (s_waitcnt
 * vmcnt(0), which on gfx9 counts stores as well) before the store or atomic that signals them;
 * the consumer issues its payload loads only after the load that observed the signal has
 * returned and been compared (a wave issues memory instructions in program order, and the
 * loop's exit branch depends on that value). Both waits are volatile asm with a memory clobber,
 * so the compiler moves no memory access across them either. Agent-scope release/acquire
 * fences would give the same guarantee by writing back and invalidating the whole L2 of the
 * XCD, which costs more than the hand-over itself.
 *
 * Signals are generation-stamped: a launch that hands over data gets a generation number
 * (nonzero, new per call of its layer) and raises flags to that value; a consumer waits for
 * equality, so a flag left over from an earlier call, or raised late by a producer whose
 * consumer gave up, never satisfies a later call's wait. Arrival counters are reset by their
 * last arriver. */
__device__ __forceinline__ void aos_publish(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float aos_collect(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Wait until this wave's earlier loads and stores are complete; a compiler barrier as well. */
__device__ __forceinline__ void aos_mem_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

/* Compiler barrier only (no instruction). */
__device__ __forceinline__ void aos_compiler_barrier() { asm volatile("" ::: "memory"); }

/* Wait for this wave's published stores, then count the arrival (call from one lane).
 * Returns the previous count. */
__device__ __forceinline__ uint32_t aos_arrive(uint32_t *ctr) {
  aos_mem_wait();
  const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  aos_compiler_barrier();
  return old;
}

/* Reset a counter for the next launch (the last arriver's job). */
__device__ __forceinline__ void aos_reset(uint32_t *ctr) {
  __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Arrival idx of n (one lane per workgroup) on the counter lines ctr (AOS_ARRIVE_WORDS(n) words,
 * zero between launches): true for the last of the n, which has then reset every counter. Each
 * arrival first waits for its wave's stores, so when the last returns, the payload of all n is
 * complete. */
__device__ __forceinline__ bool aos_arrive_tree(uint32_t *ctr, uint32_t idx, uint32_t n) {
  if (n <= AOS_ARRIVE_GROUP) {
    if (aos_arrive(ctr) != n - 1u) return false;
    aos_reset(ctr);
    return true;
  }
  const uint32_t g = idx / AOS_ARRIVE_GROUP, ng = (n + AOS_ARRIVE_GROUP - 1u) / AOS_ARRIVE_GROUP;
  const uint32_t gsize = n - g * AOS_ARRIVE_GROUP < AOS_ARRIVE_GROUP ? n - g * AOS_ARRIVE_GROUP : AOS_ARRIVE_GROUP;
  uint32_t *gc = ctr + (size_t)(1u + g) * AOS_ARRIVE_STRIDE;
  if (aos_arrive(gc) != gsize - 1u) return false;
  aos_reset(gc);
  if (aos_arrive(ctr) != ng - 1u) return false;
  aos_reset(ctr);
  return true;
}

/* Raise a generation flag once this wave's payload stores are complete. */
__device__ __forceinline__ void aos_raise(uint32_t *flag, uint32_t gen) {
  aos_mem_wait();
  __hip_atomic_store(flag, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* The bound of every wait below, in polls: 2^24 (about a second) unless the host sets another
 * value (aoship_internal_set_spin_limit, per device). With 0 every wait gives up before its first
 * poll, so that a test can drive every give-up path while every kernel still ends normally. Each
 * translation unit holds its own copy of the variable (internal linkage) and defines a host setter
 * for it with AOS_DEFINE_SPIN_SETTER; the library's setter calls all of them. */
#define AOS_SPIN_LIMIT_DEFAULT (1u << 24)
/* constant memory: waits read it with a scalar load through the constant cache, not with a vector
 * load that would queue behind the launch's streaming loads before every wait */
static __constant__ uint32_t aos_spin_limit_dev = AOS_SPIN_LIMIT_DEFAULT;
#define AOS_DEFINE_SPIN_SETTER(name)                                                        \
  extern "C" int name(uint32_t polls) {                                                     \
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(aos_spin_limit_dev), &polls, sizeof(polls)); \
  }

__device__ __forceinline__ uint32_t aos_spin_limit() { return aos_spin_limit_dev; }

/* Bounded wait (one lane) until *flag == gen. Returns false when it gave up (after about a
 * second at the default bound). The payload loads that follow are not moved above the wait. */
__device__ __forceinline__ bool aos_wait_gen(const uint32_t *flag, uint32_t gen) {
  const uint32_t limit = aos_spin_limit();
  uint32_t spins = 0;
  bool ok = true;
  while (true) {
    if (spins++ >= limit) {
      ok = false;
      break;
    }
    if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) break;
    __builtin_amdgcn_s_sleep(2);
  }
  aos_compiler_barrier();
  return ok;
}

/* Bounded wait by one wave until each of the n flag lines (32 words apart) equals gen: lane l
 * polls lines l, l + 64, ... Returns false (uniformly) when it gave up. The loads that follow
 * are not moved above the wait. */
__device__ __forceinline__ bool aos_wait_lines(const uint32_t *lines, int n, uint32_t gen, int lane) {
  const uint32_t limit = aos_spin_limit();
  uint32_t spins = 0;
  for (int base = 0; base < n; base += 64) {
    const int i = base + lane;
    const uint32_t *f = lines + (size_t)(i < n ? i : 0) * 32;
    while (true) {
      if (spins++ >= limit) {
        aos_compiler_barrier();
        return false;
      }
      const uint32_t v = i < n ? __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : gen;
      if (__ballot(v != gen) == 0ull) break;
      __builtin_amdgcn_s_sleep(2);
    }
  }
  aos_compiler_barrier();
  return true;
}

#endif
