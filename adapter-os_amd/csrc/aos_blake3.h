/*
 * aos_blake3.h — BLAKE3 (the hash of the reference's B3Hash, crate blake3 1.8.3) for host and
 * device: the compression function, a serial hasher for the host, and the tree steps the router
 * kernel runs in parallel (one lane per 1 KiB chunk).
 *
 * Written from the BLAKE3 specification (O'Connor, Aumasson, Neves, Wilcox-O'Hearn, 2020):
 * chunks of 1024 bytes split into 64-byte blocks, compressed in sequence with the chunk counter
 * and the CHUNK_START / CHUNK_END flags; chunk chaining values merged pairwise into a binary tree
 * whose left subtrees hold the largest power of two of chunks; the root compression carries ROOT.
 * The 32-byte hash is the first eight output words, little-endian.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define AOS_B3_CHUNK_START 1u
#define AOS_B3_CHUNK_END 2u
#define AOS_B3_PARENT 4u
#define AOS_B3_ROOT 8u
#define AOS_B3_CHUNK_LEN 1024
#define AOS_B3_BLOCK_LEN 64

__host__ __device__ static __forceinline__ uint32_t aos_b3_iv(int i) {
  /* the SHA-256 initial hash value, which BLAKE3 keeps as its IV */
  const uint32_t iv[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                          0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
  return iv[i];
}

__host__ __device__ static __forceinline__ uint32_t aos_b3_rotr(uint32_t v, int c) { return (v >> c) | (v << (32 - c)); }

__host__ __device__ static __forceinline__ void aos_b3_g(uint32_t *s, int a, int b, int c, int d, uint32_t mx, uint32_t my) {
  s[a] = s[a] + s[b] + mx;
  s[d] = aos_b3_rotr(s[d] ^ s[a], 16);
  s[c] = s[c] + s[d];
  s[b] = aos_b3_rotr(s[b] ^ s[c], 12);
  s[a] = s[a] + s[b] + my;
  s[d] = aos_b3_rotr(s[d] ^ s[a], 8);
  s[c] = s[c] + s[d];
  s[b] = aos_b3_rotr(s[b] ^ s[c], 7);
}

/* The compression function: cv_out[8] = the new chaining value (first half of the output). */
__host__ __device__ static __forceinline__ void aos_b3_compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter,
                                                       uint32_t block_len, uint32_t flags, uint32_t cv_out[8]) {
  uint32_t s[16];
  uint32_t m[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) s[i] = cv[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[8 + i] = aos_b3_iv(i);
  s[12] = (uint32_t)counter;
  s[13] = (uint32_t)(counter >> 32);
  s[14] = block_len;
  s[15] = flags;
#pragma unroll
  for (int i = 0; i < 16; ++i) m[i] = block[i];
#pragma unroll
  for (int r = 0; r < 7; ++r) {
    aos_b3_g(s, 0, 4, 8, 12, m[0], m[1]);
    aos_b3_g(s, 1, 5, 9, 13, m[2], m[3]);
    aos_b3_g(s, 2, 6, 10, 14, m[4], m[5]);
    aos_b3_g(s, 3, 7, 11, 15, m[6], m[7]);
    aos_b3_g(s, 0, 5, 10, 15, m[8], m[9]);
    aos_b3_g(s, 1, 6, 11, 12, m[10], m[11]);
    aos_b3_g(s, 2, 7, 8, 13, m[12], m[13]);
    aos_b3_g(s, 3, 4, 9, 14, m[14], m[15]);
    if (r < 6) {
      /* message word permutation between rounds: m'[i] = m[P[i]],
       * P = 2 6 3 10 7 0 4 13 1 11 12 5 9 14 15 8 */
      const uint32_t t[16] = {m[2], m[6], m[3], m[10], m[7], m[0], m[4], m[13],
                              m[1], m[11], m[12], m[5], m[9], m[14], m[15], m[8]};
#pragma unroll
      for (int i = 0; i < 16; ++i) m[i] = t[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) cv_out[i] = s[i] ^ s[i + 8];
}

/* A parent node: the concatenated child chaining values as one 64-byte block. */
__host__ __device__ static __forceinline__ void aos_b3_parent(const uint32_t left[8], const uint32_t right[8], uint32_t flags,
                                                     uint32_t out[8]) {
  uint32_t block[16], iv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    block[i] = left[i];
    block[8 + i] = right[i];
    iv[i] = aos_b3_iv(i);
  }
  aos_b3_compress(iv, block, 0, AOS_B3_BLOCK_LEN, AOS_B3_PARENT | flags, out);
}

/* Chaining value of chunk c of an input of len bytes given as little-endian words: srcw(j) is
 * word j (bytes 4j .. 4j+3; a partial last word zero-padded). root marks the last block as the
 * root compression (a one-chunk input). */
template <class SrcW>
__host__ __device__ static __forceinline__ void aos_b3_chunk(const SrcW &srcw, size_t len, uint64_t c, bool root, uint32_t cv[8]) {
  const size_t base = (size_t)c * AOS_B3_CHUNK_LEN;
  const size_t clen = len - base < (size_t)AOS_B3_CHUNK_LEN ? len - base : (size_t)AOS_B3_CHUNK_LEN;
  const int nblk = clen == 0 ? 1 : (int)((clen + AOS_B3_BLOCK_LEN - 1) / AOS_B3_BLOCK_LEN);
  const size_t end = base + clen;
#pragma unroll
  for (int i = 0; i < 8; ++i) cv[i] = aos_b3_iv(i);
#pragma unroll 1
  for (int b = 0; b < nblk; ++b) {
    uint32_t block[16];
    const size_t off = base + (size_t)b * AOS_B3_BLOCK_LEN;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const size_t j = (off >> 2) + (size_t)w;
      block[w] = 4 * j < end ? srcw(j) : 0u;
    }
    const size_t blen = clen - (size_t)b * AOS_B3_BLOCK_LEN;
    uint32_t flags = (b == 0 ? AOS_B3_CHUNK_START : 0u) | (b == nblk - 1 ? AOS_B3_CHUNK_END : 0u);
    if (root && b == nblk - 1) flags |= AOS_B3_ROOT;
    aos_b3_compress(cv, block, c, (uint32_t)(blen < (size_t)AOS_B3_BLOCK_LEN ? blen : (size_t)AOS_B3_BLOCK_LEN), flags,
                    cv);
  }
}

/* Number of chunks of an input of len bytes (an empty input is one empty chunk). */
__host__ __device__ static __forceinline__ int aos_b3_nchunks(size_t len) {
  return len == 0 ? 1 : (int)((len + AOS_B3_CHUNK_LEN - 1) / AOS_B3_CHUNK_LEN);
}

/* Merge the chunk chaining values cvs[0..n) into the root hash (n >= 2): the incremental
 * hasher's stack (push each chunk after merging completed subtrees), then the right spine
 * folded into the stack with ROOT on the last parent. cvs is overwritten. */
__host__ __device__ static __forceinline__ void aos_b3_merge(uint32_t (*cvs)[8], int n, uint32_t out[8]) {
  int depth = 0; /* stack entries live in cvs[0 .. depth) */
#pragma unroll 1
  for (int c = 0; c < n - 1; ++c) {
    uint32_t cv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cv[i] = cvs[c][i];
    uint64_t total = (uint64_t)c + 1;
#pragma unroll 1
    while ((total & 1u) == 0) {
      --depth;
      aos_b3_parent(cvs[depth], cv, 0u, cv);
      total >>= 1;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) cvs[depth][i] = cv[i];
    ++depth;
  }
  uint32_t cv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cv[i] = cvs[n - 1][i];
#pragma unroll 1
  while (depth > 0) {
    --depth;
    aos_b3_parent(cvs[depth], cv, depth == 0 ? AOS_B3_ROOT : 0u, cv);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = cv[i];
}
