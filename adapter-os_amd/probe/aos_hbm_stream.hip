/*
 * aos_hbm_stream.hip — what one launch can read from HBM on this GPU, for the bench's decode
 * roofline (measured beside the 8 TB/s datasheet peak).
 *
 * The read pattern is the decode GEMVs' weight stream: the buffer is a sequence of 1 KiB chunks,
 * every wave of the grid streams a contiguous range of them (an even share, rounded to whole
 * chunks), each lane loading 16 bytes of a chunk, `depth` chunks in flight per wave in a register
 * ring. Workgroups have 4 waves. Before every timed launch a 1 GiB buffer is read (more than the
 * 256 MB last-level cache), so the timed buffer comes from HBM. The loaded words are folded and
 * stored once per workgroup under a condition that never holds, so nothing is optimised away.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

template <int D>
__global__ void __launch_bounds__(256) stream_kernel(const u32x4 *a, long nchunks, uint32_t *out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long nw = (long)gridDim.x * 4, w = (long)blockIdx.x * 4 + wave;
  const long lo = w * nchunks / nw, hi = (w + 1) * nchunks / nw;
  uint32_t s = 0;
  u32x4 r[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const long j = lo + d < hi ? lo + d : lo;
    r[d] = a[j * 64 + lane];
  }
  for (long c = lo; c < hi; c += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (c + d < hi) s ^= r[d].x ^ r[d].y ^ r[d].z ^ r[d].w;
      long j = c + d + D;
      j = j < hi ? j : lo;
      r[d] = a[j * 64 + lane];
    }
  }
  if (s == 0x9e3779b9u) out[blockIdx.x] = s;
}

struct State {
  char *big = nullptr, *buf = nullptr;
  uint32_t *out = nullptr;
  size_t big_bytes = 0, buf_bytes = 0;
  hipEvent_t e0 = nullptr, e1 = nullptr;
};

State g_state;

bool launch(int depth, const void *p, long nchunks, int wgs, hipEvent_t e0, hipEvent_t e1) {
  const dim3 grid(wgs), block(256);
  if (depth == 8)
    hipExtLaunchKernelGGL(stream_kernel<8>, grid, block, 0, 0, e0, e1, 0, (const u32x4 *)p, nchunks, g_state.out);
  else if (depth == 2)
    hipExtLaunchKernelGGL(stream_kernel<2>, grid, block, 0, 0, e0, e1, 0, (const u32x4 *)p, nchunks, g_state.out);
  else
    hipExtLaunchKernelGGL(stream_kernel<4>, grid, block, 0, 0, e0, e1, 0, (const u32x4 *)p, nchunks, g_state.out);
  return hipGetLastError() == hipSuccess;
}

}  // namespace

/* Median duration in microseconds of `reps` launches reading `bytes` (a multiple of 1 KiB, at
 * most 1 GiB) with `wgs` workgroups and `depth` (2, 4 or 8) chunks in flight per wave; each launch
 * follows a 1 GiB read that evicts the timed buffer from every cache. Times come from events the
 * dispatches record themselves. Returns a negative value on a HIP error or bad arguments. The
 * buffers are allocated on the first call and kept (aos_hbm_stream_free releases them). */
extern "C" double aos_hbm_stream_us(long bytes, int wgs, int depth, int reps) {
  const long GiB = 1L << 30;
  if (bytes < 1024 || bytes % 1024 || bytes > GiB || wgs < 1 || wgs > 65536 || reps < 1 || reps > 1000 ||
      (depth != 2 && depth != 4 && depth != 8))
    return -1.0;
  State &s = g_state;
  if (!s.big) {
    if (hipMalloc(&s.big, GiB) != hipSuccess) return -1.0;
    if (hipMalloc(&s.buf, GiB) != hipSuccess) return -1.0;
    if (hipMalloc(&s.out, 65536 * sizeof(uint32_t)) != hipSuccess) return -1.0;
    if (hipMemset(s.big, 1, GiB) != hipSuccess || hipMemset(s.buf, 2, GiB) != hipSuccess) return -1.0;
    if (hipEventCreate(&s.e0) != hipSuccess || hipEventCreate(&s.e1) != hipSuccess) return -1.0;
    s.big_bytes = s.buf_bytes = GiB;
  }
  std::vector<float> t;
  for (int r = 0; r <= reps; ++r) {
    if (!launch(4, s.big, GiB / 1024, 4096, nullptr, nullptr)) return -1.0; /* evict */
    if (!launch(depth, s.buf, bytes / 1024, wgs, s.e0, s.e1)) return -1.0;
    if (hipEventSynchronize(s.e1) != hipSuccess) return -1.0;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, s.e0, s.e1) != hipSuccess) return -1.0;
    if (r > 0) t.push_back(ms * 1000.0f); /* the first launch is a warm-up */
  }
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

extern "C" void aos_hbm_stream_free(void) {
  State &s = g_state;
  if (s.big) (void)hipFree(s.big);
  if (s.buf) (void)hipFree(s.buf);
  if (s.out) (void)hipFree(s.out);
  if (s.e0) (void)hipEventDestroy(s.e0);
  if (s.e1) (void)hipEventDestroy(s.e1);
  s = State();
}
