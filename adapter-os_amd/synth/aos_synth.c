/*
 * aos_synth.c — seeded synthetic inputs for the adapter-augmented layer workloads.
 *
 * Every value is a pure function of (seed, stream, index): element i of a stream is derived
 * from splitmix64(key(seed, stream) + i), so tensors can be generated in parallel and in any
 * order with identical results. Normals use Box-Muller (cosine branch) on two 53-bit uniforms,
 * evaluated in float64 with the C library and rounded once to float32.
 *
 * The workloads seed with 0xAD0500 + config_id and give each tensor its own stream number.
 */
#include <math.h>
#include <stdint.h>

static inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return splitmix64(seed ^ splitmix64(stream * 0xD1B54A32D192ED03ull));
}

/* n uniform 32-bit words (8 uniform nibbles each). */
void aos_synth_u32(uint64_t seed, uint64_t stream, int64_t n, uint32_t *out) {
  uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = (uint32_t)(splitmix64(key + (uint64_t)i) >> 32);
}

/* n normals N(mean, std^2) as float32. */
void aos_synth_normal(uint64_t seed, uint64_t stream, int64_t n, double mean, double std,
                      float *out) {
  uint64_t key = stream_key(seed, stream);
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint64_t a = splitmix64(key + 2 * (uint64_t)i);
    uint64_t b = splitmix64(key + 2 * (uint64_t)i + 1);
    double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53; /* (0, 1] */
    double u2 = (double)(b >> 11) * 0x1.0p-53;         /* [0, 1) */
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    out[i] = (float)(mean + std * z);
  }
}

/* n integers uniform in [0, m) (m > 0), via the high 32 bits times m. */
void aos_synth_randint(uint64_t seed, uint64_t stream, int64_t n, uint32_t m, uint32_t *out) {
  uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    out[i] = (uint32_t)(((splitmix64(key + (uint64_t)i) >> 32) * (uint64_t)m) >> 32);
}
