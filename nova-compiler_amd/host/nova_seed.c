/*
 * nova_seed -- deterministic, counter-based synthetic inputs for the Nova
 * GPU matmul / reduction path.
 *
 * The reference owns no usable generator for these configs: `nova.rndm2d`
 * derives its seed as (min+max)^max and fills through linalg.fill_rng_2d
 * (NovaToLinalg.cpp:1410-1432).  Inputs are therefore produced once on the
 * host by this file and handed unchanged to both the CPU oracle and the GPU
 * path.
 *
 * Generator (documented so that any implementation can reproduce it):
 *   key        = splitmix64(seed)
 *   word(c)    = splitmix64(key + (c + 1) * 0x9E3779B97F4A7C15)   -- counter c
 *   u24(c)     = word(c) >> 40                   (24 random bits)
 *   uniform    : element g  -> lo + (hi - lo) * (u24(off+g) * 2^-24), in f32
 *   normal     : element g  -> mean + std * sqrt(-2 ln u1) cos(2 pi u2) (f64,
 *                 then rounded to f32), u1 = (u24(2(off+g)) + 1) * 2^-24,
 *                 u2 = u24(2(off+g)+1) * 2^-24  -- two counters per element
 *   int labels : element g  -> ((word(off+g) >> 32) * n) >> 32  in [0, n)
 *   bf16 / f16 : the f32 value rounded to nearest-even.
 * `off` lets several tensors share one seed as a continued stream: a caller
 * advances it by n for uniform/int tensors and by 2n for normal tensors.
 *
 * Every element depends only on (seed, counter), so the OpenMP loops below
 * produce identical bytes for any thread count.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

static inline uint64_t word_at(uint64_t key, uint64_t c) {
  return splitmix64(key + (c + 1) * 0x9E3779B97F4A7C15ULL);
}

static inline float u01(uint64_t key, uint64_t c) {
  return (float)(word_at(key, c) >> 40) * (1.0f / 16777216.0f);
}

static inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline uint16_t f32_to_f16_rne(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (ax < 0x38800000u) {                                 /* f16 subnormal */
    if (ax < 0x33000000u) return (uint16_t)sign;          /* < 2^-25 -> 0  */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - e; /* 14..24 */
    uint32_t r = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ax - 0x38000000u; /* rebias 127 -> 15 */
  uint32_t lsb = (r >> 13) & 1u;
  r += 0xfffu + lsb;
  return (uint16_t)(sign | (r >> 13));
}

/* dtype codes shared with the Python side: 0 = f32, 1 = bf16, 2 = f16 */
static inline void put(void *dst, int dtype, int64_t i, float v) {
  if (dtype == 0) ((float *)dst)[i] = v;
  else if (dtype == 1) ((uint16_t *)dst)[i] = f32_to_bf16_rne(v);
  else ((uint16_t *)dst)[i] = f32_to_f16_rne(v);
}

int nova_seed_uniform(void *dst, int dtype, int64_t n, uint64_t seed,
                      uint64_t off, float lo, float hi) {
  if (!dst || n < 0 || dtype < 0 || dtype > 2) return -1;
  const uint64_t key = splitmix64(seed);
  const float span = hi - lo;
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    float u = u01(key, off + (uint64_t)g);
    put(dst, dtype, g, lo + span * u);
  }
  return 0;
}

int nova_seed_normal(void *dst, int dtype, int64_t n, uint64_t seed,
                     uint64_t off, float mean, float std) {
  if (!dst || n < 0 || dtype < 0 || dtype > 2) return -1;
  const uint64_t key = splitmix64(seed);
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    uint64_t c = 2 * (off + (uint64_t)g);
    double u1 = ((double)(word_at(key, c) >> 40) + 1.0) * (1.0 / 16777216.0);
    double u2 = (double)(word_at(key, c + 1) >> 40) * (1.0 / 16777216.0);
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    put(dst, dtype, g, (float)((double)mean + (double)std * z));
  }
  return 0;
}

int nova_seed_labels(int32_t *dst, int64_t n, uint64_t seed, uint64_t off,
                     int32_t n_classes) {
  if (!dst || n < 0 || n_classes <= 0) return -1;
  const uint64_t key = splitmix64(seed);
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < n; ++g) {
    uint64_t w = word_at(key, off + (uint64_t)g) >> 32;
    dst[g] = (int32_t)((w * (uint64_t)n_classes) >> 32);
  }
  return 0;
}

/* Rounding helpers exported for the host side (casts of a11). */
int nova_seed_round_f32(const float *src, void *dst, int dtype, int64_t n) {
  if (!src || !dst || n < 0 || dtype < 1 || dtype > 2) return -1;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) put(dst, dtype, i, src[i]);
  return 0;
}
