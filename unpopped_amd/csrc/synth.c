/*
 * Seeded synthetic inputs for the benchmark configurations and the parity tests.
 *
 * Every stream is the 64-bit LCG the reference's tests use for their corpora,
 *   s <- s * 6364136223846793005 + 1442695040888963407   (mod 2^64)
 * (crates/unpopped/tests/kernel_parallel_reduction_float_sum_bound.rs:40-45), started from the
 * configuration's seed; element i of a stream that takes d draws per element reads draws
 * i*d+1 .. i*d+d.  Streams are generated in parallel chunks, each chunk starting from the LCG
 * state jumped ahead in O(log n) (s_k = a^k s_0 + c (a^(k-1) + ... + 1)), so the output does not
 * depend on the thread count.
 *
 * Floats are dyadic where the configuration allows it, so exact sums exist:
 *   uniform[-1, 1) f32 = (k - 2^24) * 2^-24, k = the top 25 bits of s;
 *   uniform[0, 1)  f32 = k * 2^-24,          k = the top 24 bits of s;
 *   integer uniform in [0, 16) = s >> 60.
 * normal(0, 1) is Box-Muller in f64 on the pair of draws u = (s >> 11) * 2^-53 of each even
 * element (cos to the even element, sin to the odd one).
 * Zipf(s) over [0, range) draws a rank r by inverse CDF of (r + 1)^-s and maps it to the row
 * (r * 2654435761) mod range for a power-of-two range (an odd multiplier: a bijection).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LCG_A 6364136223846793005ull
#define LCG_C 1442695040888963407ull
#define CHUNK (1ll << 20)

static inline uint64_t next(uint64_t* s) {
  *s = *s * LCG_A + LCG_C;
  return *s;
}

/* The state after k steps from s. */
static uint64_t jump(uint64_t s, uint64_t k) {
  uint64_t a = LCG_A, c = LCG_C, A = 1, Cc = 0;
  while (k) {
    if (k & 1) {
      A = A * a;
      Cc = Cc * a + c;
    }
    c = c * (a + 1);
    a = a * a;
    k >>= 1;
  }
  return A * s + Cc;
}

static inline double unit53(uint64_t* s) { return (double)(next(s) >> 11) * (1.0 / 9007199254740992.0); }

static uint32_t f32_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

/* Round a finite f32 to bf16, nearest even. */
static uint16_t bf16_rne(float f) {
  const uint32_t b = f32_bits(f);
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

/* f16 bits, nearest even, of a value first rounded to f32 (normal f16 range only). */
static uint16_t f16_rne(double v) {
  const uint32_t b = f32_bits((float)v);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const int e = (int)((b >> 23) & 0xff) - 127 + 15;
  const uint32_t m = b & 0x7fffffu;
  if (e <= 0 || e >= 31) return (uint16_t)sign; /* outside the configured ranges */
  uint32_t m10 = m >> 13, ee = (uint32_t)e;
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (m10 & 1u))) {
    if (++m10 == 0x400u) {
      m10 = 0;
      ++ee;
    }
  }
  return (uint16_t)(sign | (ee << 10) | m10);
}

#define PARALLEL_CHUNKS(n, draws, ...)                                    \
  do {                                                                    \
    const int64_t nchunks_ = ((n) + CHUNK - 1) / CHUNK;                   \
    _Pragma("omp parallel for schedule(static)")                          \
    for (int64_t ch_ = 0; ch_ < nchunks_; ++ch_) {                        \
      const int64_t lo = ch_ * CHUNK;                                     \
      const int64_t hi = lo + CHUNK < (n) ? lo + CHUNK : (n);             \
      uint64_t s = jump(seed, (uint64_t)lo * (draws));                    \
      __VA_ARGS__                                                         \
    }                                                                     \
  } while (0)

void unp_synth_uniform_pm1_f32(uint64_t seed, int64_t n, float* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; ++i) {
      const int64_t k = (int64_t)(next(&s) >> 39);
      out[i] = (float)((double)(k - (1 << 24)) * (1.0 / 16777216.0));
    }
  });
}

void unp_synth_uniform_01_f32(uint64_t seed, int64_t n, float* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; ++i) out[i] = (float)((double)(next(&s) >> 40) * (1.0 / 16777216.0));
  });
}

void unp_synth_int16_i32(uint64_t seed, int64_t n, int32_t* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; ++i) out[i] = (int32_t)(next(&s) >> 60);
  });
}

/* Box-Muller on the pair of draws of element 2j: cos for 2j, sin for 2j + 1. */
static inline void normal_pair(uint64_t* s, double* a, double* b) {
  double u1 = unit53(s);
  const double u2 = unit53(s);
  if (u1 < 1e-300) u1 = 1e-300;
  const double r = sqrt(-2.0 * log(u1));
  const double t = 6.283185307179586 * u2;
  *a = r * cos(t);
  *b = r * sin(t);
}

void unp_synth_normal_f32(uint64_t seed, int64_t n, float* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; i += 2) {
      double a, b;
      normal_pair(&s, &a, &b);
      out[i] = (float)a;
      if (i + 1 < hi) out[i + 1] = (float)b;
    }
  });
}

/* bf16 bits of (float)(sigma * N(0, 1)), nearest even. */
void unp_synth_normal_bf16(uint64_t seed, int64_t n, double sigma, uint16_t* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; i += 2) {
      double a, b;
      normal_pair(&s, &a, &b);
      out[i] = bf16_rne((float)(sigma * a));
      if (i + 1 < hi) out[i + 1] = bf16_rne((float)(sigma * b));
    }
  });
}

void unp_synth_uniform_ids_i32(uint64_t seed, int64_t n, int64_t range, int32_t* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; ++i) out[i] = (int32_t)(int64_t)(unit53(&s) * (double)range);
  });
}

/* Zipf(exponent) ids over [0, range); range must be a power of two. Returns 0 on success. */
int unp_synth_zipf_ids_i32(uint64_t seed, int64_t n, int64_t range, double exponent, int32_t* out) {
  if (range <= 0 || (range & (range - 1)) != 0) return 1;
  double* cdf = (double*)malloc((size_t)range * sizeof(double));
  if (!cdf) return 2;
  double acc = 0.0;
  for (int64_t r = 0; r < range; ++r) {
    acc += pow((double)(r + 1), -exponent);
    cdf[r] = acc;
  }
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; ++i) {
      const double u = unit53(&s) * acc;
      int64_t a = 0, b = range - 1;
      while (a < b) { /* the first rank whose cumulative weight exceeds u */
        const int64_t mid = a + (b - a) / 2;
        if (cdf[mid] > u) b = mid;
        else a = mid + 1;
      }
      out[i] = (int32_t)(((uint64_t)a * 2654435761ull) & (uint64_t)(range - 1));
    }
  });
  free(cdf);
  return 0;
}

/* n 4-bit values uniform in [0, 16), packed two per byte, low nibble first (n even). */
void unp_synth_nibbles(uint64_t seed, int64_t n, uint8_t* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; i += 2) {
      const uint8_t v0 = (uint8_t)(next(&s) >> 60);
      const uint8_t v1 = i + 1 < hi ? (uint8_t)(next(&s) >> 60) : 0;
      out[i >> 1] = (uint8_t)(v0 | (v1 << 4));
    }
  });
}

/* f16 bits of lo + (hi - lo) * u (rounded to f32, then to f16 nearest even). */
void unp_synth_uniform_f16(uint64_t seed, int64_t n, double lo_v, double hi_v, uint16_t* out) {
  PARALLEL_CHUNKS(n, 1, {
    for (int64_t i = lo; i < hi; ++i) out[i] = f16_rne(lo_v + (hi_v - lo_v) * unit53(&s));
  });
}
