/*
 * CPU oracle for the unpopped-hip hot path.  TEST INFRASTRUCTURE ONLY (see oracle.h): the
 * parity tests, the smoke check and the benchmark's CPU-baseline leg call it as the checker.
 *
 * Single-threaded plain C, compiled with -O2 -ffp-contract=off like the reference's C leg
 * (crates/unpopped-cpu-c/tests/support/cc.rs:163-176), so every float operation rounds as
 * written.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t bits32(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}
static float from32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* ======================================================================================
 * Codecs
 * ==================================================================================== */

/* f32 -> bf16, nearest even; a NaN keeps its top half and is quieted.
 * crates/unpopped/src/oracle/float_codec.rs:259-266 */
uint16_t orc_f32_to_bf16_bits(float x) {
  const uint32_t b = bits32(x);
  if (x != x) return (uint16_t)((b >> 16) | 0x40u);
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

/* bf16 is the top half of an f32.  float_codec.rs:201-204 */
double orc_bf16_to_f64(uint16_t b) { return (double)from32((uint32_t)b << 16); }

/* binary16 decode, subnormals as mant * 2^-24, a NaN keeps its sign.  float_codec.rs:11-28 */
double orc_f16_to_f64(uint16_t h) {
  const double sign = (h & 0x8000u) ? -1.0 : 1.0;
  const int e = (h >> 10) & 0x1f;
  const int m = h & 0x3ff;
  if (e == 0) return sign * ldexp((double)m, -24);
  if (e == 0x1f) return m ? copysign(NAN, sign) : sign * INFINITY;
  return sign * ldexp(1.0 + (double)m / 1024.0, e - 15);
}

/* f32 -> binary16, nearest even, overflow to infinity.  float_codec.rs:206-257 */
uint16_t orc_f32_to_f16_bits(float x) {
  const uint32_t b = bits32(x);
  const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
  const int exp = (int)((b >> 23) & 0xff);
  const uint32_t mant = b & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
  const int e = exp - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return sign;
    const uint32_t m = mant | 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    const uint32_t half = 1u << (shift - 1), rem = m & ((1u << shift) - 1);
    uint32_t r = m >> shift;
    if (rem > half || (rem == half && (r & 1u))) r += 1;
    return (uint16_t)(sign | r);
  }
  const uint32_t rem = mant & 0x1fffu;
  uint32_t m10 = mant >> 13;
  int ee = e;
  if (rem > 0x1000u || (rem == 0x1000u && (m10 & 1u))) {
    if (++m10 == 0x400u) {
      m10 = 0;
      if (++ee >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    }
  }
  return (uint16_t)(sign | ((uint32_t)ee << 10) | m10);
}

/* f64 -> f32 rounded to odd, so a second rounding to a 16-bit float is correct.
 * crates/unpopped/src/oracle/expr_eval.rs:503-518 */
float orc_f64_to_f32_odd(double f) {
  const float r = (float)f;
  if (!isfinite(f) || f == 0.0 || (double)r == f) return r;
  uint32_t b = bits32(r);
  if (fabs((double)r) > fabs(f)) b -= 1; /* step back toward zero */
  return from32(b | 1u);
}

/* Storing an f64 compute value into a Bf16 buffer.  expr_eval.rs:520-527 (encode_float) */
uint16_t orc_store_bf16(double v) { return orc_f32_to_bf16_bits(orc_f64_to_f32_odd(v)); }

void orc_f32_to_bf16_array(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16_bits(x[i]);
}
void orc_f16_to_f64_array(const uint16_t* h, int64_t n, double* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f64(h[i]);
}

/* ======================================================================================
 * Sub-byte elements: two per byte, element i in byte i/2, low nibble = even index; U4
 * zero-extends, I4 sign-extends.  crates/unpopped/src/cfamily.rs:446-475,
 * crates/unpopped-cpu-c/src/kernel.rs:515-536
 * ==================================================================================== */
int32_t orc_u4_load(const uint8_t* p, int64_t i) { return (int32_t)((p[i >> 1] >> ((i & 1) * 4)) & 15u); }
int32_t orc_i4_load(const uint8_t* p, int64_t i) {
  const int32_t n = orc_u4_load(p, i);
  return n >= 8 ? n - 16 : n;
}
void orc_sub4_store(uint8_t* p, int64_t i, int32_t v) {
  const uint8_t nib = (uint8_t)(v & 15);
  uint8_t* b = &p[i >> 1];
  *b = (i & 1) ? (uint8_t)((*b & 0x0f) | (nib << 4)) : (uint8_t)((*b & 0xf0) | nib);
}

/* ======================================================================================
 * Reductions: lift_reduction_opdef's order (crates/unpopped/src/kernel_lift.rs:447-484,
 * ReductionShape :838-1025): per kept row, the reduced elements ascending into an
 * accumulator (f64 for a float, the dtype itself for an integer), Max/Min with a `have` flag
 * that keeps a NaN once seen (extremum_step :1097-1160), MaxNum/MinNum that skip a NaN element
 * and replace a NaN accumulator (nan_arm :1129-1160), And/Or/Xor seeded by the first element
 * (bit_step :1071-1095), Mean divides by the reduced extent, and one cast down at the store
 * (:965-983).  An empty fold stores the starting value.
 * ==================================================================================== */

static double fold_f64(int op, double acc, double v, int* have) {
  switch (op) {
    case ORC_SUM:
    case ORC_MEAN:
      return acc + v;
    case ORC_PROD:
      return acc * v;
    case ORC_MAX:
    case ORC_MIN: {
      double r = acc;
      if (!*have) r = v;
      else if (v != v) r = v;
      else if (op == ORC_MAX ? v > acc : v < acc) r = v;
      *have = 1;
      return r;
    }
    case ORC_MAXNUM:
    case ORC_MINNUM: {
      double r = acc;
      if (!*have) r = v;
      else if (acc != acc) r = v;
      else if (v == v && (op == ORC_MAXNUM ? v > acc : v < acc)) r = v;
      *have = 1;
      return r;
    }
  }
  return acc;
}

static double row_fold_f64(const double* xs, int64_t n, int op) {
  double acc = (op == ORC_PROD) ? 1.0 : 0.0;
  int have = 0;
  for (int64_t i = 0; i < n; ++i) acc = fold_f64(op, acc, xs[i], &have);
  if (op == ORC_MEAN) acc = acc / (double)n;
  return acc;
}

void orc_reduce_rows_f32(const float* in, int64_t rows, int64_t cols, int op, float* out) {
  double* tmp = (double*)malloc((size_t)(cols > 0 ? cols : 1) * sizeof(double));
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) tmp[c] = (double)in[r * cols + c];
    out[r] = (float)row_fold_f64(tmp, cols, op);
  }
  free(tmp);
}

void orc_reduce_rows_f64(const double* in, int64_t rows, int64_t cols, int op, double* out) {
  for (int64_t r = 0; r < rows; ++r) out[r] = row_fold_f64(in + r * cols, cols, op);
}

/* Integers fold exactly at their own width, wrapping (kernel_lift.rs:883-889). */
#define INT_REDUCE(NAME, T, U)                                                       \
  void NAME(const T* in, int64_t rows, int64_t cols, int op, T* out) {             \
    for (int64_t r = 0; r < rows; ++r) {                                           \
      U acc = (op == ORC_PROD) ? 1u : 0u;                                          \
      int have = 0;                                                                \
      for (int64_t c = 0; c < cols; ++c) {                                         \
        const T v = in[r * cols + c];                                              \
        if (op == ORC_SUM) acc = acc + (U)v;                                       \
        else if (op == ORC_PROD) acc = acc * (U)v;                                 \
        else if (op == ORC_AND) acc = have ? (acc & (U)v) : (U)v;                  \
        else if (op == ORC_OR) acc = have ? (acc | (U)v) : (U)v;                   \
        else if (op == ORC_XOR) acc = have ? (acc ^ (U)v) : (U)v;                  \
        else if (!have || ((op == ORC_MAX || op == ORC_MAXNUM) ? v > (T)acc        \
                                                                : v < (T)acc))     \
          acc = (U)v;                                                              \
        have = 1;                                                                  \
      }                                                                            \
      out[r] = (T)acc;                                                             \
    }                                                                              \
  }
INT_REDUCE(orc_reduce_rows_i32, int32_t, uint32_t)
INT_REDUCE(orc_reduce_rows_i64, int64_t, uint64_t)

/* The launched lift's float Sum order (kernel_lift/block_reduce.rs:14-24, Fold::rounds
 * :207-220): thread t folds xs[t], xs[t+B], ... from 0 in f64; then acc[t] += acc[t+s] for
 * s = B/2 .. 1; thread 0's total (divided by n for Mean).  Unrounded. */
double orc_sum_launched_order(const double* xs, int64_t n, int64_t block, int mean) {
  double* acc = (double*)calloc((size_t)block, sizeof(double));
  for (int64_t t = 0; t < block; ++t)
    for (int64_t i = t; i < n; i += block) acc[t] = acc[t] + xs[i];
  for (int64_t s = block / 2; s > 0; s /= 2)
    for (int64_t t = 0; t < s; ++t) acc[t] = acc[t] + acc[t + s];
  const double total = mean ? acc[0] / (double)n : acc[0];
  free(acc);
  return total;
}

/* Neumaier's compensated sum, the near-exact reference of the bound test
 * (crates/unpopped/tests/kernel_parallel_reduction_float_sum_bound.rs:171-186). */
double orc_neumaier(const double* xs, int64_t n) {
  double s = 0.0, c = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double x = xs[i];
    const double t = s + x;
    c += (fabs(s) >= fabs(x)) ? (s - t) + x : (x - t) + s;
    s = t;
  }
  return s + c;
}

/* The declared bound on a Sum/Mean result `got`: gamma_(n-1) * sum|x| (scaled for Mean),
 * half an ulp of the f32 rounding, and 4u |exact| for the reference sum's own error
 * (kernel_parallel_reduction_float_sum_bound.rs:188-214; the statement of the bound is
 * kernel_lift/block_reduce.rs:14-24). */
double orc_sum_bound(const double* xs, int64_t n, int mean, int f32, double got) {
  const double u = ldexp(1.0, -53);
  const double k = n > 1 ? (double)(n - 1) : 0.0;
  const double gamma = k * u / (1.0 - k * u);
  double sum_abs = 0.0;
  for (int64_t i = 0; i < n; ++i) sum_abs += fabs(xs[i]);
  const double scale = mean ? 1.0 / (double)n : 1.0;
  double rounding = 0.0;
  if (f32) {
    const uint32_t b = bits32(fabsf((float)got));
    rounding = 0.5 * ((double)from32(b + 1) - (double)from32(b));
  }
  return gamma * sum_abs * scale + rounding + 4.0 * u * fabs(orc_neumaier(xs, n)) * scale;
}

/* ======================================================================================
 * Scans: lift_scan_opdef's order (kernel_lift.rs:504-753): per row the prefix starts at the
 * monoid identity (0, 1, -inf/+inf, or the integer extremes: scan_identity :712-753), each
 * element is folded in (f64 for a float, wrapping for an integer), and the prefix is written
 * after the fold (inclusive) or before it (exclusive), walking the row descending for a
 * reverse scan; one cast down per written element.  A Mean scan writes acc / count.
 * ==================================================================================== */

static double scan_identity_f64(int op) {
  switch (op) {
    case ORC_PROD: return 1.0;
    case ORC_MAX: return -INFINITY;
    case ORC_MIN: return INFINITY;
    default: return 0.0;
  }
}

static void scan_row_f64(const double* x, int64_t n, int op, int excl, int rev, double* prefix_out) {
  double acc = scan_identity_f64(op);
  int have = 0;
  int64_t count = 0; /* a running Mean divides by the elements folded so far (0/0 first) */
  for (int64_t s = 0; s < n; ++s) {
    const int64_t i = rev ? n - 1 - s : s;
    if (excl) prefix_out[i] = (op == ORC_MEAN) ? acc / (double)count : acc;
    acc = fold_f64(op, acc, x[i], &have);
    ++count;
    if (!excl) prefix_out[i] = (op == ORC_MEAN) ? acc / (double)count : acc;
  }
}

void orc_scan_rows_f64(const double* in, int64_t rows, int64_t cols, int op, int exclusive, int reverse, double* out) {
  for (int64_t r = 0; r < rows; ++r) scan_row_f64(in + r * cols, cols, op, exclusive, reverse, out + r * cols);
}

void orc_scan_rows_f32(const float* in, int64_t rows, int64_t cols, int op, int exclusive, int reverse, float* out) {
  const size_t n = (size_t)(cols > 0 ? cols : 1);
  double* x = (double*)malloc(n * sizeof(double));
  double* p = (double*)malloc(n * sizeof(double));
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) x[c] = (double)in[r * cols + c];
    scan_row_f64(x, cols, op, exclusive, reverse, p);
    for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = (float)p[c];
  }
  free(x);
  free(p);
}

#define INT_SCAN(NAME, T, U, LO, HI)                                                  \
  void NAME(const T* in, int64_t rows, int64_t cols, int op, int excl, int rev, T* out) { \
    for (int64_t r = 0; r < rows; ++r) {                                              \
      U acc = (op == ORC_PROD) ? 1u : (op == ORC_MAX ? (U)(LO) : (op == ORC_MIN ? (U)(HI) : 0u)); \
      int have = 0;                                                                   \
      for (int64_t s = 0; s < cols; ++s) {                                            \
        const int64_t i = rev ? cols - 1 - s : s;                                     \
        const T v = in[r * cols + i];                                                 \
        if (excl) out[r * cols + i] = (T)acc;                                         \
        if (op == ORC_SUM) acc = acc + (U)v;                                          \
        else if (op == ORC_PROD) acc = acc * (U)v;                                    \
        else if (!have || (op == ORC_MAX ? v > (T)acc : v < (T)acc)) acc = (U)v;      \
        have = 1;                                                                     \
        if (!excl) out[r * cols + i] = (T)acc;                                        \
      }                                                                               \
    }                                                                                 \
  }
INT_SCAN(orc_scan_rows_i32, int32_t, uint32_t, INT32_MIN, INT32_MAX)
INT_SCAN(orc_scan_rows_i64, int64_t, uint64_t, INT64_MIN, INT64_MAX)

/* The launched scan's order for an f32 Sum row (kernel_lift/scan_launched.rs:1-26):
 * c = ceil(n / B); thread t folds scan positions [t*c, min(t*c + c, n)); a Kogge-Stone scan
 * over the B totals (total[t] = total[t] + total[t - d], own value on the left, old values);
 * thread t re-walks its chunk from total[t - 1] (the identity for t = 0). */
void orc_scan_launched_order_f32(const float* in, int64_t n, int64_t block, int exclusive, int reverse, float* out) {
  int64_t c = 0;
  while (c * block < n) ++c;
  double* tot = (double*)calloc((size_t)block, sizeof(double));
  double* old = (double*)calloc((size_t)block, sizeof(double));
  for (int64_t t = 0; t < block; ++t) {
    const int64_t lo = t * c, hi = lo + c < n ? lo + c : n;
    for (int64_t p = lo; p < hi; ++p) tot[t] = tot[t] + (double)in[reverse ? n - 1 - p : p];
  }
  for (int64_t d = 1; d < block; d *= 2) {
    memcpy(old, tot, (size_t)block * sizeof(double));
    for (int64_t t = d; t < block; ++t) tot[t] = old[t] + old[t - d];
  }
  for (int64_t t = 0; t < block; ++t) {
    double acc = t == 0 ? 0.0 : tot[t - 1];
    const int64_t lo = t * c, hi = lo + c < n ? lo + c : n;
    for (int64_t p = lo; p < hi; ++p) {
      const int64_t i = reverse ? n - 1 - p : p;
      if (exclusive) out[i] = (float)acc;
      acc = acc + (double)in[i];
      if (!exclusive) out[i] = (float)acc;
    }
  }
  free(tot);
  free(old);
}

/* ======================================================================================
 * Gather (crates/unpopped/src/kernel_lift/gather.rs:184-232): load the index once, clamp the
 * load address into [0, extent - 1] at the index dtype, then apply the policy to the store:
 * Skip leaves the row, ZeroFill writes zero, Clamp stores the clamped row.  The move is a raw
 * bit copy (oracle/expr_eval.rs:480-485: a Raw value of the output's dtype moves verbatim).
 * ==================================================================================== */
void orc_gather_rows(const uint8_t* table, int64_t src_extent, int64_t row_bytes, const void* ids, int idx_kind,
                     int64_t n_rows, int policy, uint8_t* out) {
  for (int64_t r = 0; r < n_rows; ++r) {
    int below = 0, above = 0;
    int64_t clamped = 0;
    if (idx_kind == ORC_IDX_U32) {
      const uint32_t raw = ((const uint32_t*)ids)[r];
      const uint32_t last = (uint32_t)src_extent - 1u;
      above = !(raw < (uint32_t)src_extent);
      clamped = (int64_t)(raw < last ? raw : last);
    } else {
      const int64_t raw = idx_kind == ORC_IDX_I32 ? (int64_t)((const int32_t*)ids)[r] : ((const int64_t*)ids)[r];
      below = raw < 0;
      above = raw >= src_extent;
      const int64_t lo = raw > 0 ? raw : 0;
      clamped = lo < src_extent - 1 ? lo : src_extent - 1;
    }
    uint8_t* dst = out + r * row_bytes;
    if (below || above) {
      if (policy == ORC_SKIP) continue;
      if (policy == ORC_ZEROFILL) {
        memset(dst, 0, (size_t)row_bytes);
        continue;
      }
    }
    if (clamped < 0 || clamped >= src_extent) continue; /* an empty source: nothing to read */
    memcpy(dst, table + clamped * row_bytes, (size_t)row_bytes);
  }
}

/* ======================================================================================
 * Sub-byte dequant: the KernelFn chain Load U4/I4 -> Cast I32 (zero/sign extend, widen to an
 * integer first: crates/unpopped/tests/kernel_subbyte_load.rs:206-212) -> Sub zero (exact) ->
 * Cast F32 -> Mul scale (F16 decoded exactly) -> store Bf16 (f32_to_bf16_bits after the
 * round-to-odd narrowing, expr_eval.rs:520-527).  Group g = column / group; the scale and the
 * zero point of (row, g) are element row * ceil(cols / group) + g of their buffers.
 * ==================================================================================== */
void orc_dequant4_bf16(const uint8_t* q, int q_signed, const uint16_t* scale, const uint8_t* zero, int z_signed,
                       int64_t rows, int64_t cols, int64_t group, uint16_t* out) {
  const int64_t ng = (cols + group - 1) / group;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const int64_t e = r * cols + c;
      const int64_t zi = r * ng + c / group;
      const int32_t qv = q_signed ? orc_i4_load(q, e) : orc_u4_load(q, e);
      const int32_t zv = z_signed ? orc_i4_load(zero, zi) : orc_u4_load(zero, zi);
      const float d = (float)(qv - zv);
      const double v = (double)d * orc_f16_to_f64(scale[zi]);
      out[e] = orc_store_bf16(v);
    }
  }
}

/* ---- row reduction --------------------------------------------------------------------- */
/* UnaryOp codes: the order of ORC_UNARY_NAMES in oracle/__init__.py. */
/* The dequantizing GEMM of crates/unpopped/tests/support/dequant.rs:107-181 (ROADMAP U9b S3,
 * docs/options-u9b-subbyte-dequant.md:28-30): out[r][c] = sum over k of
 * (w[r][k] - zero[r][k / group]) * scale[r][k / group] * x[k][c], w packed two 4-bit elements to
 * a byte (U4, or I4 sign-extended), zero and scale I32 per (row, group), the activations int8
 * widened to I32.  Every operation wraps at 32 bits, as the kernel's I32 arithmetic does; the
 * groups of a row are ceil(k / group), the last one ragged when group does not divide k. */
void orc_dequant_gemm_i32(const uint8_t* w, int w_signed, const int32_t* zero, const int32_t* scale, const void* x,
                          int x_i32, int64_t rows, int64_t k, int64_t cols, int64_t group, int32_t* out) {
  const int8_t* x8 = (const int8_t*)x;
  const int32_t* x32 = (const int32_t*)x;
  const int64_t ng = (k + group - 1) / group;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      uint32_t acc = 0;
      for (int64_t kk = 0; kk < k; ++kk) {
        const int64_t gi = r * ng + kk / group;
        const int32_t wv = w_signed ? orc_i4_load(w, r * k + kk) : orc_u4_load(w, r * k + kk);
        const uint32_t d = (uint32_t)wv - (uint32_t)zero[gi];
        const int32_t xv = x_i32 ? x32[kk * cols + c] : (int32_t)x8[kk * cols + c];
        acc += d * (uint32_t)scale[gi] * (uint32_t)xv;
      }
      out[r * cols + c] = (int32_t)acc;
    }
}

static double rx_unary(int32_t code, double x, int f32) {
  switch (code) {
    case 0: return -x;                                  /* Neg */
    case 1: return fabs(x);                             /* Abs */
    case 2: return x * x;                               /* Sqr */
    case 3: return sqrt(x);                             /* Sqrt */
    case 4: return 1.0 / sqrt(x);                       /* Rsqrt */
    case 5: return 1.0 / x;                             /* Recip */
    case 6: return exp(x);                              /* Exp */
    case 7: return log(x);                              /* Log */
    case 8: return tanh(x);                             /* Tanh */
    case 9: return 1.0 / (1.0 + exp(-x));               /* Sigmoid */
    case 10: return x < 0.0 ? 0.0 : x;                  /* Relu: NaN and -0 pass */
    case 11: return erf(x);                             /* Erf */
    case 12: return 0.5 * x * (1.0 + erf(x * 0.70710678118654752440)); /* Gelu */
    case 13: return x * (1.0 / (1.0 + exp(-x)));        /* Silu */
    case 14: return sin(x);
    case 15: return cos(x);
    case 16: return floor(x);
    case 17: return ceil(x);
    case 18: return nearbyint(x);                       /* Round: ties to even */
    case 19: { const double c = f32 ? (double)(float)x : x; return c > 0.0 ? 1.0 : (c < 0.0 ? -1.0 : 0.0); } /* Sign */
    case 20: { const double c = f32 ? (double)(float)x : x; return c > 0.0 ? 1.0 : 0.0; }                   /* Step */
    case 21: return erfc(x);
    case 22: return trunc(x);
    case 23: return exp2(x);
    case 24: return expm1(x);
    case 25: return log2(x);
    case 26: return log10(x);
    case 27: return log1p(x);
    case 28: return sinh(x);
    case 29: return cosh(x);
    case 30: return tan(x);
    case 31: return asin(x);
    case 32: return acos(x);
    case 33: return atan(x);
    case 34: return asinh(x);
    case 35: return acosh(x);
    case 36: return copysign(atanh(fabs(x)), x);        /* Atanh, on |x| (scalar_ops.rs) */
    case 37: return cbrt(x);
    default: return NAN;
  }
}

/* BinaryOp codes: the order of ORC_BINARY_NAMES in oracle/__init__.py. */
static double rx_binary(int32_t code, double a, double b) {
  switch (code) {
    case 0: return a != a ? a : (b != b ? b : (a >= b ? a : b)); /* Max: NaN-propagating, a on ties */
    case 1: return a != a ? a : (b != b ? b : (a <= b ? a : b)); /* Min */
    case 2: return pow(a, b);
    case 3: return a - floor(a / b) * b;                         /* Rem: floored */
    case 4: return fmod(a, b);                                   /* RemTrunc */
    case 5: return atan2(a, b);
    case 6: return copysign(a, b);
    case 7: return fmax(a, b);                                   /* FmaxIeee */
    case 8: return fmin(a, b);                                   /* FminIeee */
    case 9: return a == b ? 1.0 : 0.0;
    case 10: return a != b ? 1.0 : 0.0;
    case 11: return a < b ? 1.0 : 0.0;
    case 12: return a <= b ? 1.0 : 0.0;
    case 13: return a > b ? 1.0 : 0.0;
    case 14: return a >= b ? 1.0 : 0.0;
    default: return NAN;
  }
}

double orc_rx_eval(const orc_rx* prog, int32_t len, const double* x, const double* red, int f32) {
  double st[64];
  int sp = 0;
  for (int32_t i = 0; i < len; ++i) {
    const orc_rx* p = &prog[i];
    switch (p->op) {
      case ORC_RX_INPUT: st[sp++] = x[p->arg]; break;
      case ORC_RX_REDUCED: st[sp++] = red[p->arg]; break;
      case ORC_RX_CONST: st[sp++] = p->c; break;
      case ORC_RX_ADD: sp--; st[sp - 1] = st[sp - 1] + st[sp]; break;
      case ORC_RX_SUB: sp--; st[sp - 1] = st[sp - 1] - st[sp]; break;
      case ORC_RX_MUL: sp--; st[sp - 1] = st[sp - 1] * st[sp]; break;
      case ORC_RX_DIV: sp--; st[sp - 1] = st[sp - 1] / st[sp]; break;
      case ORC_RX_FMA: sp -= 2; st[sp - 1] = fma(st[sp - 1], st[sp], st[sp + 1]); break;
      case ORC_RX_SELECT: sp -= 2; st[sp - 1] = st[sp - 1] != 0.0 ? st[sp] : st[sp + 1]; break;
      case ORC_RX_UNARY: st[sp - 1] = rx_unary(p->arg, st[sp - 1], f32); break;
      case ORC_RX_BINARY: sp--; st[sp - 1] = rx_binary(p->arg, st[sp - 1], st[sp]); break;
      default: return NAN;
    }
  }
  return sp == 1 ? st[0] : NAN;
}

void orc_row_reduce(const void* const* ins, int32_t n_inputs, int64_t rows, int64_t cols, int f64, int32_t n_stages,
                    const int32_t* ops, const orc_rx* const* pres, const int32_t* pre_lens, const orc_rx* epi,
                    int32_t epi_len, void* out) {
  double x[16], red[16];
  const int f32 = !f64;
#define ORC_LOAD(k, i) (f64 ? ((const double*)ins[k])[i] : (double)((const float*)ins[k])[i])
#define ORC_ROUND(v) (f64 ? (v) : (double)(float)(v))
  for (int64_t r = 0; r < rows; ++r) {
    for (int32_t s = 0; s < n_stages; ++s) {
      double acc = ops[s] == ORC_PROD ? 1.0 : 0.0;
      int have = 0;
      for (int64_t c = 0; c < cols; ++c) {
        for (int32_t k = 0; k < n_inputs; ++k) x[k] = ORC_LOAD(k, r * cols + c);
        const double v = ORC_ROUND(orc_rx_eval(pres[s], pre_lens[s], x, red, f32));
        switch (ops[s]) {
          case ORC_SUM:
          case ORC_MEAN: acc = acc + v; break;
          case ORC_PROD: acc = acc * v; break;
          default:
            if (!have) acc = v;
            else if (v != v) acc = v;
            else if (ops[s] == ORC_MAX ? v > acc : v < acc) acc = v;
            have = 1;
        }
      }
      const double fin = ops[s] == ORC_MEAN ? acc / (double)cols : acc;
      red[s] = ORC_ROUND(fin);
    }
    for (int64_t c = 0; c < cols; ++c) {
      for (int32_t k = 0; k < n_inputs; ++k) x[k] = ORC_LOAD(k, r * cols + c);
      const double v = orc_rx_eval(epi, epi_len, x, red, f32);
      if (f64) ((double*)out)[r * cols + c] = v;
      else ((float*)out)[r * cols + c] = (float)v;
    }
  }
#undef ORC_LOAD
#undef ORC_ROUND
}

/* ======================================================================================
 * Scan with a pre-map and a fused post: lift_scan_opdef (kernel_lift.rs:504-519) with
 * scan_loads (:530-545, `val = up(pre)`), scan_pass (:548-576), scan_write (:578-602, the prefix
 * rounded once into `red`, the post over it and the loaded elements) and scan_stored (:604-619).
 * ==================================================================================== */

void orc_scan_x(const void* const* ins, int32_t n_inputs, int64_t a_ext, int64_t s_ext, int64_t b_ext, int f64, int op,
                int exclusive, int reverse, const orc_rx* pre, int32_t pre_len, const orc_rx* post, int32_t post_len,
                void* out) {
  double x[16], red[1] = {0.0};
  const int f32 = !f64;
#define ORC_LOAD(k, i) (f64 ? ((const double*)ins[k])[i] : (double)((const float*)ins[k])[i])
#define ORC_ROUND(v) (f64 ? (v) : (double)(float)(v))
#define ORC_STORE(i, v) (f64 ? (void)(((double*)out)[i] = (v)) : (void)(((float*)out)[i] = (float)(v)))
  for (int64_t a = 0; a < a_ext; ++a)
    for (int64_t b = 0; b < b_ext; ++b) {
      double acc = scan_identity_f64(op);
      int have = 0;
      int64_t count = 0;
      for (int64_t s = 0; s < s_ext; ++s) {
        const int64_t i = reverse ? s_ext - 1 - s : s;
        const int64_t off = (a * s_ext + i) * b_ext + b;
        for (int32_t k = 0; k < n_inputs; ++k) x[k] = ORC_LOAD(k, off);
        const double v = ORC_ROUND(orc_rx_eval(pre, pre_len, x, red, f32));
        for (int pass = 0; pass < 2; ++pass) {
          if (pass == (exclusive ? 1 : 0)) {
            acc = fold_f64(op, acc, v, &have);
            ++count;
            continue;
          }
          const double r = ORC_ROUND(op == ORC_MEAN ? acc / (double)count : acc);
          if (post_len > 0) {
            red[0] = r;
            ORC_STORE(off, orc_rx_eval(post, post_len, x, red, f32));
          } else {
            ORC_STORE(off, r);
          }
        }
      }
    }
#undef ORC_LOAD
#undef ORC_ROUND
#undef ORC_STORE
}

/* ======================================================================================
 * Access::Elementwise: lift_elementwise_opdef (kernel_lift.rs:96-130) run by the kernel
 * evaluator.  A float statement is evaluated in f64 and rounded once at the store
 * (kernel_eval.rs:763-771); an integer one by eval_int (kernel_eval.rs:809-848) with int_div,
 * int_binary, int_shift and wrap (:1114-1175).
 * ==================================================================================== */

void orc_elementwise_f(const void* const* ins, int32_t n_inputs, int64_t count, int f64, const orc_rx* prog,
                       int32_t len, void* out) {
  double x[16], red[1] = {0.0};
  for (int64_t i = 0; i < count; ++i) {
    for (int32_t k = 0; k < n_inputs; ++k)
      x[k] = f64 ? ((const double*)ins[k])[i] : (double)((const float*)ins[k])[i];
    const double v = orc_rx_eval(prog, len, x, red, !f64);
    if (f64) ((double*)out)[i] = v;
    else ((float*)out)[i] = (float)v;
  }
}

typedef __int128 i128;

/* The kind's value range (types.rs int_range). */
static void int_range(int32_t kind, i128* lo, i128* hi) {
  switch (kind) {
    case ORC_K_I32: *lo = -((i128)1 << 31); *hi = ((i128)1 << 31) - 1; break;
    case ORC_K_U32: *lo = 0; *hi = ((i128)1 << 32) - 1; break;
    case ORC_K_I64: *lo = -((i128)1 << 63); *hi = ((i128)1 << 63) - 1; break;
    default: *lo = 0; *hi = ((i128)1 << 64) - 1; break;
  }
}

/* wrap (kernel_eval.rs:1165-1174): v taken into the kind's range modulo its size. */
static i128 int_wrap(int32_t kind, i128 v) {
  i128 lo, hi;
  int_range(kind, &lo, &hi);
  if (v >= lo && v <= hi) return v;
  const i128 m = hi - lo + 1;
  i128 r = (v - lo) % m;
  if (r < 0) r += m;
  return r + lo;
}

/* int_div (kernel_eval.rs:1114-1120): a zero divisor and signed MIN / -1 give the dividend;
 * otherwise the quotient truncated toward zero (C's `/` on the 128-bit values). */
static i128 int_div(int32_t kind, i128 x, i128 y, int32_t mutant) {
  i128 lo, hi;
  int_range(kind, &lo, &hi);
  if (y == 0) return (mutant & ORC_MUT_DIV0) ? 0 : x;
  if (lo < 0 && x == lo && y == -1) return (mutant & ORC_MUT_MINNEG1) ? hi : x;
  i128 q = x / y;
  if ((mutant & ORC_MUT_FLOOR) && (x % y != 0) && ((x < 0) != (y < 0))) q -= 1;
  return q;
}

/* int_shift (kernel_eval.rs:1151-1163): the count's two's-complement bits modulo the width (64
 * for a 64-bit kind, else 32); Shl wraps, Shr is arithmetic on the signed value (logical for an
 * unsigned kind, whose values are non-negative). */
static i128 int_shift(int32_t kind, int left, i128 x, i128 y, int32_t mutant) {
  const int width = (kind == ORC_K_I64 || kind == ORC_K_U64) ? 64 : 32;
  const unsigned __int128 ybits = (unsigned __int128)y;
  unsigned k = (unsigned)(ybits & (unsigned __int128)(width - 1));
  if ((mutant & ORC_MUT_CLAMP) && (y < 0 || y >= width)) {
    /* a count past the width clamps to the width: every bit shifted out */
    if (left) return 0;
    return x < 0 ? -1 : 0;
  }
  if (left) return int_wrap(kind, x * ((i128)1 << k));
  if ((mutant & ORC_MUT_LOGICAL) && x < 0) {
    i128 lo, hi;
    int_range(kind, &lo, &hi);
    const i128 m = (hi - lo + 1);
    return int_wrap(kind, (x + m) >> k);
  }
  return x >> k; /* gcc's >> of a negative __int128 is arithmetic */
}

static i128 ix_input(int32_t kind, int64_t raw) {
  switch (kind) {
    case ORC_K_I32: return (int32_t)(uint32_t)(uint64_t)raw;
    case ORC_K_U32: return (uint32_t)(uint64_t)raw;
    case ORC_K_I64: return raw;
    default: return (uint64_t)raw;
  }
}

void orc_elementwise_i(const int64_t* const* ins, int32_t n_inputs, int64_t count, const orc_ix* prog, int32_t len,
                       int32_t mutant, int64_t* out) {
  (void)n_inputs;
  i128 st[64];
  for (int64_t i = 0; i < count; ++i) {
    int sp = 0;
    for (int32_t j = 0; j < len; ++j) {
      const orc_ix* p = &prog[j];
      const int32_t t = p->kind;
      i128 a = 0, b = 0, c = 0;
      switch (p->op) {
        case ORC_IX_INPUT: st[sp++] = ix_input(t, ins[p->arg][i]); continue;
        case ORC_IX_CONST: st[sp++] = int_wrap(t, (i128)p->v); continue;
        case ORC_IX_CAST: st[sp - 1] = int_wrap(t, st[sp - 1]); continue;
        case ORC_IX_SELECT:
          sp -= 2;
          c = st[sp - 1];
          st[sp - 1] = c != 0 ? st[sp] : st[sp + 1];
          continue;
        default: break;
      }
      sp--;
      a = st[sp - 1];
      b = st[sp];
      i128 r = 0;
      switch (p->op) {
        case ORC_IX_ADD: r = int_wrap(t, a + b); break;
        case ORC_IX_SUB: r = int_wrap(t, a - b); break;
        case ORC_IX_MUL: {
          /* the product of two 64-bit values can pass 2^127: wrap through the unsigned 128-bit
           * product, whose low 64 bits are the product's */
          const unsigned __int128 u = (unsigned __int128)a * (unsigned __int128)b;
          r = int_wrap(t, (i128)(uint64_t)u);
          if (t == ORC_K_I32 || t == ORC_K_U32) r = int_wrap(t, (i128)(uint32_t)(uint64_t)u);
          break;
        }
        case ORC_IX_DIV: r = int_div(t, a, b, mutant); break;
        case ORC_IX_SHL: r = int_shift(t, 1, a, b, mutant); break;
        case ORC_IX_SHR: r = int_shift(t, 0, a, b, mutant); break;
        case ORC_IX_MIN: r = a < b ? a : b; break;
        case ORC_IX_MAX: r = a > b ? a : b; break;
        case ORC_IX_AND: r = a & b; break;
        case ORC_IX_OR: r = a | b; break;
        case ORC_IX_XOR: r = a ^ b; break;
        case ORC_IX_CMP:
          switch (p->arg) {
            case 0: r = a == b; break;
            case 1: r = a != b; break;
            case 2: r = a < b; break;
            case 3: r = a <= b; break;
            case 4: r = a > b; break;
            default: r = a >= b; break;
          }
          break;
        default: r = 0; break;
      }
      st[sp - 1] = r;
    }
    out[i] = (int64_t)(uint64_t)(unsigned __int128)st[0];
  }
}
