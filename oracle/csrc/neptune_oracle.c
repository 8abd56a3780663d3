/*
 * neptune_oracle.c -- test infrastructure: plain-C restatement of the bit-level numerics of
 * neptune-opt's structured folds, used only by tests/ (and bench's CPU baseline leg) as the
 * checker of the HIP kernels.  Nothing in the product links or loads this file.
 *
 * Each function cites the reference code it restates (paths relative to the reference tree):
 *   f32 <-> bf16 / fp16   Triton .to(dtype, fp_downcast_rounding="rtne") used at
 *                         neptune_codegen/emitters.py:588 and torch_op.py:296,302
 *                         (IEEE 754 round-to-nearest-even, done here in integer arithmetic)
 *   rsqrt_rn              libdevice.rsqrt_rn at emitters.py:594,623 (correctly rounded 1/sqrt)
 *   rms_norm              emitters.py:583-595 + template.py:294-309 (serial RMS map, no FMA
 *                         contraction: build with -ffp-contract=off)
 *   l2_normalize          no reference function; x / max(sqrt_rn(sum x^2), eps) in the RMS staging
 *   segment_pool          torch_op.py:286-306 (ordered per-token fp32 add + RTNE to storage,
 *                         mean divides by fp32(storage(count)), empty/invalid policy)
 *
 * Parity pins live in tests/test_oracle_exact.py: conversions against torch's own conversions
 * over large bit-pattern sweeps, rsqrt_rn exhaustively over [1, 4) against an independent exact
 * integer test, segment pooling bit-exact against torch.segment_reduce on the reference's case
 * table, RMS/L2 against the canonical eager forms.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { NOR_F32 = 0, NOR_BF16 = 1, NOR_F16 = 2 };

static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---------------------------------------------------------------- storage conversions */
uint16_t nor_f32_to_bf16(float f) {
  uint32_t x = bits_of(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7fc0u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float nor_bf16_to_f32(uint16_t b) { return float_of((uint32_t)b << 16); }

uint16_t nor_f32_to_f16(float f) {
  const uint32_t x = bits_of(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t a = x & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;              /* NaN */
  if (a >= 0x477ff000u) return sign | 0x7c00u;             /* >= 65520 rounds to inf */
  if (a >= 0x38800000u) {                                  /* normal binary16 (>= 2^-14) */
    const uint32_t e = (a >> 23) - 127 + 15;
    uint32_t m = (e << 10) | ((a & 0x7fffffu) >> 13);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) m += 1; /* carry may raise exponent */
    return sign | (uint16_t)m;
  }
  if (a <= 0x33000000u) return sign;                       /* <= 2^-25 rounds to (signed) 0 */
  /* subnormal: value = mant * 2^(E-150) = k * 2^-24  ->  k = mant >> (126 - E), RTNE */
  const uint32_t E = a >> 23;
  const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  const uint32_t s = 126 - E;                              /* 14 .. 24 */
  uint32_t k = mant >> s;
  const uint32_t rem = mant & ((1u << s) - 1u), half = 1u << (s - 1);
  if (rem > half || (rem == half && (k & 1u))) k += 1;
  return sign | (uint16_t)k;
}

float nor_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1f) return float_of(sign | 0x7f800000u | (m << 13));
  if (e == 0) return (sign ? -1.0f : 1.0f) * (float)m * 5.9604644775390625e-08f; /* exact */
  return float_of(sign | ((e + 112u) << 23) | (m << 13));
}

static inline float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == NOR_F32) return ((const float*)p)[i];
  if (dtype == NOR_BF16) return nor_bf16_to_f32(((const uint16_t*)p)[i]);
  return nor_f16_to_f32(((const uint16_t*)p)[i]);
}

static inline float round_storage(float v, int dtype) {
  if (dtype == NOR_F32) return v;
  if (dtype == NOR_BF16) return nor_bf16_to_f32(nor_f32_to_bf16(v));
  return nor_f16_to_f32(nor_f32_to_f16(v));
}

static inline void store_elem(void* p, int64_t i, float v, int dtype) {
  if (dtype == NOR_F32) ((float*)p)[i] = v;
  else if (dtype == NOR_BF16) ((uint16_t*)p)[i] = nor_f32_to_bf16(v);
  else ((uint16_t*)p)[i] = nor_f32_to_f16(v);
}

/* ---------------------------------------------------------------- rsqrt_rn */
/* 1/sqrt(x) correctly rounded to fp32: r0 = fp32(1/sqrt(double x)) is within one ulp; the
 * midpoints between r0 and its neighbours decide exactly (h*h*x vs 1, with h*h exact in double
 * and one rounding in the fma, which cannot flip the sign of h*h*x - 1). */
float nor_rsqrt_rn(float x) {
  if (!(x > 0.0f) || isinf(x)) {
    if (x == 0.0f) return copysignf(INFINITY, x);
    if (isinf(x) && x > 0) return 0.0f;
    return NAN;
  }
  const double xd = (double)x;
  const float r = (float)(1.0 / sqrt(xd));
  const float r_dn = float_of(bits_of(r) - 1u), r_up = float_of(bits_of(r) + 1u);
  const double h_lo = 0.5 * ((double)r + (double)r_dn), h_hi = 0.5 * ((double)r + (double)r_up);
  const double lo = fma(h_lo * h_lo, xd, -1.0), hi = fma(h_hi * h_hi, xd, -1.0);
  if (lo > 0.0) return r_dn;
  if (hi < 0.0) return r_up;
  if (lo == 0.0) return (bits_of(r) & 1u) ? r_dn : r;
  if (hi == 0.0) return (bits_of(r) & 1u) ? r_up : r;
  return r;
}

/* Independent exact check that r is the correctly rounded 1/sqrt(x) for positive normal or
 * subnormal x: with exact integers, h*h*x compared against 1 for both midpoints around r. */
static void split(float f, uint64_t* mant, int* exp2) { /* f = mant * 2^exp2, mant < 2^24 */
  const uint32_t b = bits_of(f);
  const uint32_t e = (b >> 23) & 0xffu, m = b & 0x7fffffu;
  if (e == 0) { *mant = m; *exp2 = -149; }
  else { *mant = m | 0x800000u; *exp2 = (int)e - 150; }
}
/* sign of (h^2 * x - 1) where h = (a + b) / 2 and a, b positive floats */
static int mid_sign(float a, float b, float x) {
  uint64_t ma, mb, mx; int ea, eb, ex;
  split(a, &ma, &ea); split(b, &mb, &eb); split(x, &mx, &ex);
  /* bring a and b to the common exponent e = min(ea, eb): h = (A + B) * 2^(e-1) */
  int e = ea < eb ? ea : eb;
  unsigned __int128 A = (unsigned __int128)ma << (ea - e), B = (unsigned __int128)mb << (eb - e);
  unsigned __int128 H = A + B;                         /* h = H * 2^(e-1), H < 2^26 */
  unsigned __int128 P = H * H * mx;                    /* h^2 x = P * 2^(2e - 2 + ex) */
  int k = 2 * e - 2 + ex;                              /* compare P * 2^k with 1 */
  if (k >= 0) return P == 0 ? -1 : 1;                  /* P >= 1 here */
  if (-k >= 127) return P == 0 ? -1 : -1;
  unsigned __int128 one = (unsigned __int128)1 << (-k);
  return P > one ? 1 : (P < one ? -1 : 0);
}

int nor_rsqrt_is_correctly_rounded(float x, float r) {
  const float r_dn = float_of(bits_of(r) - 1u), r_up = float_of(bits_of(r) + 1u);
  const int lo = mid_sign(r_dn, r, x), hi = mid_sign(r, r_up, x);
  /* exact value y = 1/sqrt(x):  y >= h_lo  <=> h_lo^2 x <= 1;  y <= h_hi <=> h_hi^2 x >= 1 */
  if (lo > 0 || hi < 0) return 0;
  if (lo == 0 && (bits_of(r) & 1u)) return 0;   /* tie: even neighbour must win */
  if (hi == 0 && (bits_of(r) & 1u)) return 0;
  return 1;
}

/* Checks every fp32 bit pattern in [lo, hi) with the given stride; returns the number of
 * patterns that were not correctly rounded and the first such pattern in *first_bad. */
int64_t nor_check_rsqrt_range(uint32_t lo, uint32_t hi, uint32_t stride, uint32_t* first_bad) {
  int64_t bad = 0;
  for (uint64_t b = lo; b < hi; b += stride) {
    const float x = float_of((uint32_t)b);
    if (!nor_rsqrt_is_correctly_rounded(x, nor_rsqrt_rn(x))) {
      if (bad == 0 && first_bad) *first_bad = (uint32_t)b;
      ++bad;
    }
  }
  return bad;
}

/* ---------------------------------------------------------------- RMSNorm / L2-normalize */
void nor_rms_norm(const void* x, const void* gamma, void* out, int64_t rows, int64_t ncols,
                  int dtype, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    float total = 0.0f;
    for (int64_t c = 0; c < ncols; ++c) {
      const float v = load_elem(x, r * ncols + c, dtype);
      const float sq = v * v;
      total = total + sq;
    }
    const float mean = total / (float)ncols;
    const float scale = nor_rsqrt_rn(mean + eps);
    for (int64_t c = 0; c < ncols; ++c) {
      const float v = load_elem(x, r * ncols + c, dtype);
      const float normalized = round_storage(v * scale, dtype);
      store_elem(out, r * ncols + c, normalized * load_elem(gamma, c, dtype), dtype);
    }
  }
}

void nor_l2_normalize(const void* x, void* out, int64_t rows, int64_t ncols, int dtype, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    float total = 0.0f;
    for (int64_t c = 0; c < ncols; ++c) {
      const float v = load_elem(x, r * ncols + c, dtype);
      const float sq = v * v;
      total = total + sq;
    }
    const float den = fmaxf(sqrtf(total), eps);
    for (int64_t c = 0; c < ncols; ++c)
      store_elem(out, r * ncols + c, load_elem(x, r * ncols + c, dtype) / den, dtype);
  }
}

/* ---------------------------------------------------------------- segment pooling */
/* data [nrows, channels] contiguous in `dtype`; spans [nsegments + 1]; out [nsegments,
 * channels].  initial_bits: the fp32 pattern of the initial value (0.0 when none). */
void nor_segment_pool(const void* data, const int64_t* spans, void* out, int64_t nrows,
                      int64_t channels, int64_t nsegments, int dtype, int mean,
                      int has_initial, uint32_t initial_bits) {
  const float init = round_storage(float_of(initial_bits), dtype);
  for (int64_t s = 0; s < nsegments; ++s) {
    const int64_t start = spans[s], end = spans[s + 1];
    const int valid = start >= 0 && end >= start && end <= nrows;
    for (int64_t c = 0; c < channels; ++c) {
      float acc = init;
      if (valid)
        for (int64_t t = start; t < end; ++t)
          acc = round_storage(acc + load_elem(data, t * channels + c, dtype), dtype);
      float result = acc;
      if (mean) {
        const float den = round_storage((float)(end - start), dtype);
        result = acc / den;
        if (end == start) result = has_initial ? acc : NAN;
      }
      if (!valid) result = NAN;
      store_elem(out, s * channels + c, result, dtype);
    }
  }
}
