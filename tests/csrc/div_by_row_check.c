/* CPU check of the L2 readout's division by the row norm (nep_rms.h, div_by_row):
 *   y = RN(1/s); q0 = RN(v*y); r = fma(q0, s, -v); q = fma(-r, y, q0)
 * equals the IEEE quotient RN(v/s) bit for bit, signed zeros included, whenever s and 1/s are
 * normal, v is zero or |v| >= 2^-100, and the quotient is zero or normal.  Random pairs over
 * those ranges, then every fp32 v in [2^-100, 2) (step `stride`) for eight divisors.
 * Usage: div_by_row_check <random pairs> <stride>.  Exit status 0 when nothing differs. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t bits(float x) { uint32_t v; memcpy(&v, &x, 4); return v; }
static uint64_t state = 88172645463325252ull;
static uint64_t next(void) { state ^= state << 13; state ^= state >> 7; state ^= state << 17; return state; }

static long mismatches = 0;
static void check(float v, float s) {
  const float want = v / s;
  const float y = 1.0f / s;
  const float q0 = v * y;
  const float r = fmaf(q0, s, -v);
  const float q = fmaf(-r, y, q0);
  if (bits(q) != bits(want) && !(isnan(q) && isnan(want))) {
    if (++mismatches <= 5) printf("mismatch v=%a s=%a want=%a got=%a\n", v, s, want, q);
  }
}
static int in_range(float v, float s) {
  const float q = v / s;
  if (!isfinite(v) || !isfinite(q)) return 0;
  if (v != 0.0f && fabsf(v) < 0x1p-100f) return 0;
  if (q != 0.0f && fabsf(q) < 0x1p-126f) return 0;
  return 1;
}

int main(int argc, char** argv) {
  const long n = argc > 1 ? atol(argv[1]) : 1000000;
  const uint32_t stride = argc > 2 ? (uint32_t)atol(argv[2]) : 1;
  long checked = 0;
  for (long i = 0; i < n; ++i) {
    const uint64_t w = next();
    const uint32_t ub = (uint32_t)w, ua = (uint32_t)(w >> 32);
    const float s = ldexpf(1.0f + (ub & 0x7fffff) / 8388608.0f, (int)(ub >> 24) % 146 - 20);
    float v;
    switch ((int)(next() % 3)) {
      case 0: v = from_bits(ua); break;
      case 1: v = s * ldexpf(1.0f + (ua & 0x7fffff) / 8388608.0f, (int)(ua >> 24) % 60 - 50); break;
      default: v = nextafterf(s * ldexpf(1.0f, (int)(ua % 80) - 70), (ua & 1) ? INFINITY : -INFINITY);
    }
    if (!in_range(v, s)) continue;
    check(v, s);
    ++checked;
  }
  const float divisors[] = {1e-6f, 0x1.fffffep-1f, 1.0f, 3.0f, 0x1.000002p+0f, 7.123457e3f,
                            0x1.6a09e6p+20f, 1.8e19f};
  long swept = 0;
  for (int d = 0; d < 8; ++d) {
    for (uint32_t b = bits(0x1p-100f); b < bits(2.0f); b += stride) {
      const float v = from_bits(b);
      if (!in_range(v, divisors[d])) continue;
      check(v, divisors[d]);
      check(-v, divisors[d]);
      swept += 2;
    }
    check(0.0f, divisors[d]);
    check(-0.0f, divisors[d]);
  }
  printf("random %ld, swept %ld, mismatches %ld\n", checked, swept, mismatches);
  return mismatches != 0;
}
