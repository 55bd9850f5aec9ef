/* Exhaustive check of the fast kernels' quotient of a bfloat16 weight by a
 * float32 scale (mround_amd/csrc/mr_quant.hip, quotients()):
 *
 *   y = RN(1/s),  q0 = RN(w * y),  r = RN(q0 * s - w) (fused),
 *   t = RN(q0 - r * y) (fused)
 *
 * must equal the IEEE quotient RN(w / s). While no intermediate leaves the
 * normal range every step scales exactly with the exponents of w and s, so
 * the identity depends only on the two significands: this program runs every
 * pair of a bfloat16 significand (7 stored bits) and a float32 significand
 * (23 stored bits), 2^30 pairs, and then the signed zeros and negative scales
 * (the symmetric modes divide -w by -s).
 *
 * It also checks the division of a float32 numerator by each maxq, 2^b - 1
 * for b = 1..8 and 2^(b - 1) for b = 1..8 (divisors of at most 8 significant
 * bits; div_maxq()), the same way: every float32 significand.
 *
 * Prints "ok <pairs>" and exits 0, or prints the first mismatches and exits 1.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* The kernels' sequence for s > 0. The volatile keeps the compiler from
 * folding the negation of r into the first fused multiply-add (a rewrite that
 * changes the sign of a zero r and so of a zero quotient); the GPU code
 * evaluates the two fused operations as written. */
static float quotient(float w, float s, float y) {
  const float q0 = w * y;
#ifdef DROP_CORRECTION /* the test suite's planted mistake: must be caught */
  return q0;
#endif
  volatile float r = fmaf(q0, s, -w);
  return fmaf(-r, y, q0);
}

/* A negative scale: -w divided by |s|. */
static float quotient_signed(float w, float s) {
  const float sa = fabsf(s);
  const float y = 1.0f / sa;
  const uint32_t sgn = to_bits(s) & 0x80000000u;
  return quotient(from_bits(to_bits(w) ^ sgn), sa, y);
}

static long bad = 0;
static void report(const char* what, float w, float s, float got, float want) {
  if (bad++ < 10)
    printf("%s: w=%a s=%a got=%a want=%a\n", what, (double)w, (double)s, (double)got, (double)want);
}

int main(void) {
  long pairs = 0;
  /* bfloat16 numerators in [1, 2), every float32 divisor significand in [1, 2). */
  for (uint32_t ms = 0; ms < (1u << 23); ++ms) {
    const float s = from_bits((127u << 23) | ms);
    const float y = 1.0f / s;
    for (uint32_t mw = 0; mw < (1u << 7); ++mw) {
      const float w = from_bits((127u << 23) | (mw << 16));
      const float got = quotient(w, s, y);
      const float want = w / s;
      if (to_bits(got) != to_bits(want)) report("bf16 / f32", w, s, got, want);
      ++pairs;
    }
  }
  /* Signs and zeros, at scales across the admissible range. */
  const float scales[] = {0x1p-60f, 3.0e-5f, 0.0123f, 1.0f, 1.5f, 7.0f, 1.0e7f, 0x1p60f};
  const float weights[] = {0.0f, -0.0f, 0x1p-60f, -0x1p-60f, 0.02f, -0.02f, 1.0f, -3.5f, 0x1p60f};
  for (size_t i = 0; i < sizeof scales / sizeof scales[0]; ++i) {
    for (size_t j = 0; j < sizeof weights / sizeof weights[0]; ++j) {
      const float w = from_bits(to_bits(weights[j]) & 0xffff0000u); /* a bfloat16 value */
      for (int sign = 0; sign < 2; ++sign) {
        const float s = sign ? -scales[i] : scales[i];
        const float got = quotient_signed(w, s);
        const float want = w / s;
        if (to_bits(got) != to_bits(want)) report("signed", w, s, got, want);
        ++pairs;
      }
    }
  }
  /* Float32 numerators over maxq = 2^b - 1 and 2^(b - 1). */
  for (int b = 1; b <= 16; ++b) {
    const float d = (float)(b <= 8 ? (1 << b) - 1 : 1 << (b - 9));
    const float y = 1.0f / d;
    for (uint32_t e = 0; e < 2; ++e) {
      for (uint32_t m = 0; m < (1u << 23); ++m) {
        const float x = from_bits(((127u + e) << 23) | m);
        const float got = quotient(x, d, y);
        const float want = x / d;
        if (to_bits(got) != to_bits(want)) report("f32 / maxq", x, d, got, want);
        ++pairs;
      }
    }
    const float zero = quotient(0.0f, d, y);
    if (to_bits(zero) != 0u) report("f32 / maxq", 0.0f, d, zero, 0.0f);
  }
  if (bad) {
    printf("%ld mismatches in %ld pairs\n", bad, pairs);
    return 1;
  }
  printf("ok %ld\n", pairs);
  return 0;
}
