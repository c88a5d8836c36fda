/* Exhaustive check of the per-element quotient used by the reference-format
 * quantizer on the GPU.  The reference computes, per element,
 *
 *   t = rint(RN16(RN32(x / s)))      (fp16 tensors: an fp32 division whose
 *                                      result is stored as fp16, then round)
 *
 * and the kernel computes, with y = RN32(1 / s) once per token row,
 *
 *   t' = rint(RN16(RN32(x * y)))     (one multiply per element)
 *
 * For every finite fp16 numerator x and every positive finite fp16 divisor s
 * this program checks t' == t.  It also checks the form in which the product
 * is rounded to fp16 once, rint(RN16(x * y)) with x * y exact, so the result
 * holds whether or not the compiler fuses the multiply and the conversion.
 * (The fp16 quotients themselves differ in a few thousand pairs in either
 * form, all with quotients below 2^-14, the fp16 subnormal range, where rint
 * gives 0.)  RN16 is round-to-nearest-even onto the fp16 value set, infinity
 * beyond 65504 + 16; rint rounds half to even.  Prints the pair count and
 * both mismatch counts and exits 1 if either is nonzero.
 * Build: gcc -O2 -ffp-contract=off -fopenmp quotient_rint_check.c -lm. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 0x400u), (int)e - 25);
  uint32_t u;
  memcpy(&u, &v, 4);
  u |= sign;
  memcpy(&v, &u, 4);
  return v;
}

/* v rounded to the nearest fp16 value, ties to even, as a double.  fp16 has
 * 11 significant bits down to 2^-14 and a fixed spacing of 2^-24 below it;
 * magnitudes from 65520 (the midpoint between 65504 and 2^16, which ties to
 * the even 2^16) up overflow to infinity. */
static double rn16(double v) {
  if (isnan(v) || isinf(v)) return v;
  const double a = fabs(v);
  if (a >= 65520.0) return copysign(INFINITY, v);
  int e;
  frexp(a, &e);   /* a in [2^(e-1), 2^e) */
  int ulp = e - 11;
  if (ulp < -24) ulp = -24;
  return copysign(ldexp(nearbyint(ldexp(a, -ulp)), ulp), v);
}

int main(void) {
  long long bad_double = 0, bad_single = 0, total = 0;
#pragma omp parallel for reduction(+ : bad_double, bad_single, total) schedule(dynamic, 64)
  for (int sb = 1; sb < 0x7c00; ++sb) {
    const float s = half_to_float((uint16_t)sb);
    const float y = 1.0f / s;
    for (int xb = 0; xb < 0x10000; ++xb) {
      if ((xb & 0x7c00) == 0x7c00) continue;   /* finite numerators only */
      const float x = half_to_float((uint16_t)xb);
      const double t = nearbyint(rn16((double)(x / s)));
      const double t_double = nearbyint(rn16((double)(x * y)));
      const double t_single = nearbyint(rn16((double)x * (double)y));   /* 11 x 24 bits: exact */
      bad_double += !(t_double == t);
      bad_single += !(t_single == t);
      ++total;
    }
  }
  printf("pairs %lld mismatches %lld %lld\n", total, bad_double, bad_single);
  return (bad_double != 0 || bad_single != 0);
}
