/* Exhaustive check of the division used by the reference-format quantizer
 * on the GPU: for every finite fp16 numerator x and every positive finite
 * fp16 divisor s (as fp32 values),
 *
 *   y  = RN(1 / s)           (one IEEE division per token row)
 *   q0 = RN(x * y)
 *   r  = fma(-q0, s, x)      (the exact residual)
 *   q1 = copysign(fma(r, y, q0), q0)   (keeps the sign of a zero quotient)
 *
 * equals the correctly rounded quotient RN(x / s) bit for bit (Markstein's
 * correction step: with y the correctly rounded reciprocal and q0 within an
 * ulp of x / s, one FMA correction rounds correctly).  Prints the number of
 * mismatches and exits 1 if there is any.  Build: gcc -O2 -ffp-contract=off
 * -fopenmp div_correction_check.c -lm. */
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

int main(void) {
  long long bad = 0, total = 0;
#pragma omp parallel for reduction(+ : bad, total) schedule(dynamic, 64)
  for (int sb = 1; sb < 0x7c00; ++sb) {
    const float s = half_to_float((uint16_t)sb);
    const float y = 1.0f / s;
    for (int xb = 0; xb < 0x10000; ++xb) {
      if ((xb & 0x7c00) == 0x7c00) continue;   /* inf / NaN numerators take the IEEE path */
      const float x = half_to_float((uint16_t)xb);
      const float q0 = x * y;
      const float r = fmaf(-q0, s, x);
      const float q1 = copysignf(fmaf(r, y, q0), q0);
      const float q = x / s;
      uint32_t a, b;
      memcpy(&a, &q1, 4);
      memcpy(&b, &q, 4);
      bad += (a != b);
      ++total;
    }
  }
  printf("pairs %lld mismatches %lld\n", total, bad);
  return bad != 0;
}
