/* Exhaustive check of the reciprocal used by the reference-format quantizer
 * on the GPU: for every positive finite fp16 value s (as an fp32 value) and
 * every fp32 y0 within one ulp of 1 / s (the two fp32 neighbours of the
 * exact reciprocal, which is the accuracy the hardware reciprocal
 * instruction guarantees; tested as RN(1 / s) and its two neighbours),
 *
 *   e  = fma(-s, y0, 1)       (exact: |1 - s y0| < 2^-22 on a 2^-33 grid)
 *   y1 = fma(e, y0, y0)       (one Newton step, one rounding)
 *
 * equals the correctly rounded reciprocal RN(1 / s) bit for bit.  The step
 * leaves y0 (2 - s y0), within e^2 < 2^-44 of 1 / s, and 1 / s lies at
 * least 2^-36 (relative) from every fp32 rounding midpoint because s has an
 * 11-bit significand, so the final rounding is the correct one.  Prints the
 * number of mismatches and exits 1 if there is any.  Build: gcc -O2
 * -ffp-contract=off rcp_newton_check.c -lm. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float half_to_float(uint16_t h) {
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) return ldexpf((float)m, -24);
  return ldexpf((float)(m | 0x400u), (int)e - 25);
}

int main(void) {
  long long bad = 0, total = 0;
  for (int sb = 1; sb < 0x7c00; ++sb) {
    const float s = half_to_float((uint16_t)sb);
    const float y = 1.0f / s;
    const float cand[3] = {nextafterf(y, 0.0f), y, nextafterf(y, INFINITY)};
    for (int i = 0; i < 3; ++i) {
      const float y0 = cand[i];
      const float e = fmaf(-s, y0, 1.0f);
      const float y1 = fmaf(e, y0, y0);
      uint32_t a, b;
      memcpy(&a, &y1, 4);
      memcpy(&b, &y, 4);
      bad += (a != b);
      ++total;
    }
  }
  printf("cases %lld mismatches %lld\n", total, bad);
  return bad != 0;
}
