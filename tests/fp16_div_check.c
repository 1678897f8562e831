/*
 * Exhaustive check of the quantizer's fp16-input normalisation: for every
 * fp16 value a and every positive fp16 value d (both widened to fp32),
 *     e = fma(-q0, d, a),  q1 = (e == 0) ? q0 : fma(e, r, q0),   q0 = a * r,   r = 1 / d   (fp32)
 * equals the correctly rounded fp32 quotient a / d bit for bit (Markstein's
 * correction step: with r the correctly rounded reciprocal and the operands
 * and quotient in the normal range, one FMA correction gives the correctly
 * rounded quotient).  The kernel computes r once per vector and q1 per
 * element instead of one IEEE division per element.  e == 0 means q0 is exact
 * (and keeps the sign of a zero quotient, which the correction would turn
 * into +0 for a = -0).  NaN quotients (0/0 when
 * a vector is all zeros and d rounds to 0) are compared as NaN == NaN.
 *
 * Build and run:  gcc -O2 -fopenmp -ffp-contract=off fp16_div_check.c -lm -o fp16_div_check
 *                 ./fp16_div_check [d_stride]   (prints the mismatch count; 0 = pass)
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  float f;
  if (exp == 0) {
    f = ldexpf((float)man, -24);  /* subnormal (or zero) */
    if (sign) f = -f;
    return f;
  }
  if (exp == 31) {
    uint32_t bits = sign | 0x7f800000u | (man << 13);
    memcpy(&f, &bits, 4);
    return f;
  }
  uint32_t bits = sign | ((exp + 112) << 23) | (man << 13);
  memcpy(&f, &bits, 4);
  return f;
}

static uint32_t bits_of(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

int main(int argc, char** argv) {
  const int stride = argc > 1 ? atoi(argv[1]) : 1;
  long long bad = 0, checked = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad, checked)
  for (int dh = 1; dh < 0x7c00; dh += stride) {  /* every positive finite fp16 d */
    const float d = half_to_float((uint16_t)dh);
    const float r = 1.0f / d;
    for (int ah = 0; ah < 0x10000; ++ah) {
      if (((ah >> 10) & 0x1f) == 31) continue;  /* a finite */
      const float a = half_to_float((uint16_t)ah);
      const float ref = a / d;
      const float q0 = a * r;
      const float e = fmaf(-q0, d, a);
      const float q1 = (e == 0.0f) ? q0 : fmaf(e, r, q0);
      const int same = (isnan(ref) && isnan(q1)) || bits_of(ref) == bits_of(q1);
      bad += !same;
      checked += 1;
    }
  }
  printf("checked %lld pairs, mismatches %lld\n", checked, bad);
  return bad != 0;
}
