/* The prepass divides by a fixed scale s as
 *   q = x * r;  q' = fmaf(fmaf(-q, s, x), r, q)   with r = 1/s correctly rounded
 * and relies on q' == x / s (IEEE, round to nearest even) for every quotient of
 * magnitude >= 2^-12.  This program checks that identity over a sweep of
 * scales (mantissas near 0, near all-ones, random) and of x at every 2^e
 * binade of the quotient from 2^-12 to 2^9, with a mantissa stride argv[1].
 * The result carries x's sign (copysignf): for x = -0, or a product x * r
 * that underflows to -0, the correction alone would give +0.  Quotients below
 * 2^-12 (x = +-0, denormal and tiny x) must encode to E4M3 zero on both sides
 * (magnitude < 2^-10) with the same sign.
 * Exit status 0 iff no mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float fu(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t uf(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 7u;
  const int nscale = argc > 2 ? atoi(argv[2]) : 400;
  unsigned long long bad = 0, tot = 0;
  srand(1);
  for (int t = 0; t < nscale; ++t) {
    uint32_t sm;
    if (t == 0) sm = 0;
    else if (t == 1) sm = 0x7fffff;
    else if (t < nscale / 10) sm = 0x7fffff - (uint32_t)(rand() % 64);
    else if (t < nscale / 5) sm = (uint32_t)(rand() % 64);
    else sm = (((uint32_t)rand() << 8) ^ (uint32_t)rand()) & 0x7fffff;
    const int se = 100 + rand() % 40; /* scale 2^-27 .. 2^12 */
    const float s = fu(((uint32_t)se << 23) | sm);
    const float r = 1.0f / s;
    for (int e = -12; e <= 9; ++e) {
      const uint32_t be = (uf(s * ldexpf(1.0f, e)) >> 23) & 0xff;
      for (uint32_t m = 0; m < (1u << 23); m += stride) {
        for (uint32_t sg = 0; sg < 2; ++sg) {
          const float x = fu((sg << 31) | (be << 23) | m);
          const float q = x * r;
          const float q1 = copysignf(fmaf(fmaf(-q, s, x), r, q), x);
          const float ex = x / s;
          ++tot;
          if (uf(q1) != uf(ex)) {
            if (bad < 5) printf("mismatch s=%a x=%a got=%a want=%a\n", s, x, q1, ex);
            ++bad;
          }
        }
      }
    }
    /* zero, denormal and tiny x: quotients below 2^-12 */
    for (int k = -1; k < 300; ++k) {
      uint32_t mag;
      if (k < 0) mag = 0u;                                   /* +-0 */
      else if (k < 100) mag = (uint32_t)(rand() & 0x7fffff); /* denormals */
      else mag = (uf(s * ldexpf(1.0f, -13 - (k % 40))) & 0x7f800000u) | ((uint32_t)rand() & 0x7fffff);
      for (uint32_t sg = 0; sg < 2; ++sg) {
        const float x = fu((sg << 31) | mag);
        const float q = x * r;
        const float q1 = copysignf(fmaf(fmaf(-q, s, x), r, q), x);
        const float ex = x / s;
        ++tot;
        if (signbit(q1) != signbit(ex) || fabsf(q1) >= 0x1p-10f || fabsf(ex) >= 0x1p-10f) {
          if (bad < 5) printf("small-quotient mismatch s=%a x=%a got=%a want=%a\n", s, x, q1, ex);
          ++bad;
        }
      }
    }
  }
  printf("checked %llu, mismatches %llu\n", tot, bad);
  return bad != 0;
}
