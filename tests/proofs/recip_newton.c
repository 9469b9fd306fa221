/*
 * Exhaustive check that one FMA Newton step turns ANY faithful fp32
 * approximation r0 of 1/s into the correctly rounded fp32 1/s:
 *     e  = fma(-s, r0, 1)
 *     r1 = fma(e, r0, r0)
 * For each of the 2^23 significands of s in [1, 2) both faithful candidates
 * (1/s rounded down and rounded up) are tried.  The rounding of 1/s depends
 * only on the significand of s as long as 1/s and the intermediate values
 * are normal, which holds for the operator's scales (1e-12 <= s < 2^100).
 * A second pass repeats the check at the binades of s = 1e-12 and s = 2^100.
 * Prints the number of failures; exit status 0 iff none.
 */
#include <fenv.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static long check_binade(int exp_field) {
  long bad = 0;
  for (uint32_t m = 0; m < (1u << 23); ++m) {
    const float s = u2f(((uint32_t)exp_field << 23) | m);
    const float rn = 1.0f / s;                         /* correctly rounded */
    const double exact = 1.0 / (double)s;              /* exact to 2^-53 rel */
    const float lo = (double)rn <= exact ? rn : nextafterf(rn, 0.0f);
    const float hi = (double)rn >= exact ? rn : nextafterf(rn, INFINITY);
    const float cand[2] = {lo, hi};
    for (int c = 0; c < 2; ++c) {
      const float r0 = cand[c];
      const float e = fmaf(-s, r0, 1.0f);
      const float r1 = fmaf(e, r0, r0);
      if (r1 != rn) {
        if (bad < 5) printf("fail s=%a r0=%a r1=%a rn=%a\n", s, r0, r1, rn);
        ++bad;
      }
    }
  }
  return bad;
}

int main(void) {
  fesetround(FE_TONEAREST);
  long bad = 0;
  bad += check_binade(127);          /* s in [1, 2) */
  bad += check_binade(127 - 40);     /* s in [2^-40, 2^-39), holds 1e-12 */
  bad += check_binade(127 + 100);    /* s in [2^100, 2^101) */
  printf("failures %ld\n", bad);
  return bad != 0;
}
