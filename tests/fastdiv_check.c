/* Checks that q = fma(fma(-x*r, d, x), r, x*r), r = RN(1/d), equals the IEEE
 * quotient x/d for every positive normal float x in [2^-20, 2^24) (the range
 * the HIP phase kernels use it on), for the divisors given on the command
 * line; with "sample" only every 7th float is visited.  Prints the number of
 * mismatches per divisor; exit status 1 if any. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int main(int argc, char** argv) {
  int step = 1, bad_any = 0;
  for (int a = 1; a < argc; ++a) {
    if (!strcmp(argv[a], "sample")) {
      step = 7;
      continue;
    }
    const float d = strtof(argv[a], NULL), r = 1.0f / d;
    float lo_f = ldexpf(1.f, -20), hi_f = ldexpf(1.f, 24);
    uint32_t lo, hi;
    memcpy(&lo, &lo_f, 4);
    memcpy(&hi, &hi_f, 4);
    long bad = 0;
    for (uint32_t u = lo; u < hi; u += step) {
      float x;
      memcpy(&x, &u, 4);
      volatile float ref = x / d;
      const float q0 = x * r;
      const float q = fmaf(fmaf(-q0, d, x), r, q0);
      if (q != ref || -q != (-x) / d) ++bad;
    }
    printf("%g %ld\n", d, bad);
    bad_any |= bad != 0;
  }
  return bad_any;
}
