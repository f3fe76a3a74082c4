/* Exhaustive check of the reciprocal-corrected division used by the gfx950 kernels
 * (krea2-svdquant_amd/csrc/svdq_common.h: div_rcp):
 *     q0 = x * rs;  r = fma(-q0, s, x);  q = fma(r, rs, q0),   rs = RN(1/s)
 * equals the IEEE float32 quotient RN(x / s) for every pair of bf16 operands (all 128
 * mantissas of each, both signs) over the exponent window given on the command line.
 * Prints "mismatches=<n> checked=<n>". Compile: gcc -O2 -mfma -ffp-contract=off ... -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bf16(uint32_t h) { uint32_t u = h << 16; float f; memcpy(&f, &u, 4); return f; }

int main(int argc, char** argv) {
  int x_lo = argc > 1 ? atoi(argv[1]) : 100, x_hi = argc > 2 ? atoi(argv[2]) : 160;
  int s_lo = argc > 3 ? atoi(argv[3]) : 110, s_hi = argc > 4 ? atoi(argv[4]) : 146;
  long bad = 0, total = 0;
  for (int ex = x_lo; ex <= x_hi; ++ex)
    for (int mx = 0; mx < 128; ++mx)
      for (int sx = 0; sx < 2; ++sx) {
        const float x = from_bf16((uint32_t)(sx << 15 | ex << 7 | mx));
        for (int es = s_lo; es <= s_hi; ++es)
          for (int ms = 0; ms < 128; ++ms) {
            const float s = from_bf16((uint32_t)(es << 7 | ms));
            const float rs = 1.0f / s;
            const float q0 = x * rs;
            const float r = fmaf(-q0, s, x);
            const float q = fmaf(r, rs, q0);
            const float ref = x / s;
            ++total;
            if (memcmp(&q, &ref, 4) != 0) {
              if (bad < 5) fprintf(stderr, "x=%a s=%a got=%a want=%a\n", x, s, q, ref);
              ++bad;
            }
          }
      }
  printf("mismatches=%ld checked=%ld\n", bad, total);
  return bad != 0;
}
