/* Exhaustive check of the single-multiply smoothing used by the gfx950 activation pass
 * (krea2-svdquant_amd/csrc/svdq_act.hip: smooth64_fast):
 *     x_hat = bf16(RN(x * RN(1/s)))
 * equals the reference's bf16(RN(x / s)) (float32 division, then round to bf16, as torch
 * evaluates bf16 / bf16) for every pair of bf16 operands (all 128 mantissas of each, both
 * signs of x) over the exponent window given on the command line, wherever the exact quotient
 * lies in [2^-90, 2^100] and RN(1/s) is finite (otherwise the kernel takes IEEE division; pairs
 * with an infinite reciprocal are counted as "routed").  Why it holds: x and s
 * carry 8 significant bits, so x / s is never a bf16 rounding midpoint and stays at least
 * 2^-17 (relative) away from one, while RN(x * RN(1/s)) is within 2^-23 of x / s.
 * Prints "mismatches=<n> checked=<n> routed=<n>".  Compile: gcc -O2 -ffp-contract=off ... -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bf16(uint32_t h) { uint32_t u = h << 16; float f; memcpy(&f, &u, 4); return f; }
static uint32_t bf16_rne(float f) {  /* finite f */
  uint32_t u; memcpy(&u, &f, 4);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

int main(int argc, char** argv) {
  int x_lo = argc > 1 ? atoi(argv[1]) : 100, x_hi = argc > 2 ? atoi(argv[2]) : 160;
  int s_lo = argc > 3 ? atoi(argv[3]) : 110, s_hi = argc > 4 ? atoi(argv[4]) : 146;
  long bad = 0, total = 0, routed = 0;
  for (int ex = x_lo; ex <= x_hi; ++ex)
    for (int mx = 0; mx < 128; ++mx)
      for (int sg = 0; sg < 2; ++sg) {
        const float x = from_bf16((uint32_t)(sg << 15 | ex << 7 | mx));
        for (int es = s_lo; es <= s_hi; ++es)
          for (int ms = 0; ms < 128; ++ms) {
            const float s = from_bf16((uint32_t)(es << 7 | ms));
            const double exact = fabs((double)x / (double)s);
            if (x != 0.0f && (exact < 0x1p-90 || exact > 0x1p100)) continue;
            const float rs = 1.0f / s;
            if (isinf(rs)) { ++routed; continue; }
            const float y = x * rs;
            const float ref = x / s;
            ++total;
            if (bf16_rne(y) != bf16_rne(ref)) {
              if (bad < 5) fprintf(stderr, "x=%a s=%a got=%a want=%a\n", x, s, y, ref);
              ++bad;
            }
          }
      }
  printf("mismatches=%ld checked=%ld routed=%ld\n", bad, total, routed);
  return bad != 0;
}
