/*
 * Checks the division the Hadamard kernels use for the reference's x / math.sqrt(n)
 * (rotation.py:28): for d = fp32(sqrt(n)) and r = fp32(1 / d),
 *     q = x * r;  e = fma(-q, d, x);  y = fma(e, r, q)
 * must equal the IEEE fp32 division x / d bit for bit for every x whose exponent field is
 * in [22, 254] (the kernels send every other x to the IEEE division).
 *
 * usage: fp_div_check N [exhaustive]
 *   default: every binade of the range, both signs, 65536 mantissas per binade (the
 *            first and last 256 and an evenly spaced set in between);
 *   exhaustive: all 2^31 non-negative patterns in the range, both signs.
 * Prints the mismatch count; exit status 1 on any mismatch.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t to_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

static int check(uint32_t u, float d, float r) {
  const float x = from_bits(u);
  const float q = x * r;
  const float e = fmaf(-q, d, x);
  const float y = fmaf(e, r, q);
  return to_bits(y) != to_bits(x / d);
}

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  const int n = atoi(argv[1]);
  const int exhaustive = argc > 2;
  const float d = (float)sqrt((double)n);
  const float r = 1.0f / d;
  long long bad = 0, done = 0;
  for (uint32_t ex = 22; ex <= 254; ++ex) {
#pragma omp parallel for reduction(+ : bad, done) schedule(static)
    for (long long k = 0; k < (exhaustive ? (1LL << 23) : 65536LL); ++k) {
      uint32_t m;
      if (exhaustive) m = (uint32_t)k;
      else if (k < 256) m = (uint32_t)k;
      else if (k >= 65536 - 256) m = (uint32_t)((1u << 23) - (65536 - k));
      else m = (uint32_t)(k * 127u + 97u) & 0x7FFFFFu;
      const uint32_t u = (ex << 23) | m;
      bad += check(u, d, r) + check(u | 0x80000000u, d, r);
      done += 2;
    }
  }
  printf("n=%d checked %lld mismatches %lld\n", n, done, bad);
  return bad != 0;
}
