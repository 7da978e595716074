/*
 * Host restatement of the attention kernel's softcap tanh (softcap_tanh in
 * faquant-public_amd/csrc/hif4_attention.hip): for x = |u|,
 *     x < 0.625:  x + (x x^2) q(x^2), q a degree-4 polynomial (Horner, fma)
 *     otherwise:  1 - 2 r,  r = 1 / (exp2(2 log2(e) x) + 1)
 * with the sign of u.  The GPU's v_exp_f32 and v_rcp_f32 are within 1 ulp; here exp2f and
 * the IEEE reciprocal stand in for them, and every result is also evaluated with each of
 * them moved by one ulp either way.  The error against tanh() in double is reported in
 * fp32 ulps of the exact result.
 *
 * usage: tanh_check [stride]   (every stride-th fp32 pattern of [0, 12]; default 61)
 * Prints the worst error; exit status 1 above 3 ulp.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t to_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float step(float x, int d) { return d == 0 ? x : nextafterf(x, d > 0 ? INFINITY : 0.0f); }

static float softcap_tanh(float u, int de, int dr) {
  const float x = fabsf(u);
  const float t = x * x;
  float p = fmaf(t, -0.005705005954951048f, 0.020639128983020782f);
  p = fmaf(t, p, -0.05373973771929741f);
  p = fmaf(t, p, 0.13331443071365356f);
  p = fmaf(t, p, -0.3333328068256378f);
  const float small = fmaf(x * t, p, x);
  const float e = step(exp2f(x * 2.8853900817779268f), de);
  const float r = step(1.0f / (e + 1.0f), dr);
  const float big = 1.0f - (r + r);
  return copysignf(x < 0.625f ? small : big, u);
}

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], NULL, 10) : 61u;
  const uint32_t last = to_bits(12.0f);
  double worst = 0.0;
  float worst_x = 0.0f;
  for (uint32_t u = 1; u <= last; u += stride) {
    const float x = from_bits(u);
    const double ref = tanh((double)x);
    const double ulp = (double)nextafterf((float)ref, INFINITY) - (double)(float)ref;
    for (int de = -1; de <= 1; ++de)
      for (int dr = -1; dr <= 1; ++dr) {
        const double err = fabs((double)softcap_tanh(x, de, dr) - ref) / ulp;
        if (err > worst) {
          worst = err;
          worst_x = x;
        }
        /* odd symmetry */
        if (to_bits(softcap_tanh(-x, de, dr)) != (to_bits(softcap_tanh(x, de, dr)) ^ 0x80000000u)) {
          printf("sign mismatch at %.9g\n", x);
          return 1;
        }
      }
  }
  /* saturation and special values */
  if (softcap_tanh(100.0f, 0, 0) != 1.0f || softcap_tanh(-1e30f, 0, 0) != -1.0f || !isnan(softcap_tanh(NAN, 0, 0)) ||
      softcap_tanh(0.0f, 0, 0) != 0.0f) {
    printf("special values wrong\n");
    return 1;
  }
  printf("worst %.3f ulp at %.9g\n", worst, worst_x);
  return worst <= 3.0 ? 0 : 1;
}
