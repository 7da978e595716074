/*
 * Checks the companding quotient of the quantized Linear's activation path
 * (quantization.py:268, x / compand_scale in the activation dtype T = bf16 or fp16, which
 * torch computes as the fp32 quotient rounded once to T): for every pair of T values x, c
 * with r = fp32(1 / c),
 *     T(fp32(x * r))  ==  T(fp32(x / c))
 * bit for bit (NaN against NaN).  The activation kernel takes the product form for a column
 * whose scale passes uses_product() below -- bf16: c not zero or subnormal; fp16: |c| < 8,
 * which holds the reference's scales exp(clamp(log_scale, -2.079, 2.079)) < 7.9963 -- and
 * the IEEE division for the other columns.
 *
 * usage: compand_div_check bf16|fp16 [exhaustive]
 *   default:    all x against 4096 scales (every 16th pattern);
 *   exhaustive: all 2^16 x against all 2^16 c.
 * Prints the mismatch counts, in all and where uses_product(c) holds, and per exponent
 * field of c the scales with a mismatch; exit status 1 on any mismatch where
 * uses_product(c) holds.
 *
 * usage: compand_div_check conv16 < in.f32 > out.u16
 *   writes the fp16 rounding of every fp32 value read (the conversion the check uses, for
 *   comparison with numpy's float16 cast).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t to_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

/* fp32 -> bf16 bits, round to nearest even, NaN kept NaN */
static uint16_t bf16_rne(float f) {
  const uint32_t u = to_bits(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static float bf16_val(uint16_t h) { return from_bits((uint32_t)h << 16); }

/* fp32 -> fp16 bits, round to nearest even, overflow to infinity, NaN kept NaN */
static uint16_t f16_rne(float f) {
  const uint32_t u = to_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u;
  if (a >= 0x477FF000u) return sign | 0x7C00u; /* >= 65520: the tie above 65504 goes to inf */
  if (a >= 0x38800000u) {                     /* >= 2^-14: a normal fp16 */
    uint32_t h = ((((a >> 23) - 127u + 15u) << 10) | ((a & 0x7FFFFFu) >> 13));
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return sign | (uint16_t)h;
  }
  /* subnormal (or zero): units of 2^-24, round half to even; 1024 units is 2^-14 */
  const double units = (double)from_bits(a) * 16777216.0; /* exact */
  double n = floor(units);
  const double rest = units - n;
  if (rest > 0.5 || (rest == 0.5 && fmod(n, 2.0) != 0.0)) n += 1.0;
  return sign | (uint16_t)n;
}
static float f16_val(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1Fu) return from_bits(sign | 0x7F800000u | (m << 13));
  if (e == 0) return from_bits(sign) + (float)((h & 0x8000u) ? -1.0 : 1.0) * (float)m * 5.9604644775390625e-8f;
  return from_bits(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

static int is_bf16;
static uint16_t rt(float f) { return is_bf16 ? bf16_rne(f) : f16_rne(f); }
static float val(uint16_t h) { return is_bf16 ? bf16_val(h) : f16_val(h); }
static int isnan16(uint16_t h) {
  return is_bf16 ? ((h & 0x7FFFu) > 0x7F80u) : ((h & 0x7FFFu) > 0x7C00u);
}

/* the activation kernel's rule (on the fp32 value of c): which columns take x * r */
static int uses_product(float c) {
  const uint32_t a = to_bits(c) & 0x7FFFFFFFu;
  return is_bf16 ? (a & 0x7F800000u) != 0 : a < 0x41000000u;
}

/* mismatches of the product form over all x for one scale pattern */
static long long bad_for_c(uint16_t cb) {
  const float c = val(cb);
  const float r = 1.0f / c;
  long long bad = 0;
  for (uint32_t xb = 0; xb < 65536u; ++xb) {
    const float x = val((uint16_t)xb);
    const uint16_t want = rt(x / c), got = rt(x * r);
    if (want != got && !(isnan16(want) && isnan16(got))) ++bad;
  }
  return bad;
}

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  if (!strcmp(argv[1], "conv16")) {
    float f;
    while (fread(&f, 4, 1, stdin) == 1) {
      const uint16_t h = f16_rne(f);
      fwrite(&h, 2, 1, stdout);
    }
    return 0;
  }
  is_bf16 = !strcmp(argv[1], "bf16");
  if (!is_bf16 && strcmp(argv[1], "fp16")) return 2;
  const int exhaustive = argc > 2;
  const int step = exhaustive ? 1 : 16;
  const int mbits = is_bf16 ? 7 : 10, ebits = is_bf16 ? 8 : 5;
  static long long bad_c[65536];
#pragma omp parallel for schedule(dynamic, 64)
  for (int cb = 0; cb < 65536; cb += step) bad_c[cb] = bad_for_c((uint16_t)cb);
  long long bad = 0, bad_rule = 0, cs_bad = 0, cs_rule = 0;
  for (int cb = 0; cb < 65536; cb += step) {
    const int rule = uses_product(val((uint16_t)cb));
    cs_rule += rule;
    if (!bad_c[cb]) continue;
    bad += bad_c[cb];
    ++cs_bad;
    if (rule) bad_rule += bad_c[cb];
  }
  printf("%s %s: checked %lld pairs, mismatches %lld over %lld scales; %lld scales take the product, "
         "mismatches there %lld\n",
         argv[1], exhaustive ? "exhaustive" : "sampled", 65536LL * (65536 / step), bad, cs_bad, cs_rule, bad_rule);
  /* per exponent field of c (positive c): how many scales mismatch */
  for (int e = 0; e < (1 << ebits); ++e) {
    int n = 0, first = -1;
    long long pairs = 0;
    for (int m = 0; m < (1 << mbits); ++m) {
      const int cb = (e << mbits) | m;
      if (cb % step) continue;
      if (bad_c[cb]) {
        if (first < 0) first = cb;
        ++n;
        pairs += bad_c[cb];
      }
    }
    if (n) printf("  c exponent field %3d: %d scales (first %.9g), %lld pairs\n", e, n, val((uint16_t)first), pairs);
  }
  return bad_rule != 0;
}
