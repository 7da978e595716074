// HiF4 arithmetic on gfx950: device helpers shared by the quantizer, the operand
// prologue and the attention kernel.
//
// Every function here reproduces src/faquant/hif4.py of the reference bit for bit
// (the steps are IEEE float32 operations or exact power-of-two scalings):
//   bf16_rne          hif4.py:87-88   fp32 -> bf16 round-to-nearest-even -> fp32
//   hif4_scale        hif4.py:91-115  E6M2 base scale and its bf16 reciprocal
//   hif4_micro        hif4.py:200-213 level-2/level-3 micro exponents
//   hif4_element      hif4.py:255-271 floor(|x| qm 4 + 0.5) clamped at 7, times ds/4
// The translation unit must be compiled with -ffp-contract=off: `a * b + c` must
// round twice, exactly as torch's separate elementwise kernels do.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace faq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

__device__ __forceinline__ float bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  return __uint_as_float(u);
}

// fp32 -> bf16 -> fp32 with the hardware conversion (v_cvt_pk_bf16_f32): round to nearest
// even like bf16_rne for every non-NaN input (checked exhaustively on gfx950), and a NaN
// stays a NaN (bf16_rne can carry a NaN's payload into infinity).
__device__ __forceinline__ float bf16_round_hw(float x) {
  const __bf16 h = static_cast<__bf16>(x);
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return __uint_as_float(static_cast<uint32_t>(u) << 16);
}

// Two fp32 values rounded to bf16 (hardware conversion, as bf16_round_hw) and packed, the
// first in the low half: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2_bf16_hw(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  const bf16x2v r = __builtin_convertvector((f32x2){lo, hi}, bf16x2v);
  uint32_t u;
  __builtin_memcpy(&u, &r, 4);
  return u;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Upper half of an fp32 whose value is exactly representable in bf16.
__device__ __forceinline__ uint16_t f32_to_bf16_bits_exact(float x) {
  return static_cast<uint16_t>(__float_as_uint(x) >> 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits_rne(float x) {
  return static_cast<uint16_t>(__float_as_uint(bf16_rne(x)) >> 16);
}

// 2^k for |k| well inside the normal range.
__device__ __forceinline__ float pow2i(int k) {
  return __uint_as_float(static_cast<uint32_t>(127 + k) << 23);
}

// bf16(1/7) for levels 123, bf16(1/3.5) for levels 12 and 13 (hif4.py:102, 192).
template <int LV>
__device__ __forceinline__ constexpr float divisor_reciprocal() {
  return LV == 123 ? 0.142578125f : 0.28515625f;
}

// E6M2 scale s = 2^e (1 + m/4) and rec = bf16(fp32(1/s)) of a block maximum.
//   s0 = bf16(max * bf16(1/div)), clamped to [2^-48, 49152]; the two-bit significand
//   rounding with ties to even is an integer add on the bit pattern (the carry into
//   the exponent field is the E6M2 carry).  1/s = 2^-e / (1 + m/4), and because the
//   exponent shift is exact, bf16(fp32(1/s)) = T[m] * 2^-e with the four-entry table
//   T[m] = bf16(fp32(1 / (1 + m/4))) = {1, 0.80078125, 0.66796875, 0.5703125}.
template <int LV>
__device__ __forceinline__ void hif4_scale(float m1, float& s, float& rec) {
  float s0 = bf16_rne(m1 * divisor_reciprocal<LV>());
  s0 = fminf(fmaxf(s0, 0x1p-48f), 49152.0f);
  uint32_t b = __float_as_uint(s0);
  b = (b + 0x000FFFFFu + ((b >> 21) & 1u)) & 0xFFE00000u;
  s = __uint_as_float(b);
  const uint32_t m = (b >> 21) & 3u;
  const int e = static_cast<int>(b >> 23) - 127;
  const uint32_t t = m == 0 ? 0x3F800000u : m == 1 ? 0x3F4D0000u : m == 2 ? 0x3F2B0000u : 0x3F120000u;
  rec = __uint_as_float(static_cast<uint32_t>(static_cast<int>(t) - e * (1 << 23)));
}

// Micro exponents of two adjacent 4-value groups that form one 8-value group.
// Returns k = lv2 + lv3 for each 4-group; the reference's per-value multipliers are
// qm = rec 2^-k and ds = s 2^k (hif4.py:236-239).  Comparisons use fp32 products
// m3 * rec; the 8-group maximum's product is the larger of the two (rounding is
// monotonic), and the lv3 test (m3 rec) / 2^lv2 >= 2 is m3 rec >= 2^(1+lv2).
template <int LV>
__device__ __forceinline__ void hif4_micro(float m3a, float m3b, float rec, int& ka, int& kb) {
  const float t3a = m3a * rec;
  const float t3b = m3b * rec;
  if (LV == 123) {
    const float t2 = fmaxf(t3a, t3b);
    const int e2 = t2 >= 4.0f;
    const float thr = e2 ? 4.0f : 2.0f;
    ka = e2 + (t3a >= thr);
    kb = e2 + (t3b >= thr);
  } else if (LV == 12) {
    const int e2 = fmaxf(t3a, t3b) >= 2.0f;
    ka = e2;
    kb = e2;
  } else {
    ka = t3a >= 2.0f;
    kb = t3b >= 2.0f;
  }
}

// Per-4-group multipliers: qm4 = 4 rec 2^-k, dq = s 2^k / 4 (both exact scalings).
__device__ __forceinline__ void hif4_group_mults(float s, float rec, int k, float& qm4, float& dq) {
  qm4 = rec * pow2i(2 - k);
  dq = s * pow2i(k - 2);
}

// Magnitude QDQ of one value a = |x| >= 0:
//   min(floor(fp32(fp32(a qm) * 4) + 0.5), 7) * ds / 4, where fp32(a qm) * 4 = fp32(a qm4).
__device__ __forceinline__ float hif4_element(float a, float qm4, float dq) {
  const float t = a * qm4;
  const float u = t + 0.5f;
  const float c = fminf(floorf(u), 7.0f);
  return c * dq;
}

// Code index 0..7 of the same value (for the packed format).
__device__ __forceinline__ uint32_t hif4_code(float a, float qm4) {
  const float t = a * qm4;
  const float u = t + 0.5f;
  return static_cast<uint32_t>(fminf(floorf(u), 7.0f));
}


// In-register butterfly stage of stride S (1, 2 or 4) on 8 consecutive values: each pair
// (i, i + S) becomes (left + right, left - right), the order of rotation.py:21-28.
template <int S>
__device__ __forceinline__ void fwht_inlane_stage(float* v) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if ((i & S) == 0) {
      const float l = v[i];
      const float r = v[i + S];
      v[i] = l + r;
      v[i + S] = l - r;
    }
  }
}

// Division by d = fp32(sqrt(n)) with the result of the IEEE division x / d (the reference
// divides by math.sqrt(n), rotation.py:28).  For square n the divisor is a power of two
// and x * (1/d) is exact.  Otherwise q = x r (r = fp32(1/d)), e = fma(-q, d, x) (the exact
// remainder) and fma(e, r, q) equal x / d for every fp32 x whose exponent field lies in
// [22, 254] (checked exhaustively for n = 2, 8, 32, 128, 512: tests/fp_div_check.c); a
// lane holding a smaller magnitude (zeros included), an infinity or a NaN takes the IEEE
// division for its 8 values.
struct SqrtDiv {
  float d;   // fp32(sqrt(n))
  float r;   // fp32(1 / d)
  int pow2;  // d is a power of two
};

__device__ __forceinline__ void div_sqrt_n(float* v, const SqrtDiv& s) {
  if (s.pow2) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * s.r;
    return;
  }
  float y[8];
  float lo = fabsf(v[0]), hi = fabsf(v[0]);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float q = v[i] * s.r;
    const float e = __builtin_fmaf(-q, s.d, v[i]);
    y[i] = __builtin_fmaf(e, s.r, q);
    lo = fminf(lo, fabsf(v[i]));
    hi = fmaxf(hi, fabsf(v[i]));
  }
  // exponent field >= 22 is |x| >= 2^-105; a NaN fails the comparisons
  if (!(lo >= 0x1p-105f && hi <= 3.40282347e38f)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = v[i] / s.d;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = y[i];
}

}  // namespace faq
