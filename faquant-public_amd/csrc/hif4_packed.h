// Packed HiF4 rows on gfx950: decoding a row's code and meta words into the HiF4 QDQ values
// (shared by the decode kernels and the packed-weight Linear).
//
// A row holds 128 values: 16 code words, dims 8u .. 8u + 7 in word (u & 1) 8 + u / 2, dim
// 8u + i in nibble i as 8 + the signed code; and 2 meta words, one per 64-dim group: the E6M2
// byte ((e + 48) << 2) | m of the scale 2^e (1 + m / 4), the level-2 bits << 8 and the
// level-3 bits << 16 (the content of hif4.py:67-79).  A value is
// (nibble - 8) 2^(lv2 + lv3) s / 4.
#pragma once

#include "hif4_device.h"

namespace faq {

// s / 4 of a 64-dim group from its meta word (E6M2 byte ((e + 48) << 2) | m in bits 0-7):
// exponent e - 2, mantissa m; an E6M2 byte of 0xFF marks a group that held a NaN (its
// values are NaN).
__device__ __forceinline__ float hif4_group_s4(uint32_t meta) {
  const uint32_t sb = meta & 0xFFu;
  return sb == 0xFFu ? __builtin_nanf("") : __uint_as_float((sb << 21) + (77u << 23));
}

// The 8 values of code word `word` (dims 8 g8 .. 8 g8 + 7 of one 64-dim group with
// s / 4 = s4): (nibble - 8) f = fma(nibble, f, -8 f) with f = 2^(lv2 + lv3) s / 4 of its
// 4-dim group (ldexp: exact, and NaN stays NaN).  The nibbles are converted as bytes of the
// two masked words (even and odd nibbles), four per word.
__device__ __forceinline__ void hif4_unpack8(uint32_t word, float s4, uint32_t meta, int g8, float* v) {
  const int lv2 = static_cast<int>((meta >> (8 + g8)) & 1u);
  const int lv3 = static_cast<int>((meta >> (16 + 2 * g8)) & 3u);
  const float fa = __builtin_ldexpf(s4, lv2 + (lv3 & 1));
  const float fb = __builtin_ldexpf(s4, lv2 + (lv3 >> 1));
  const float na = fa * -8.0f, nb = fb * -8.0f;
  uint32_t lo = word & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 as bytes
  uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
  // (opaque to the compiler, which would otherwise fold each mask into a per-nibble
  // bit-field extract and lose the byte conversions v_cvt_f32_ubyte0..3)
  asm volatile("" : "+v"(lo), "+v"(hi));
  float bl[4], bh[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bl[i] = static_cast<float>(static_cast<uint32_t>(static_cast<uint8_t>(lo >> (8 * i))));
    bh[i] = static_cast<float>(static_cast<uint32_t>(static_cast<uint8_t>(hi >> (8 * i))));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float f = i < 2 ? fa : fb;
    const float nf = i < 2 ? na : nb;
    v[2 * i] = __builtin_fmaf(bl[i], f, nf);
    v[2 * i + 1] = __builtin_fmaf(bh[i], f, nf);
  }
}

}  // namespace faq
