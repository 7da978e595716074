// Decode-shaped HiF4 W4A4 Linear over packed weights: arguments and launcher.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace faq {

// Waves per workgroup of the packed-weight Linear; every wave owns `rows_per_wave` output
// features.
constexpr int kLinWaves = 4;
// At most this many rows of x per call (decode steps, small batches).
constexpr int kLinMaxRows = 8;

struct LinArgs {
  const uint16_t* x;  // bf16 [M, K], row stride x_sm elements, last stride 1
  int64_t x_sm;
  // packed HiF4 weight rows: row r = n nkb + j holds columns 128 j .. 128 j + 127 of output
  // feature n (16 code words and 2 meta words per row, the decode caches' row format)
  const uint32_t* wc;
  const uint32_t* wm;
  const void* bias;  // [N] fp32 or bf16, or null
  int bias_f32;
  void* y;  // [M, N] fp32 or bf16, row stride y_sm elements, last stride 1
  int y_f32;
  int64_t y_sm;
  int M, N, K;
  int nkb;  // K / 128
};

// rows_per_wave: 1, 2 or 4; the grid covers ceil(N / rows_per_wave) waves.
void launch_linear_packed(const LinArgs& a, int rows_per_wave, hipStream_t st);

}  // namespace faq
