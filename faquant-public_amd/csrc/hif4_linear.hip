// Decode-shaped HiF4 W4A4 Linear on gfx950: y = x W^T (+ bias) for a few rows x (at most 8)
// over packed HiF4 weights (4.5 bits per weight), the contraction of FakeQuantLinear.forward
// (src/faquant/quantization.py:199-277, F.linear on the HiF4-exact operands) where reading the
// weight dominates: decode steps and small batches.
//
// Work: each wave owns R consecutive output features and reads their packed rows whole.  Lane
// pair (2 b, 2 b + 1) takes 128-column block j = 32 i + b (i = 0, 1, ..), the lane of the pair
// `h` its code words 8 h .. 8 h + 7 (dims 128 j + 16 c + 8 h .. + 7, c < 8) and the block's two
// meta words: a wave reads 32 consecutive blocks of a row (2 KiB of codes) per instruction
// pair.  The lane decodes its words in registers (the decode caches' unpack), packs the exact
// values as bf16 pairs and accumulates v_dot2_f32_bf16 against the same dims of each x row,
// in a fixed order (blocks, chunks, pairs); the 64 lane sums of a feature are then added by a
// fixed butterfly (lane distances 1, 2, .., 32).  No workspace, no counters and no
// communication between waves: every call gives the same bits.  The fp32 sums run in another
// order than the library GEMM of F.linear, so the two agree to fp32 rounding, and the bf16
// results to one ulp.
#include "hif4_linear.h"
#include "hif4_packed.h"

namespace faq {
namespace {

typedef unsigned int lin_u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 lin_bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ lin_bf16x2 as_bf16x2(uint32_t u) {
  lin_bf16x2 r;
  __builtin_memcpy(&r, &u, 4);
  return r;
}

// The code words (8 h .. 8 h + 7) and the two meta words of one packed row.
struct LinWords {
  lin_u32x4 lo, hi;
  uint32_t ma, mb;
};

__device__ __forceinline__ LinWords lin_load(const LinArgs& a, int64_t row, int h) {
  LinWords w;
  const uint32_t* cp = a.wc + row * 16 + 8 * h;
  w.lo = *reinterpret_cast<const lin_u32x4*>(cp);
  w.hi = *reinterpret_cast<const lin_u32x4*>(cp + 4);
  const uint2 mm = *reinterpret_cast<const uint2*>(a.wm + row * 2);
  w.ma = mm.x;
  w.mb = mm.y;
  return w;
}

__device__ __forceinline__ float lin_bias(const LinArgs& a, int n) {
  if (a.bias == nullptr) return 0.0f;
  return a.bias_f32 ? static_cast<const float*>(a.bias)[n] : bf16_bits_to_f32(static_cast<const uint16_t*>(a.bias)[n]);
}

template <int MR, int R>
__global__ __launch_bounds__(256) void linear_gemv_kernel(LinArgs a) {
  const int lane = threadIdx.x & 63;
  const int h = lane & 1;
  const int b = lane >> 1;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kLinWaves + static_cast<int>(threadIdx.x >> 6));
  const int n0 = wave * R;
  if (n0 >= a.N) return;

  float acc[R][MR];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;

  for (int i = 0; 32 * i < a.nkb; ++i) {
    const int j = 32 * i + b;
    const bool jv = j < a.nkb;
    const int jc = jv ? j : a.nkb - 1;  // a lane past the last block reads it again; its sums are dropped
    LinWords w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = lin_load(a, static_cast<int64_t>(min(n0 + r, a.N - 1)) * a.nkb + jc, h);
    float part[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m) part[r][m] = 0.0f;
    float s4[R][2];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      s4[r][0] = hif4_group_s4(w[r].ma);
      s4[r][1] = hif4_group_s4(w[r].mb);
    }
    const uint16_t* xb = a.x + static_cast<int64_t>(jc) * 128 + 8 * h;
    // x's chunks in groups loaded before they are used: left to itself the compiler issues each
    // chunk's load after the previous chunk's products, one memory round trip per chunk.  Per
    // Qwen3-8B layer: eight rows of x in groups of 2, 156 against 172 us; four rows keep the
    // compiler's order (groups of 4: 95.9 against 88.9 us); one or two rows load all 8 chunks
    // (the same time either way).
    constexpr int kXG = MR <= 2 ? 8 : MR == 4 ? 1 : 2;
#pragma unroll
    for (int cg = 0; cg < 8; cg += kXG) {
      lin_u32x4 xp[kXG][MR];
#pragma unroll
      for (int cc = 0; cc < kXG; ++cc)
#pragma unroll
        for (int m = 0; m < MR; ++m)
          xp[cc][m] = *reinterpret_cast<const lin_u32x4*>(xb + static_cast<int64_t>(min(m, a.M - 1)) * a.x_sm + 16 * (cg + cc));
      if constexpr (kXG > 1) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int cc = 0; cc < kXG; ++cc) {
        const int c = cg + cc;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float v[8];
          const uint32_t word = c < 4 ? w[r].lo[c & 3] : w[r].hi[c & 3];
          hif4_unpack8(word, s4[r][c >> 2], c < 4 ? w[r].ma : w[r].mb, 2 * (c & 3) + h, v);
          uint32_t p[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            p[q] = __builtin_amdgcn_perm(__float_as_uint(v[2 * q + 1]), __float_as_uint(v[2 * q]), 0x07060302u);
#pragma unroll
          for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              part[r][m] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(p[q]), as_bf16x2(xp[cc][m][q]), part[r][m], false);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[r][m] += jv ? part[r][m] : 0.0f;
  }

  // the 64 lane sums of each (feature, row): a fixed butterfly
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) acc[r][m] += __shfl_xor(acc[r][m], d, 64);

  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = n0 + r;
      if (n >= a.N) continue;
      const float bn = lin_bias(a, n);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m >= a.M) continue;
        const float o = acc[r][m] + bn;
        if (a.y_f32) static_cast<float*>(a.y)[static_cast<int64_t>(m) * a.y_sm + n] = o;
        else static_cast<uint16_t*>(a.y)[static_cast<int64_t>(m) * a.y_sm + n] = static_cast<uint16_t>(pack2_bf16_hw(o, 0.0f) & 0xFFFFu);
      }
    }
  }
}

template <int MR>
void launch_mr(const LinArgs& a, int rows_per_wave, hipStream_t st) {
  const int64_t waves = (static_cast<int64_t>(a.N) + rows_per_wave - 1) / rows_per_wave;
  const dim3 grid(static_cast<unsigned>((waves + kLinWaves - 1) / kLinWaves));
  if (rows_per_wave == 4) hipLaunchKernelGGL((linear_gemv_kernel<MR, 4>), grid, dim3(64 * kLinWaves), 0, st, a);
  else if (rows_per_wave == 2) hipLaunchKernelGGL((linear_gemv_kernel<MR, 2>), grid, dim3(64 * kLinWaves), 0, st, a);
  else hipLaunchKernelGGL((linear_gemv_kernel<MR, 1>), grid, dim3(64 * kLinWaves), 0, st, a);
}

}  // namespace

void launch_linear_packed(const LinArgs& a, int rows_per_wave, hipStream_t st) {
  if (a.M <= 1) launch_mr<1>(a, rows_per_wave, st);
  else if (a.M <= 2) launch_mr<2>(a, rows_per_wave, st);
  else if (a.M <= 4) launch_mr<4>(a, rows_per_wave, st);
  else launch_mr<8>(a, rows_per_wave, st);
}

}  // namespace faq
