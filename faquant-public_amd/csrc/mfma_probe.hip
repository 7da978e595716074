// MFMA rate probe: the dense bf16 rate the attention kernel's MFMA shape can sustain on
// this device, as the measured reference point next to the 2.5 PF/s specification peak.
// Same launch shape as attn_fwd_kernel (512 threads, two waves per SIMD, one workgroup
// per CU); each wave runs four independent v_mfma_f32_32x32x16_bf16 accumulation chains
// (no other instructions in the loop).  FLOP = blocks * 8 waves * iters * 4 * 32768.
#pragma once
#include "hif4_device.h"

namespace faq {

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfma_probe_kernel(float* out, int iters) {
  const int t = threadIdx.x;
  bf16x8 a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = static_cast<__bf16>(static_cast<float>((t + j) % 5 - 2) * 0.125f);
    b[j] = static_cast<__bf16>(static_cast<float>((t * 3 + j) % 7 - 3) * 0.125f);
  }
  floatx16 c0{}, c1{}, c2{}, c3{};
  for (int i = 0; i < iters; ++i) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, b, c3, 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  out[static_cast<int64_t>(blockIdx.x) * blockDim.x + t] = s;
}

// Stream probe: the read rate a plain coalesced stream reaches on this device, the measured
// reference point next to the 8 TB/s specification for the HBM-bound decode kernels.
// 256-thread workgroups read `n16` 16-byte units in a grid-stride loop, four independent
// 16-byte loads per thread in flight, and write one word per workgroup (so that the loads are
// not removed).
__global__ __launch_bounds__(256) void stream_probe_kernel(const uint4* __restrict__ x, int64_t n16, float* out) {
  uint32_t acc = 0;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 1024 + threadIdx.x;
  const int64_t step = static_cast<int64_t>(gridDim.x) * 1024;
  for (; i + 768 < n16; i += step) {
    const uint4 a = x[i], b = x[i + 256], c = x[i + 512], d = x[i + 768];
    acc += (a.x ^ a.y ^ a.z ^ a.w) + (b.x ^ b.y ^ b.z ^ b.w) + (c.x ^ c.y ^ c.z ^ c.w) + (d.x ^ d.y ^ d.z ^ d.w);
  }
  for (; i < n16; i += 256) {
    const uint4 a = x[i];
    acc += a.x ^ a.y ^ a.z ^ a.w;
  }
  acc += __shfl_xor(acc, 1, 64);
  if (threadIdx.x == 0) out[blockIdx.x] = static_cast<float>(acc);
}

}  // namespace faq
