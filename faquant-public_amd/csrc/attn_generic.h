// General-shape HiF4 attention (any head_dim up to 256, any key tile up to 1024, fp32, bf16
// or fp16 operands multiplied in fp32): arguments and launcher.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace faq {

constexpr int kGenRows = 16;         // query rows per workgroup
constexpr int kGenMaxDim = 256;      // head_dim limit
constexpr int kGenMaxTile = 1024;    // key tile limit
constexpr int kGenChunk = 32;        // keys staged in LDS at a time

struct GenAttnArgs {
  // operands [B, H, L, D] at element strides (last stride 1); dtype 0 fp32, 1 bf16, 2 fp16
  const void* q;
  int q_dt;
  int64_t q_sb, q_sh, q_sl;
  const void* k;
  int k_dt;
  int64_t k_sb, k_sh, k_sl;
  const void* v;
  int v_dt;
  int64_t v_sb, v_sh, v_sl;
  void* o;  // [B, Hq, Lq, D], dtype as the operands
  int o_dt;
  int64_t o_sb, o_sh, o_sl;
  int B, Hq, Hkv, Lq, Lk, D, T;
  int causal;
  float scale;
  float softcap;  // > 0: scores -> softcap tanh(scores / softcap) after the scale
  int quant_p;    // HiF4 QDQ of P per 64-key group of each key tile
  int p_levels;
  int norm_same;  // the normalizer sums P^ (quantized_same) instead of P
  float* row_den;  // optional fp32 [B, Hq, Lq]
  // key ranges (all or none): query position p of batch b sees the keys in
  // [row_lo[b Lq + p], row_hi[b Lq + p]] whose bit in key_bits[b key_words + k / 32] is set
  const int* row_lo;
  const int* row_hi;
  const uint32_t* key_bits;
  int64_t key_words;
  // dense additive mask: fp32 [b, h, p, k] at element strides (0 broadcasts); -inf masks
  const float* amask;
  int64_t am_sb, am_sh, am_sq;
  float* diag;  // PV-normalizer probe sums per row, [B, Hq, Lq, 5] (needs quant_p)
};

// Dynamic LDS bytes of one workgroup for head_dim D and key tile T.
size_t gen_attention_lds_bytes(int D, int T);

// hipSuccess, or the error of raising the kernel's dynamic LDS limit (nothing launched).
hipError_t launch_gen_attention(const GenAttnArgs& a, hipStream_t st);

}  // namespace faq
