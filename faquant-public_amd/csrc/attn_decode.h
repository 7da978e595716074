// Decode-shaped HiF4 attention (few query rows per KV head): arguments and launchers.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace faq {

// Waves per decode workgroup; every wave is an independent (item, key split).
constexpr int kDecWaves = 4;

struct DecodeArgs {
  const uint16_t* q;  // bf16 [B, Hq, Lq, 128] at element strides, last stride 1
  int64_t q_sb, q_sh, q_sl;
  // bf16 operands: K and V [B, Hkv, Lk, 128] at element strides, last stride 1
  const uint16_t* k;
  int64_t k_sb, k_sh, k_sl;
  const uint16_t* v;
  int64_t v_sb, v_sh, v_sl;
  // packed HiF4 operands (one 128-value row per key): 16 code words (dims 8u .. 8u + 7 in
  // word (u & 1) 8 + u / 2, dim 8u + i in nibble i, nibble = 8 + signed code) and 2 meta words (per 64-dim
  // group: E6M2 byte | level-2 bits << 8 | level-3 bits << 16); strides in key rows
  const uint32_t* kc;
  const uint32_t* km;
  int64_t kp_sb, kp_sh;
  const uint32_t* vc;
  const uint32_t* vm;
  int64_t vp_sb, vp_sh;
  int B, Hq, Hkv, Lq, Lk;
  int causal;
  float c1;       // softmax scale * log2(e)
  int G;          // query heads per KV head (<= 32)
  int pb;         // positions per 32-row block: 32 / G
  int n_rb;       // row blocks per KV head: ceil(Lq / pb)
  int ntiles;     // ceil(Lk / 128)
  int tps;        // key tiles per split
  int nsplit;
  int rows_total;  // B Hq Lq; row r = (b Hq + hq) Lq + pos
  float* s;        // scores S (masked keys -inf) [rows_total, s_stride], s_stride >= 128 ntiles
  int64_t s_stride;
  float* gmx;      // lane maxima of S per tile: [rows_total, ntiles, 2] (keys 0-63, 64-127)
  float* smx;      // row maximum of S per split: [rows_total, nsplit]
  float* part_o;   // unnormalized O per split: [nsplit, rows_total, 128]
  float* part_lm;  // (l, running maximum) per split: [nsplit, rows_total, 2]
};

// Scores pass, then the values pass (partials per split; the caller combines them).
void launch_decode(const DecodeArgs& a, int packed, int quant_p, int p_levels, int norm_same, hipStream_t st);

// The one-pass form of the same (the same partials, bitwise): decode steps with P quantized,
// the quantized-same normalizer, at most 8 live columns per row block, one key tile per
// split and at most 64 key tiles.  epoch: nonzero, different for every call; spin_limit: rounds a split
// waits for the maxima of the splits before it before computing them itself (< 0: always).
bool decode_fused_fits(const DecodeArgs& a, int quant_p, int norm_same);
void launch_decode_fused(const DecodeArgs& a, int packed, int p_levels, uint32_t epoch, int spin_limit, hipStream_t st);

}  // namespace faq
