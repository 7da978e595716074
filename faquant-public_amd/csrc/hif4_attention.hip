// HiF4 QK/PV flash attention forward on gfx950 (MI355X).
//
// Reference semantics: src/faquant/simulated_flash_attention.py:457-909 (tiled online
// softmax, bottom-right causal mask, fully-future tile skip, P-Reordering) and
// src/faquant/wan22_attention.py:105-183 (non-causal kernel, exp2 on log2-scaled
// scores).  Per query row and per 128-key tile in ascending key order:
//   S = Q^ K^T (bf16 MFMA, fp32 accumulate), masked keys -> -inf
//   m' = max(m, rowmax S * c1)            c1 = scale * log2(e)
//   P  = exp2(S c1 - m'),  alpha = exp2(m - m')
//   P^ = HiF4(P) along keys in 64-key groups aligned at the tile start
//   l  = alpha l + sum(P^ or P);  acc = alpha acc + P^ V^
// and O = acc / l (0 where l == 0).  HiF4-quantized Q/K/V/P values carry at most six
// significant bits, so they are exact bf16 MFMA operands.
//
// Work decomposition: a 256-thread workgroup owns 128 query rows that share one KV
// head (GQA: up to 4 query heads x 32 positions), so each K/V tile staged in LDS is
// reused by every row of the group.  Each wave owns 32 rows.
//
// MFMA layout (v_mfma_f32_32x32x16_bf16; lane l, m = l % 32, half = l / 32):
//   QK computes S^T = K Q^T.  The B operand is the wave's Q fragment (lane holds
//   Q[row m][16c + 8 half .. +7]); the A operand row m of key block kb is key
//   pi(kb, m) = 64 ((m >> 2) & 1) + 16 kb + 4 (m >> 3) + (m & 3).  With the C layout
//   (register i of lane l is C[8 (i/4) + 4 half + i%4][m]) lane (m, half) then holds
//   keys 64 half + 16 kb + i of query row m: each lane half owns one whole 64-key HiF4
//   group of its row, in key order, so all group maxima are lane-local.
//   PV computes O^T = V^T P^T.  For k-chunk c the B operand slots 8 half + t are keys
//   64 half + 8 c + t, i.e. this lane's own P values (8c .. 8c+7), and the A operand is
//   the matching 16-byte run of the transposed V tile.  The row sum of P^ (P-Reordering)
//   is one more MFMA against an all-ones A operand.
// LDS tiles are 128 rows x 256 bytes with the 16-byte pieces XOR-swizzled per row so
// that the MFMA operand reads of 16 consecutive lanes hit distinct banks.
#include "hif4_device.h"

namespace faq {

constexpr int kKeyTile = 128;
constexpr int kDim = 128;

struct AttnArgs {
  const uint16_t* q;  // bf16 [B, Hq, Lq, 128] (any strides, last stride 1)
  int64_t q_sb, q_sh, q_sl;
  const uint16_t* k;  // bf16 [B, Hkv, Lk, 128]
  int64_t k_sb, k_sh, k_sl;
  const uint16_t* vt;  // bf16 [B, Hkv, 128, Lpad] transposed V, zero past Lk
  int64_t v_sb, v_sh, v_sd;
  void* o;  // [B, Hq, Lq, 128] via strides, fp32 or bf16
  int64_t o_sb, o_sh, o_sl;
  int o_f32;
  int B, Hq, Hkv, Lq, Lk;
  int causal;
  float c1;  // softmax scale * log2(e)
  int hpw;        // query heads per workgroup: 1, 2 or 4
  int n_pblocks;  // position blocks per head group
  float* row_den;  // optional fp32 [B, Hq, Lq]: final denominator l
};

__device__ __forceinline__ int k_swz(int r) { return (r & 15) ^ (((r >> 6) & 1) << 3); }
__device__ __forceinline__ int v_swz(int d) { return d & 15; }

__device__ __forceinline__ floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 lds_read16(const uint16_t* base, int row, int piece) {
  return *reinterpret_cast<const bf16x8*>(base + row * kDim + piece * 8);
}

// Pack 8 fp32 values as bf16; `exact` values are bf16-representable (truncation is exact).
template <bool kExact>
__device__ __forceinline__ bf16x8 pack8(const float* v) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (kExact) {
      w[i] = __builtin_amdgcn_perm(__float_as_uint(v[2 * i + 1]), __float_as_uint(v[2 * i]), 0x07060302u);
    } else {
      w[i] = static_cast<uint32_t>(f32_to_bf16_bits_rne(v[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16_bits_rne(v[2 * i + 1])) << 16);
    }
  }
  bf16x8 r;
  __builtin_memcpy(&r, w, 16);
  return r;
}

template <int LV, bool kQuantP, bool kSame>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[kKeyTile * kDim];
  __shared__ __attribute__((aligned(16))) uint16_t vs[kDim * kKeyTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int n = lane & 31;
  const int half = lane >> 5;

  const int G = a.Hq / a.Hkv;
  const int hgroups = G / a.hpw;
  const int bx = blockIdx.x;
  const int hg = bx % hgroups;
  const int kvh = (bx / hgroups) % a.Hkv;
  const int b = bx / (hgroups * a.Hkv);
  const int pb = a.causal ? (a.n_pblocks - 1 - static_cast<int>(blockIdx.y)) : static_cast<int>(blockIdx.y);
  const int pos_per_wg = 32 * (4 / a.hpw);
  const int hq = kvh * G + hg * a.hpw + (w % a.hpw);
  const int p0w = pb * pos_per_wg + (w / a.hpw) * 32;
  const int off = a.Lk - a.Lq;  // bottom-right alignment: row p sees keys <= p + off

  int kend_wg = a.Lk;
  if (a.causal) kend_wg = min(a.Lk, min(pb * pos_per_wg + pos_per_wg, a.Lq) - 1 + off + 1);
  const int ntiles = kend_wg > 0 ? (kend_wg + kKeyTile - 1) / kKeyTile : 0;
  int kend_w = p0w < a.Lq ? a.Lk : 0;
  if (a.causal && p0w < a.Lq) kend_w = max(0, min(a.Lk, min(p0w + 31, a.Lq - 1) + off + 1));

  const int pos = p0w + n;
  const bool row_live = pos < a.Lq;
  bf16x8 qf[8];
  {
    const uint16_t* qp = a.q + b * a.q_sb + hq * a.q_sh + static_cast<int64_t>(row_live ? pos : 0) * a.q_sl + 8 * half;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if (row_live) {
        qf[c] = *reinterpret_cast<const bf16x8*>(qp + 16 * c);
      } else {
        qf[c] = bf16x8{};
      }
    }
  }

  floatx16 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = floatx16{};
  floatx16 accl = floatx16{};
  float m_run = -INFINITY;
  float l_run = 0.0f;
  bf16x8 ones;
  {
    const uint32_t one2 = 0x3F803F80u;
    uint32_t w4[4] = {one2, one2, one2, one2};
    __builtin_memcpy(&ones, w4, 16);
  }

  const uint16_t* kbase = a.k + b * a.k_sb + kvh * a.k_sh;
  const uint16_t* vbase = a.vt + b * a.v_sb + kvh * a.v_sh;
  // Tile loads: thread (row r = tid/16 + 16 i, piece tid%16) moves one 16-byte piece of
  // the K tile (key rows) and of the transposed V tile (dim rows) into LDS.  Offsets
  // inside a tile are 32-bit; the tile base is wave-uniform.
  const int ld_row = tid >> 4;
  const int ld_piece = tid & 15;
  const int k_off0 = ld_row * static_cast<int>(a.k_sl) + ld_piece * 8;
  const int v_off0 = ld_row * static_cast<int>(a.v_sd) + ld_piece * 8;
  const int k_step = 16 * static_cast<int>(a.k_sl);
  const int v_step = 16 * static_cast<int>(a.v_sd);
  const int st_k_lo = ld_row * kDim + ((ld_piece ^ ld_row) * 8);       // rows r < 64: piece ^ (r & 15)
  const int st_k_hi = ld_row * kDim + ((ld_piece ^ ld_row ^ 8) * 8);   // rows r >= 64: piece ^ (r & 15) ^ 8

  for (int t = 0; t < ntiles; ++t) {
    const int key0 = t * kKeyTile;
    const uint16_t* ktile = kbase + static_cast<int64_t>(key0) * a.k_sl;
    const uint16_t* vtile = vbase + key0;
    const int krows = a.Lk - key0;  // valid key rows in this tile (> 0)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = ld_row + 16 * i;
      // rows past the last key read the last valid row and are replaced by zeros
      const int koff = r < krows ? k_off0 + i * k_step : (krows - 1) * static_cast<int>(a.k_sl) + ld_piece * 8;
      uint4 kv = *reinterpret_cast<const uint4*>(ktile + koff);
      if (r >= krows) kv = make_uint4(0, 0, 0, 0);
      const uint4 vv = *reinterpret_cast<const uint4*>(vtile + v_off0 + i * v_step);
      // K rows >= 64 (i >= 4) flip bit 3 of the piece swizzle (k_swz); V uses d & 15 (v_swz)
      *reinterpret_cast<uint4*>(ks + (i < 4 ? st_k_lo : st_k_hi) + 16 * i * kDim) = kv;
      *reinterpret_cast<uint4*>(vs + st_k_lo + 16 * i * kDim) = vv;
    }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

    if (key0 < kend_w) {
      // ---- S^T = K Q^T
      floatx16 s[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        s[kb] = floatx16{};
        const int krow = 64 * ((n >> 2) & 1) + 16 * kb + 4 * (n >> 3) + (n & 3);
        const int sw = k_swz(krow);
#pragma unroll
        for (int c = 0; c < 8; ++c) s[kb] = mfma32(lds_read16(ks, krow, (2 * c + half) ^ sw), qf[c], s[kb]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // ---- masks (ragged key tail, causal diagonal)
      const bool need_mask = (key0 + kKeyTile > a.Lk) || (a.causal && key0 + kKeyTile - 1 > p0w + off);
      if (need_mask) {
        const int lim = a.causal ? min(a.Lk - 1, pos + off) : a.Lk - 1;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (key0 + 64 * half + 16 * kb + i > lim) s[kb][i] = -INFINITY;
      }
      // ---- online softmax in the log2 domain
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx * a.c1);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      m_run = m_new;
      float p[64];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) p[16 * kb + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], a.c1, -m_use));

      if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[mb][i] *= alpha;
        accl[0] *= alpha;
        l_run *= alpha;
      }

      float rowsum = 0.0f;
      if (!(kQuantP && kSame)) {
        // the normalizer sums P (unquantized mode, or no P quantization)
#pragma unroll
        for (int i = 0; i < 64; ++i) rowsum += p[i];
      }

      if (kQuantP) {
        float m3[16];
#pragma unroll
        for (int g = 0; g < 16; ++g) m3[g] = fmaxf(fmaxf(p[4 * g], p[4 * g + 1]), fmaxf(p[4 * g + 2], p[4 * g + 3]));
        float m1 = m3[0];
#pragma unroll
        for (int g = 1; g < 16; ++g) m1 = fmaxf(m1, m3[g]);
        float sc, rec;
        hif4_scale<LV>(m1, sc, rec);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          int ka, kb2;
          hif4_micro<LV>(m3[2 * c], m3[2 * c + 1], rec, ka, kb2);
          float qa, da, qb, db;
          hif4_group_mults(sc, rec, ka, qa, da);
          hif4_group_mults(sc, rec, kb2, qb, db);
#pragma unroll
          for (int j = 0; j < 8; ++j) p[8 * c + j] = hif4_element(p[8 * c + j], j < 4 ? qa : qb, j < 4 ? da : db);
        }
      }

      // ---- O^T += V^T P^T (and the P^ row sum)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const bf16x8 pb = pack8<kQuantP>(&p[8 * c]);
        // Unquantized P is not exact in bf16: it goes in as hi + lo bf16 parts
        // (16 significant bits) so PV keeps the fp32-operand accuracy of the reference.
        bf16x8 plo;
        if (!kQuantP) {
          float r[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) r[j] = p[8 * c + j] - bf16_rne(p[8 * c + j]);
          plo = pack8<false>(r);
        }
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const int d = 32 * mb + n;
          const bf16x8 va = lds_read16(vs, d, (8 * half + c) ^ v_swz(d));
          acc[mb] = mfma32(va, pb, acc[mb]);
          if (!kQuantP) acc[mb] = mfma32(va, plo, acc[mb]);
        }
        if (kQuantP && kSame) accl = mfma32(ones, pb, accl);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (!(kQuantP && kSame)) {
        rowsum += __shfl_xor(rowsum, 32, 64);
        l_run += rowsum;
      }
    }
    __syncthreads();
  }

  if (!row_live) return;
  const float l = (kQuantP && kSame) ? accl[0] : l_run;
  const float inv_guard = fmaxf(l, 1.17549435e-38f);
  if (a.row_den && half == 0) a.row_den[(static_cast<int64_t>(b) * a.Hq + hq) * a.Lq + pos] = l;
  char* obase = static_cast<char*>(a.o);
  const int64_t orow = b * a.o_sb + hq * a.o_sh + static_cast<int64_t>(pos) * a.o_sl;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * mb + 8 * j + 4 * half;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = l > 0.0f ? acc[mb][4 * j + r] / inv_guard : 0.0f;
      if (a.o_f32) {
        *reinterpret_cast<float4*>(obase + (orow + d) * 4) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        const uint32_t w0 = static_cast<uint32_t>(f32_to_bf16_bits_rne(v[0])) |
                            (static_cast<uint32_t>(f32_to_bf16_bits_rne(v[1])) << 16);
        const uint32_t w1 = static_cast<uint32_t>(f32_to_bf16_bits_rne(v[2])) |
                            (static_cast<uint32_t>(f32_to_bf16_bits_rne(v[3])) << 16);
        *reinterpret_cast<uint2*>(obase + (orow + d) * 2) = make_uint2(w0, w1);
      }
    }
  }
}

}  // namespace faq
