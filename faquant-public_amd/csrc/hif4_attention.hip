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
// Work decomposition: a work item is 256 query rows that share one KV head (GQA: hpw
// query heads x 256 / hpw positions), so each K/V tile staged in LDS serves 256 rows.  A
// 512-thread workgroup (eight waves of 32 query rows, two waves per SIMD) runs on each
// CU and streams its items one after another.  K and V^T tiles are double-buffered in
// LDS and move HBM -> LDS by buffer loads that write LDS directly (no VGPR staging); the
// DMA of tile t + 1 (or of the next item's first tile) is issued at the top of tile t,
// behind the tile's single barrier.
//
// Masks: bottom-right causal from the shapes, or per-row key ranges [row_lo, row_hi]
// plus a key-validity bitmap (2-D padding masks in the unpadded-rank form of sfa:371-427,
// sliding windows), or a dense additive fp32 mask (3-D/4-D masks, sfa:430-454); keys
// outside become -inf before the row maximum, and key tiles no row of a wave sees are
// skipped (bitwise the same as processing an all -inf tile).  An optional logit softcap
// replaces s by softcap tanh(scale s / softcap) (sfa:725-727).
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
//   the matching 16-byte run of the transposed V tile.
// LDS rows are padded to 17 16-byte units (see kRowUnits below), which makes both the
// QK and the PV operand reads conflict-free.
//
// P quantization in registers (levels 123 shown; 12 and 13 differ only in the micro
// exponent rule), bit-exact with the reference's arithmetic (hif4.py:91-271) on the
// kernel's own P.  Per lane and tile: the group maximum m1 is exp2 of the lane's largest
// scaled score (the same fma and exp2 as that element), giving the E6M2 scale s and
// rec = bf16(1/s).  Each p is multiplied once, v = RN(p 4 rec) = 4 RN(p rec); the maximum
// of v over a 4-key group is 4 RN(m3 rec), from which the micro exponent k in {0,1,2}
// (hif4.py:200-213) is read off 4K = 4 2^k = med3(floor2(4 t3), 4 2^e2, 16), where
// floor2(x) = 2^floor(log2 x) is a mask of the exponent bits (the comparisons
// m3 rec >= 2, >= 4 of the reference are exactly floor2 comparisons).  Then, with the
// reference's two roundings,
//   w = fma(v, 1/K, 0.5) = RN(RN(p qm) 4 + 0.5),   code = min(floor(w), 7),
//   y = code * K s / 4 = code * ds / 4
// (v / K is exact, so the fma rounds only the add, and floor(w) keeps the reference's
// round-half-up of ties).  P itself differs from torch.exp by a few ulp, so the output is
// compared with the simulator within a tolerance, while the codes of the kernel's P are
// compared bit for bit (the probe form below writes P and P^ per key).
#pragma once
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
  int hpw;        // query heads per workgroup: 1, 2, 4 or 8
  int n_pblocks;  // position blocks per head group
  float* row_den;  // optional fp32 [B, Hq, Lq]: final denominator l
  int out_levels;  // 0, or HiF4 levels of a QDQ of each 64-value half of an output row
  // Split-key passes (key tiles divided among blockIdx.z; 0: one pass over all tiles).
  // Row r = (b Hq + hq) Lq + pos; rows_total = B Hq Lq.
  int tiles_per_split;
  int rows_total;
  float* mx_out;          // maxima pass: c1-scaled row maximum of each key tile, [rows_total, mx_stride]
  int mx_stride;
  const float* m_start;   // partial pass: running maximum before the split, [nsplit, rows_total]
  float* part_o;          // partial pass: unnormalized O, [nsplit, rows_total, 128]
  float* part_lm;         // partial pass: (l, running maximum) after the split, [nsplit, rows_total, 2]
  // Key-range masks (kMask >= 1; otherwise the causal flag decides).  Query position p of
  // batch b sees the keys k in [row_lo[b Lq + p], row_hi[b Lq + p]] whose bit in
  // key_bits[b key_words + k / 32] is set; bounds lie in [0, Lk - 1] or describe an empty
  // range (lo > hi), and key_words covers every key tile, 4 words per tile, zero past Lk.
  const int* row_lo;
  const int* row_hi;
  const int* row_blocks;  // [B, ceil(Lq / 32), 4] per 32 positions: min lo, max hi + 1 over
                          // non-empty rows (Lk, 0 if none), max lo, min hi over rows (an
                          // empty row counts as lo = Lk, hi = -1)
  const uint32_t* key_bits;
  int64_t key_words;
  float scale;    // softmax scale (the softcap path applies it before the tanh)
  float softcap;  // > 0 (kMask 2, 4): s -> softcap tanh(scale s / softcap)
  float softcap_rec;  // fp32(1 / softcap)
  float* diag;        // PV-normalizer probe (kMode & 8): [rows_total, 5] per-row sums
  // P dump (kMode & 8 as well): fp32 [rows_total, 2, p_dump_stride]; for every key k of every
  // processed tile, P at [row][0][k] and P^ at [row][1][k] (keys of skipped tiles untouched)
  float* p_dump;
  int64_t p_dump_stride;
  // Dense additive mask (kMask 3, 4; sfa:430-454): fp32 [b, hq, pos, key] at element strides
  // (am_sb, am_sh, am_sq; 0 broadcasts), -inf = masked, Lpad columns with -inf past Lk.
  // Scores become scale s (+ softcap) + mask; the causal flag is not applied.
  const float* amask;
  int64_t am_sb, am_sh, am_sq;
  // Q operand prologue in the item setup (q_frag_prep): q then holds the raw bf16 rows, and
  // each item applies the per-block fp32 Hadamard of q_had dims (0, 64 or 128) with the
  // division by q_div, the bf16 cast and the HiF4 QDQ with q_levels (0: none)
  int q_prep, q_had, q_levels;
  SqrtDiv q_div;
  // XCD pacing of long non-causal items (attn_pace below): the launch's epoch, 0 = off
  uint32_t pace_epoch;
  int pace_lead;  // tiles a workgroup may run ahead of its XCD's average
};

// XCD pacing.  Non-causal items all stream one head's K/V tiles in order, and the workgroups of
// one XCD start consecutive position blocks of one head together, so its L2 serves each K/V
// tile to all of them while they stay within the ~64 tiles it holds.  Over items of hundreds of
// tiles they drift further apart than that and fetch the tiles again (Wan 720p: 56 GB per
// launch against 3.1 GB of K, V, Q and output).  Each workgroup adds kPaceEvery to its XCD's
// counter every kPaceEvery tiles; one that is more than kPaceLead tiles ahead of its XCD's
// average then sleeps before its next tile, at most kPaceSpins times.  The count it compares is returned by its own add
// during the previous tile, and re-read while it waits, by atomic adds (a plain or atomic load
// can return a stale copy from the CU's own cache); a workgroup that has run all its items
// adds kPaceDone, so that the XCD's last items never wait.  The counters only time the work: any value, stale or shared with another
// launch, changes no result, and every wait is bounded.  A launch uses the 8 words of its
// epoch and clears those of the next epoch (launches on one stream run in order).
constexpr int kPaceEpochs = 64;
constexpr int kPaceEvery = 4;  // tiles per count and check (each atomic's latency is waited once)
constexpr int kPaceLead = 4;  // the default lead (AttnArgs::pace_lead)
constexpr int kPaceMinTiles = 128;
constexpr int kPaceSpins = 64;
constexpr uint32_t kPaceDone = 1u << 16;
static __device__ uint32_t attn_pace[kPaceEpochs * 8];

// Whether a workgroup `step` tiles in is more than kPaceLead tiles ahead of the average of the
// nw workgroups whose tiles add up to `seen` (wrapping differences: a stale count far ahead
// reads as not ahead).
__device__ __forceinline__ bool pace_ahead(int step, uint32_t seen, int nw, int lead) {
  return static_cast<int32_t>(static_cast<uint32_t>(step * nw) - seen - static_cast<uint32_t>(lead * nw)) > 0;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;


__device__ __forceinline__ floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// One 16-byte-per-lane DMA from global memory into LDS: lane l reads 16 bytes at byte
// offset soff + voff of the buffer `rs` and writes them to bytes [16 l, 16 l + 16) of the
// 1 KiB LDS block at `dst` (wave-uniform).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff, uint16_t* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst), 16, voff, soff, 0, 0);
}

// Raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

// Wait until every memory operation this wave issued has completed (LDS DMA included):
// the workgroup barrier alone does not order another wave's DMA writes into LDS.
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }

// v_permlane32_swap of a register with itself yields {x of lane l % 32, x of lane
// 32 + l % 32} in every lane l, so these give the same value in lanes l and l ^ 32.
__device__ __forceinline__ float halves_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float halves_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Minimum / maximum over the 64 lanes, returned as wave-uniform scalars (once per kernel).
__device__ __forceinline__ int wave_min_i32(int x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x = min(x, __shfl_xor(x, m, 64));
  return __builtin_amdgcn_readfirstlane(x);
}
__device__ __forceinline__ int wave_max_i32(int x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x = max(x, __shfl_xor(x, m, 64));
  return __builtin_amdgcn_readfirstlane(x);
}

// tanh for the logit softcap, branch-free: |u| < 0.625 takes u + u^3 q(u^2) with a degree-4
// polynomial fitted (weighted least squares on Chebyshev nodes) to (tanh(x)/x - 1)/x^2;
// larger |u| takes 1 - 2 / (exp(2|u|) + 1).  Error <= 3 ulp against a float64 tanh over
// the whole float range (tests/tanh_check.c restates it on the host); exp2 overflow
// gives 1 and NaN stays NaN.
__device__ __forceinline__ float softcap_tanh(float u) {
  const float x = fabsf(u);
  const float t = x * x;
  float p = __builtin_fmaf(t, -0.005705005954951048f, 0.020639128983020782f);
  p = __builtin_fmaf(t, p, -0.05373973771929741f);
  p = __builtin_fmaf(t, p, 0.13331443071365356f);
  p = __builtin_fmaf(t, p, -0.3333328068256378f);
  const float small = __builtin_fmaf(x * t, p, x);
  const float r = __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(x * 2.8853900817779268f) + 1.0f);
  const float big = 1.0f - (r + r);
  return __builtin_copysignf(x < 0.625f ? small : big, u);
}

// Bits [lo, hi] (inclusive, clipped to [0, 31]) of a 32-bit word; 0 when lo > hi.
__device__ __forceinline__ uint32_t bit_range32(int lo, int hi) {
  const int a = min(max(lo, 0), 32);
  const int e = min(max(hi + 1, 0), 32);  // one past the last bit
  const uint32_t below_e = e >= 32 ? ~0u : ((1u << e) - 1u);
  const uint32_t below_a = a >= 32 ? ~0u : ((1u << a) - 1u);
  return below_e & ~below_a;
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

// ---- Q operand prologue in the item setup (AttnArgs::q_prep)
// operand_prep_kernel's steps for Q (qwen3.py:97-130 without key offset or Smooth-QK:
// per-block fp32 Hadamard, division by fp32(sqrt(n)), one bf16 cast, HiF4 QDQ;
// rotation.py:14-29, hif4.py:377-390) on a wave's Q fragment, whose lane (n, half) holds
// dims 16 c + 8 half + j (c, j < 8) of row n: the butterflies of stride 1, 2, 4 inside a
// chunk, 8 between lanes n and n + 32, 16, 32, 64 between chunks c and c ^ 1, 2, 4, in that
// order and each rounded once, as the prologue kernel runs them, so the fragment equals
// its output bit for bit.  Each Q row feeds one work item: the prologue's separate pass
// over Q (a read and a write) goes away.

// lane l's copy of u at lane l ^ 32
__device__ __forceinline__ int lane_swap32(int u) {
  const auto r = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(u), static_cast<uint32_t>(u), false, false);
  return (threadIdx.x & 32) ? static_cast<int>(r[0]) : static_cast<int>(r[1]);
}

// The stride-8 butterfly (left + right at lane n, left - right at lane n + 32) of two values
// x and y at once: one v_permlane32_swap brings lane n + 32's x next to lane n's and lane n's
// y next to lane n + 32's, the sum and difference are formed in place, and a second swap
// puts each result in its lane.
__device__ __forceinline__ void butterfly32_pair(float& x, float& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  const float xs = __uint_as_float(r[0]), ys = __uint_as_float(r[1]);
  const float sum = xs + ys, dif = xs - ys;
  const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(sum), __float_as_uint(dif), false, false);
  x = __uint_as_float(r2[0]);
  y = __uint_as_float(r2[1]);
}

// HiF4 QDQ of the fragment: 64-value group g (dims 64 g ..) is chunks 4 g .. 4 g + 3 of lanes
// n and n + 32; the steps of qdq8 (group maximum of the 4-value maxima, E6M2 scale, micro
// exponents, elements, a NaN anywhere makes the group NaN).  The sign of qdq8's
// `w < 0 ? -y : y` is the sign bit of w + 0 (which turns -0 into +0, the one value where
// the sign bit and w < 0 differ), ORed into y (>= +0); the NaN select runs only when some
// lane of the wave holds a NaN group.  Both replace per-value v_cndmask, bit for bit.
template <int LV>
__device__ __forceinline__ void q_frag_qdq(float (&v)[8][8]) {
  int nan_any = 0;
  int nan_g[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    float m3a[4], m3b[4];
    int nan = 0, mx = 0;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const float* w = v[4 * g + cc];
      m3a[cc] = fmaxf(fmaxf(fabsf(w[0]), fabsf(w[1])), fmaxf(fabsf(w[2]), fabsf(w[3])));
      m3b[cc] = fmaxf(fmaxf(fabsf(w[4]), fabsf(w[5])), fmaxf(fabsf(w[6]), fabsf(w[7])));
#pragma unroll
      for (int j = 0; j < 8; ++j) nan |= w[j] != w[j];
      mx = max(mx, __float_as_int(fmaxf(m3a[cc], m3b[cc])));
    }
    mx = max(mx, lane_swap32(mx));
    nan |= lane_swap32(nan);
    float sc, rec;
    hif4_scale<LV>(__int_as_float(mx), sc, rec);
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      float* w = v[4 * g + cc];
      int ka, kb;
      hif4_micro<LV>(m3a[cc], m3b[cc], rec, ka, kb);
      float qa, da, qb, db;
      hif4_group_mults(sc, rec, ka, qa, da);
      hif4_group_mults(sc, rec, kb, qb, db);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float y = hif4_element(fabsf(w[j]), j < 4 ? qa : qb, j < 4 ? da : db);
        w[j] = __uint_as_float(__float_as_uint(y) | (__float_as_uint(w[j] + 0.0f) & 0x80000000u));
      }
    }
    nan_g[g] = nan;
    nan_any |= nan;
  }
  if (__builtin_amdgcn_ballot_w64(nan_any != 0) != 0) {
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (nan_g[c >> 2]) v[c][j] = __builtin_nanf("");
  }
}

template <int QLV>
__device__ __forceinline__ void q_frag_prep_lv(bf16x8 (&qf)[8], const AttnArgs& a) {
  float v[8][8];
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] = static_cast<float>(qf[c][j]);
  if (a.q_had) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      fwht_inlane_stage<1>(v[c]);
      fwht_inlane_stage<2>(v[c]);
      fwht_inlane_stage<4>(v[c]);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int j = 0; j < 8; j += 2) butterfly32_pair(v[c][j], v[c][j + 1]);
#pragma unroll
    for (int st = 1; st <= 4; st <<= 1) {
      if (st == 4 && a.q_had != 128) break;
#pragma unroll
      for (int c = 0; c < 8; ++c)
        if (!(c & st))
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float l = v[c][j], h = v[c + st][j];
            v[c][j] = l + h;
            v[c + st][j] = l - h;
          }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) div_sqrt_n(v[c], a.q_div);
  }
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) v[c][j] = bf16_round_hw(v[c][j]);
  if constexpr (QLV != 0) q_frag_qdq<QLV>(v);
#pragma unroll
  for (int c = 0; c < 8; ++c) qf[c] = pack8<true>(v[c]);
}

__device__ __forceinline__ void q_frag_prep(bf16x8 (&qf)[8], const AttnArgs& a) {
  if (a.q_levels == 123) q_frag_prep_lv<123>(qf, a);
  else if (a.q_levels == 12) q_frag_prep_lv<12>(qf, a);
  else if (a.q_levels == 13) q_frag_prep_lv<13>(qf, a);
  else q_frag_prep_lv<0>(qf, a);
}

// Exponent argument of P = exp2(s c1 - m), m = the running maximum of RN(s c1) (log2 units).
// kExact: RN(RN(s c1) - m), the reference's order (scores scaled, then the maximum
// subtracted: sfa:727, 797), which gives the row-maximum key exactly 0 and P = 1.  Otherwise
// one fma, s c1 - m rounded once: the row-maximum key then gets the product's rounding
// residual r = mx c1 - RN(mx c1), |r| <= ulp(m) / 2, and P = 2^r (exactly 1 for |m| < 1,
// within 2^-24 |m| ln 2 of 1 otherwise).  The quantized_same form takes the fma: there the
// normalizer sums the same P^ as the numerator, so a single key's output is V^ whatever P
// is, and a P^ code changes only if that key lies on a rounding boundary; the second
// instruction per score would cost about 5% of the kernel.
template <bool kExact>
__device__ __forceinline__ float p_arg(float s, float c1, float nm) {
  return kExact ? (s * c1) + nm : __builtin_fmaf(s, c1, nm);
}

__device__ __forceinline__ float floor2(float x) { return __uint_as_float(__float_as_uint(x) & 0xFF800000u); }

// max of two non-negative floats as an integer max of their bit patterns
__device__ __forceinline__ float fmax_nonneg(float a, float b) {
  return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

// Per-lane constants of the HiF4 QDQ of one 64-key P group (p >= 0) with maximum m1.
struct PQuant {
  float rec4;  // 4 rec
  float s16;   // s / 16
};

// Same values as hif4_scale (hif4.py:91-115) for m1 >= 0: s0 = bf16(m1 bf16(1/div)),
// clamped to [2^-48, 49152] (integer clamp of the non-negative bit pattern), E6M2
// round-half-even on the bits, and rec = bf16(1/s): 1/s = 2^-e / (1 + m/4) lies far from
// every bf16 rounding boundary, so the 1-ulp hardware reciprocal rounds to the same bf16.
template <int LV>
__device__ __forceinline__ PQuant pquant_setup(float m1) {
  const float s0 = bf16_round_hw(m1 * divisor_reciprocal<LV>());
  uint32_t b = min(max(__float_as_uint(s0), 0x27800000u), 0x47400000u);
  b = (b + 0x000FFFFFu + ((b >> 21) & 1u)) & 0xFFE00000u;
  const float sc = __uint_as_float(b);
  const float rec = bf16_round_hw(__builtin_amdgcn_rcpf(sc));
  PQuant q;
  q.rec4 = rec * 4.0f;
  q.s16 = sc * 0.0625f;
  return q;
}

// 4K for the micro exponent k of one 4-key group (K = 2^k), from x = floor2 of its
// v-maximum 4 t3 and e = 4 2^e2 of its 8-key group (levels 123).  Both are 0 or powers of
// two; med3 clamps floor2(4 t3) into [4 2^e2, 16], which is the reference's lv2 + lv3 rule
// (hif4.py:200-213): t3 < 2 gives K = 2^e2, t3 in [2, 4) gives K = 2, t3 >= 4 gives K = 4.
__device__ __forceinline__ float k4_of(float x, float e) { return __builtin_amdgcn_fmed3f(x, e, 16.0f); }

// 1/K of 4K (both exact powers of two): an integer subtraction of the exponent fields,
// 2^-k = (127 - k) << 23 = (256 << 23) - ((129 + k) << 23).
__device__ __forceinline__ float inv_k_of(float k4) { return __uint_as_float(0x80000000u - __float_as_uint(k4)); }

// HiF4 QDQ in place of one 8-key group g[0..7] (two 4-key groups) of a lane's P group,
// with the reference's roundings (hif4.py:255-271):
//   v = RN(p 4 rec), exactly 4 RN(p rec) (the exact scaling by 4 commutes with rounding);
//   4 t3 = max of v over the 4-key group (rounding is monotonic, so this is 4 RN(m3 rec),
//     the product the reference compares for the micro exponents);
//   u = v / K = RN(p qm 4) with qm = rec / K (K a power of two: exact);
//   w = RN(u + 0.5): one fma of v, 1/K and 0.5 (v / K is exact, so only the add rounds);
//   code = min(floor(w), 7), value = code K s / 4.
// floor(RN(u + 0.5)) rounds ties up and gives 1 at u = 0.5 - 2^-25, as the reference's
// floor(t + 0.5) does.
template <int LV>
__device__ __forceinline__ void pquant8(float* g, const PQuant& q) {
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] = g[j] * q.rec4;
  const float ma = fmaxf(fmaxf(g[0], g[1]), fmaxf(g[2], g[3]));
  const float mb = fmaxf(fmaxf(g[4], g[5]), fmaxf(g[6], g[7]));
  const float xa = floor2(ma);
  const float xb = floor2(mb);
  float k4a, k4b;
  if (LV == 123) {
    // e2 = [max(t3a, t3b) >= 4] <=> max(xa, xb) >= 16; 4 2^e2 = med3(max(xa, xb) / 2, 4, 8),
    // the halving an exponent decrement (0 becomes -inf, which med3 clamps)
    const float hm = __uint_as_float(max(__float_as_uint(xa), __float_as_uint(xb)) - 0x00800000u);
    const float e2 = __builtin_amdgcn_fmed3f(hm, 4.0f, 8.0f);
    k4a = k4_of(xa, e2);
    k4b = k4_of(xb, e2);
  } else if (LV == 12) {
    // e2 = [max(t3a, t3b) >= 2] <=> max(xa, xb) >= 8, e3 = 0
    k4a = __builtin_amdgcn_fmed3f(fmax_nonneg(xa, xb), 4.0f, 8.0f);
    k4b = k4a;
  } else {
    // e2 = 0, e3 = [t3 >= 2] <=> x >= 8
    k4a = __builtin_amdgcn_fmed3f(xa, 4.0f, 8.0f);
    k4b = __builtin_amdgcn_fmed3f(xb, 4.0f, 8.0f);
  }
  const float ika = inv_k_of(k4a), ikb = inv_k_of(k4b);
  const float dqa = k4a * q.s16, dqb = k4b * q.s16;  // K s / 4
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    g[j] = fminf(floorf(__builtin_fmaf(g[j], ika, 0.5f)), 7.0f) * dqa;
    g[4 + j] = fminf(floorf(__builtin_fmaf(g[4 + j], ikb, 0.5f)), 7.0f) * dqb;
  }
}

// The in-register P quantizer of the attention kernel on given values: one lane per
// 64-value group of non-negative fp32 p, group maximum m1 = max(p) (in the kernel it is
// exp2 of the largest scaled score, the same value), then pquant_setup and pquant8 on the
// eight 8-value groups.  A verification entry point for the kernel's codes.
template <int LV>
__global__ __launch_bounds__(256) void pquant_groups_kernel(const float* p, float* p_hat, int64_t groups) {
  const int64_t gi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const float* src = p + gi * 64;
  float v[64];
#pragma unroll
  for (int i = 0; i < 16; ++i) *reinterpret_cast<float4*>(&v[4 * i]) = *reinterpret_cast<const float4*>(src + 4 * i);
  float m1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; ++i) m1 = fmaxf(m1, v[i]);
  const PQuant pq = pquant_setup<LV>(m1);
#pragma unroll
  for (int c = 0; c < 8; ++c) pquant8<LV>(&v[8 * c], pq);
  float* dst = p_hat + gi * 64;
#pragma unroll
  for (int i = 0; i < 16; ++i) *reinterpret_cast<float4*>(dst + 4 * i) = *reinterpret_cast<const float4*>(&v[4 * i]);
}

// Value of x in lane l ^ 32 (v_permlane32_swap of a register with itself gives the
// lower-half lane's copy in result 0 and the upper-half lane's in result 1).
__device__ __forceinline__ float partner32(float x, int half) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(half ? r[0] : r[1]);
}

// HiF4 QDQ (levels LV) of one output row held by lanes n and n + 32: val[mb][j][r] is dim
// 32 mb + 8 j + 4 half + r, so each 4-value micro group is lane-local, an 8-value group
// pairs this lane's 4 values with the partner's, and each 64-value group is mb in
// {2g, 2g + 1} of both lanes.  Same arithmetic as the row quantizer (hif4.py:143-271):
// group maximum of |x|, E6M2 scale, micro exponents, codes; a NaN anywhere in a 64-value
// group makes the whole group NaN.
template <int LV>
__device__ __forceinline__ void qdq_out_row(float (&val)[4][4][4], int half) {
  float m3[4][4], pm3[4][4];
  uint32_t nan = 0;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float m = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        m = fmaxf(m, fabsf(val[mb][j][r]));
        if (val[mb][j][r] != val[mb][j][r]) nan |= 1u << (mb >> 1);
      }
      m3[mb][j] = m;
    }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int j = 0; j < 4; ++j) pm3[mb][j] = partner32(m3[mb][j], half);
  nan |= __float_as_uint(partner32(__uint_as_float(nan), half));
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    float m1 = 0.0f;
#pragma unroll
    for (int mb = 2 * g; mb < 2 * g + 2; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) m1 = fmaxf(m1, fmaxf(m3[mb][j], pm3[mb][j]));
    float s, rec;
    hif4_scale<LV>(m1, s, rec);
#pragma unroll
    for (int mb = 2 * g; mb < 2 * g + 2; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // the 8-value group's first 4-group lives in the lower-half lane
        const float m3a = half ? pm3[mb][j] : m3[mb][j];
        const float m3b = half ? m3[mb][j] : pm3[mb][j];
        int ka, kb;
        hif4_micro<LV>(m3a, m3b, rec, ka, kb);
        float qm4, dq;
        hif4_group_mults(s, rec, half ? kb : ka, qm4, dq);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = val[mb][j][r];
          const float y = hif4_element(fabsf(x), qm4, dq);
          val[mb][j][r] = ((nan >> g) & 1u) ? __builtin_nanf("") : (x < 0.0f ? -y : y);
        }
      }
  }
}

// ---------------------------------------------------------------------------------------
// Attention forward: one 512-thread workgroup per CU (eight waves of 32 query rows, two
// waves per SIMD), K and V^T tiles double-buffered in LDS so the DMA of tile t + 1 is issued
// a whole tile ahead, and one barrier per tile.  gfx950 services a ds_read_b128 in four
// passes of 16 lanes (lane bit 5, parity of lane bits 2..4); a pass is conflict-free when
// its 16 lanes hit 16 distinct 16-byte bank groups.  LDS rows are padded to 17 16-byte units (272 B): unit u of a tile
// holds piece u % 17 of row u / 17 (piece 16 is padding), so every operand read is a base
// register plus a constant offset, and under the ds_read_b128 pass structure (lane bit 5,
// parity of lane bits 2..4) the QK reads (rows pi(kb, n), one piece) and the PV reads
// (rows n, one piece) of a pass hit 16 distinct bank groups: (17 r + p) mod 16 = (r + p)
// mod 16 with 16 distinct r mod 16 per pass.
constexpr int kRowUnits = 17;
constexpr int kTileBytes = kKeyTile * kRowUnits * 16;  // 34816
constexpr int kStageBytes = 2 * kTileBytes;             // K tile, then V^T tile
constexpr int kOutPitch = 136;  // bf16 elements per staged output row (272 B): 8 waves x 32 rows fit one stage
static_assert(8 * 32 * kOutPitch * 2 <= kStageBytes, "staged output rows must fit one LDS stage");

__device__ __forceinline__ bf16x8 lds_read_at(const uint8_t* base, int byte_off) {
  return *reinterpret_cast<const bf16x8*>(base + byte_off);
}

// kMode & 7 (kMask) 0: masks from the shapes (none, bottom-right causal, ragged tail);
// 1: key ranges and valid-key bits (a.row_lo, a.row_hi, a.row_blocks, a.key_bits); 2: key
// ranges and the logit softcap; 3: a dense additive mask (a.amask); 4: the dense mask and
// the softcap.  kMode & 8 (kDiag): the PV-normalizer probe (a.diag).  One form per
// instantiation keeps each hot loop within its register budget.
//
// Work items: item i = y X + x with x = (b, kvh, hg) and y the position block (causal:
// the longest blocks first; non-causal with P % 8 == 0: i = x n_pblocks + y, one head per
// XCD and round); X = B Hkv (Hq / Hkv / hpw), n_items = X n_pblocks.  Workgroup
// wid of P = gridDim.x takes items wid, wid + P, wid + 2P, ... (every second round in
// reverse inside each XCD's share, so large and small items pair up), and runs them as
// one stream of key tiles: the DMA of the next item's first tile is issued during the
// current item's last tile, and no workgroup is relaunched between items.  P = n_items
// gives one item per workgroup.
template <int LV, bool kQuantP, bool kSame, int kMode>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fwd_kernel(AttnArgs a) {
  constexpr int kMask = kMode & 7;
  constexpr bool kDiag = kQuantP && (kMode & 8) != 0;
  constexpr bool kDense = kMask == 3 || kMask == 4;
  constexpr bool kSoftcap = kMask == 2 || kMask == 4;
  constexpr bool kRanges = kMask == 1 || kMask == 2;
  constexpr bool kExactArg = !(kQuantP && kSame);  // see p_arg
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int n = lane & 31;
  const int half = lane >> 5;

  const int G = a.Hq / a.Hkv;
  const int hgroups = G / a.hpw;
  const int X = a.B * a.Hkv * hgroups;
  const int n_items = X * a.n_pblocks;
  const int pos_per_wg = 32 * (8 / a.hpw);
  const int off = a.Lk - a.Lq;  // bottom-right alignment: row p sees keys <= p + off
  const int split = static_cast<int>(blockIdx.z);
  const int P = static_cast<int>(gridDim.x);
  const int wid = static_cast<int>(blockIdx.x);
  const int nblk = (a.Lq + 31) / 32;
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  typedef const __attribute__((address_space(4))) i32x4 const_i4;

  // Non-causal items all span the same keys, so no pairing of long and short items is
  // needed: items are numbered head-major (i = x n_pblocks + y) and the P / 8 workgroups of
  // one XCD (wid % 8) take P / 8 consecutive position blocks of one head per round, so
  // each XCD's L2 serves the K/V tiles of one head (two where a head's blocks end inside
  // the chunk) to all of its CUs, which stream them in step.
  const bool head_major = !a.causal && P % 8 == 0;
  // item of round k for this workgroup (n_items or more: none)
  auto item_of = [&](int k) -> int {
    if (head_major) return k * P + (wid % 8) * (P / 8) + wid / 8;
    const int r = (k & 1) ? ((P % 8 == 0) ? (wid % 8) + 8 * (P / 8 - 1 - wid / 8) : P - 1 - wid) : wid;
    return k * P + r;
  };
  // workgroup-uniform geometry of an item: coordinates and its key-tile range
  struct Geo {
    int b, kvh, hg, pb, t_lo, t_hi;
  };
  auto geo_of = [&](int i) -> Geo {
    Geo g;
    const int x = head_major ? i / a.n_pblocks : i % X, y = head_major ? i % a.n_pblocks : i / X;
    g.hg = x % hgroups;
    g.kvh = (x / hgroups) % a.Hkv;
    g.b = x / (hgroups * a.Hkv);
    g.pb = a.causal ? (a.n_pblocks - 1 - y) : y;
    int kbeg_wg = 0, kend_wg = a.Lk;
    if (kRanges) {
      // the rows' key ranges, summarized per 32 positions (scalar loads of a.row_blocks)
      const_i4* blk = (const_i4*)(a.row_blocks) + static_cast<int64_t>(g.b) * nblk;
      const int b0 = g.pb * (pos_per_wg / 32);
      kbeg_wg = a.Lk;
      kend_wg = 0;
      for (int j = 0; j < pos_per_wg / 32; ++j) {
        if (b0 + j < nblk) {
          const i32x4 v = blk[b0 + j];
          kbeg_wg = min(kbeg_wg, v.x);
          kend_wg = max(kend_wg, v.y);
        }
      }
    } else if (a.causal) {
      kend_wg = min(a.Lk, min(g.pb * pos_per_wg + pos_per_wg, a.Lq) - 1 + off + 1);
    }
    const int ntiles = kend_wg > 0 ? (kend_wg + kKeyTile - 1) / kKeyTile : 0;
    const int t_first = kbeg_wg < kend_wg ? kbeg_wg / kKeyTile : ntiles;
    g.t_lo = a.tiles_per_split ? max(t_first, min(ntiles, split * a.tiles_per_split)) : t_first;
    g.t_hi = a.tiles_per_split ? min(ntiles, split * a.tiles_per_split + a.tiles_per_split) : ntiles;
    return g;
  };

  bf16x2_t ones2;
  {
    const uint32_t one2 = 0x3F803F80u;
    __builtin_memcpy(&ones2, &one2, 4);
  }

  // DMA assignment: instruction j (0..3) of wave w fills tile units 512 j + 64 w + lane;
  // waves 0 and 1 also fill units 2048 + 64 w + lane (j = 4).  Unit u is piece u % 17 of
  // row u / 17; the padding piece re-reads piece 15 of its row.
  const int ws = __builtin_amdgcn_readfirstlane(w);
  const int nj = ws < 2 ? 5 : 4;
  uint32_t kvo[5], vvo[5];
  int krow[5];
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const int u = (j < 4 ? 512 * j : 2048) + 64 * ws + lane;
    const int r = u / kRowUnits;
    const int p = min(u - r * kRowUnits, 15);
    krow[j] = r;
    kvo[j] = static_cast<uint32_t>(r * static_cast<int>(a.k_sl) + 8 * p) * 2u;
    vvo[j] = static_cast<uint32_t>(r * static_cast<int>(a.v_sd) + 8 * p) * 2u;
  }
  const uint32_t k_bytes = a.Lk > 0 ? static_cast<uint32_t>(((a.Lk - 1) * a.k_sl + kDim) * 2) : 0u;
  const uint32_t v_bytes = static_cast<uint32_t>((127 * a.v_sd + a.v_sd) * 2);

  // DMA of key tile t of the item at (b, kvh) into LDS stage `stage`
  auto load_tile = [&](int gb, int gkvh, int t, int stage) {
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(a.k + gb * a.k_sb + gkvh * a.k_sh, k_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(a.vt + gb * a.v_sb + gkvh * a.v_sh, v_bytes);
    uint8_t* const st = lds + stage * kStageBytes;
    const int key0 = t * kKeyTile;
    const uint32_t ksoff = static_cast<uint32_t>(key0 * a.k_sl) * 2u;
    const uint32_t vsoff = static_cast<uint32_t>(key0) * 2u;
    if (key0 + kKeyTile <= a.Lk) {
#pragma unroll
      for (int j = 0; j < 5; ++j)
        if (j < nj) dma16(krs, kvo[j], ksoff, reinterpret_cast<uint16_t*>(st + ((j < 4 ? 512 * j : 2048) + 64 * ws) * 16));
    } else {
      // ragged last tile: rows past the last key re-read the last key (their scores are
      // masked to -inf before use)
#pragma unroll
      for (int j = 0; j < 5; ++j) {
        if (j < nj) {
          const int rr = min(krow[j], a.Lk - 1 - key0);
          const uint32_t vo = kvo[j] - static_cast<uint32_t>((krow[j] - rr) * static_cast<int>(a.k_sl)) * 2u;
          dma16(krs, vo, ksoff, reinterpret_cast<uint16_t*>(st + ((j < 4 ? 512 * j : 2048) + 64 * ws) * 16));
        }
      }
    }
    // the maxima pass reads K only
    if (!a.mx_out) {
#pragma unroll
      for (int j = 0; j < 5; ++j)
        if (j < nj) dma16(vrs, vvo[j], vsoff, reinterpret_cast<uint16_t*>(st + kTileBytes + ((j < 4 ? 512 * j : 2048) + 64 * ws) * 16));
    }
  };

  // LDS operand offsets (bytes).  QK: key row pi(0, n) + 16 kb, piece 2c + half.
  const int krow0 = 64 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  const int kbyte = krow0 * (kRowUnits * 16) + half * 16;
  // PV: V^T row 32 mb + n, piece 8 half + c.
  const int vbyte = kTileBytes + n * (kRowUnits * 16) + half * 128;

  int k_round = 0;
  int item = item_of(0);
  if (item >= n_items) return;
  Geo g = geo_of(item);
  int step = 0;  // key tiles processed by this workgroup: LDS stage parity
  // XCD pacing (attn_pace): plain non-causal launches whose items are long
  const int pace_nw = P / 8;
  const bool pace = kMask == 0 && head_major && a.pace_epoch != 0 && g.t_hi - g.t_lo >= kPaceMinTiles;
  uint32_t* const pace_ctr = attn_pace + (a.pace_epoch % kPaceEpochs) * 8 + (wid & 7);
  if (pace && wid == 0 && tid < 8) attn_pace[((a.pace_epoch + 1) % kPaceEpochs) * 8 + tid] = 0u;
  uint32_t pace_seen = 0;  // lane 0 of wave 0: this XCD's tile count, loaded one tile ago

  bool issued = false;  // the DMA of the current item's first tile is in flight

  for (;;) {
    // first tile of the item, unless the previous item's last tile already fetched it (its
    // stage was last read two steps ago, before the last barrier)
    if (!issued && g.t_lo < g.t_hi) load_tile(g.b, g.kvh, g.t_lo, step & 1);
    issued = false;
    // ---- per-item state: rows, bounds, Q fragment, recurrence state
    const int b = g.b;
    const int hq = g.kvh * G + g.hg * a.hpw + (w % a.hpw);
    const int p0w = g.pb * pos_per_wg + (w / a.hpw) * 32;
    const int pos = p0w + n;
    const bool row_live = pos < a.Lq;
    const int64_t row = (static_cast<int64_t>(b) * a.Hq + hq) * a.Lq + pos;

    // keys [kbeg_w, kend_w) seen by some row of this wave; a tile needs no per-key mask when
    // every row of the wave sees all of it (lo_max <= key0 and key0 + 127 <= hi_min)
    int kbeg_w = 0;
    int kend_w = p0w < a.Lq ? a.Lk : 0;
    int lo_max = 0, hi_min = a.Lk - 1;
    int rlo = a.Lk, rhi = -1;  // this row's key range
    if (kRanges) {
      kend_w = 0;
      kbeg_w = a.Lk;
      if (p0w < a.Lq) {
        const i32x4 v = ((const_i4*)(a.row_blocks))[static_cast<int64_t>(b) * nblk + p0w / 32];
        kbeg_w = v.x;
        kend_w = v.y;
        lo_max = v.z;
        hi_min = v.w;
      }
      if (row_live) {
        rlo = a.row_lo[static_cast<int64_t>(b) * a.Lq + pos];
        rhi = a.row_hi[static_cast<int64_t>(b) * a.Lq + pos];
      }
    } else if (a.causal && p0w < a.Lq) {
      kend_w = max(0, min(a.Lk, min(p0w + 31, a.Lq - 1) + off + 1));
    }

    // Q fragment of this wave's rows: lane (n, half) holds Q[row n][16 c + 8 half .. + 7].
    // (Fetching the next item's fragment during the last tile was tried: the conditional
    // overwrite of a loop-carried register array costs register copies in every tile.)
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
      // the raw rows: Q's operand prologue here (q_frag_prep)
      if (a.q_prep) q_frag_prep(qf, a);
    }

    floatx16 acc[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[mb] = floatx16{};
    // a partial pass continues the reference's recurrence from the running maximum of the
    // tiles before its split (sfa:788-806: P of tile t depends on the maximum after tile t)
    float m_run = (a.m_start && row_live) ? a.m_start[static_cast<int64_t>(split) * a.rows_total + row] : -INFINITY;
    float l_run = 0.0f;
    // probe (kDiag): sum P^ and sum P, rescaled like l, and per-element sums over this
    // lane's keys: #(P^ = 0 < P), sum (P^ - P)^2, sum P^2 (sfa:36-185, 835-869).  They are
    // taken on the P of the exact exponent argument (p_arg<true>) in both normalizer modes,
    // so the summary does not depend on the mode, as the reference's P does not; the output
    // path keeps the mode's own form, so the outputs equal the plain kernel's.
    float dq_run = 0.0f, dp_run = 0.0f, dg_zero = 0.0f, dg_err = 0.0f, dg_ref = 0.0f;

    // next item of this workgroup (its first tile is fetched during this item's last one)
    const int next_item = item_of(k_round + 1);
    Geo ng{};
    if (next_item < n_items) ng = geo_of(next_item);

    for (int t = g.t_lo; t < g.t_hi; ++t, ++step) {
      // tile t has landed for every wave; every wave is done with the previous step, whose
      // stage the DMA of the next step overwrites
      wait_all_memory();
      if (pace && w == 0 && (step & (kPaceEvery - 1)) == 1) {
        uint32_t seen = __builtin_amdgcn_readfirstlane(pace_seen);
        for (int spin = 0; spin < kPaceSpins && pace_ahead(step, seen, pace_nw, a.pace_lead); ++spin) {
          __builtin_amdgcn_s_sleep(2);
          uint32_t v = 0;
          if (lane == 0) v = __hip_atomic_fetch_add(pace_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          seen = __builtin_amdgcn_readfirstlane(v);
        }
      }
      __syncthreads();
      // The two waves of a SIMD leave the barrier together, and with equal priorities the
      // older one wins every issue conflict: it finishes its P chunks far ahead and then waits
      // at the next barrier while the younger one runs alone at the single-wave issue rate.
      // Priorities that fall as a wave advances through the tile (3 for QK, the maximum and
      // chunks 0-1, down to 0 for chunks 6-7) let the wave that is behind win instead, so the
      // two converge and reach the barrier together.
      __builtin_amdgcn_s_setprio(3);
      if (t + 1 < g.t_hi) {
        load_tile(b, g.kvh, t + 1, (step + 1) & 1);
      } else if (next_item < n_items && ng.t_lo < ng.t_hi) {
        load_tile(ng.b, ng.kvh, ng.t_lo, (step + 1) & 1);
        issued = true;
      }
      if (pace && tid == 0 && (step & (kPaceEvery - 1)) == 0)
        pace_seen = __hip_atomic_fetch_add(pace_ctr, kPaceEvery, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + kPaceEvery;
      do {
        const uint8_t* const st = lds + (step & 1) * kStageBytes;
        const uint8_t* const kp = st + kbyte;
        const uint8_t* const vp = st + vbyte;

        const int key0 = t * kKeyTile;
        if (key0 >= kend_w || key0 + kKeyTile <= kbeg_w) continue;
        floatx16 s[4];
        {
          // ---- S^T = K Q^T, c-major (four independent accumulation chains); the K fragments
          // of step c + 1 are read while the MFMAs of step c run
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) s[kb] = floatx16{};
          bf16x8 kf[2][4];
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) kf[0][kb] = lds_read_at(kp, kb * 16 * kRowUnits * 16);
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            if (c + 1 < 8) {
#pragma unroll
              for (int kb = 0; kb < 4; ++kb) kf[(c + 1) & 1][kb] = lds_read_at(kp, kb * 16 * kRowUnits * 16 + (c + 1) * 32);
            }
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) s[kb] = mfma32(kf[c & 1][kb], qf[c], s[kb]);
          }
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
          for (int c = 0; c < 7; ++c) {
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
        }
        __builtin_amdgcn_sched_barrier(0);

        if (kSoftcap) {
          // sfa:725-727: scores * scale, then softcap * tanh(scores / softcap)
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              // scale, then the quotient by softcap: q = t rc corrected by one fma step
              const float t = s[kb][i] * a.scale;
              const float q0 = t * a.softcap_rec;
              const float q = __builtin_fmaf(__builtin_fmaf(-q0, a.softcap, t), a.softcap_rec, q0);
              s[kb][i] = softcap_tanh(q) * a.softcap;
            }
        }
        if (kDense) {
          // sfa:430-454: scores (scaled, and softcapped above for kMask 4) plus the mask row
          // (its columns past Lk hold -inf, which also masks the ragged tail)
          const float* mr = a.amask + b * a.am_sb + hq * a.am_sh + (row_live ? pos : 0) * a.am_sq + key0 + 64 * half;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            float mv[16];
#pragma unroll
            for (int u = 0; u < 4; ++u) *reinterpret_cast<float4*>(&mv[4 * u]) = *reinterpret_cast<const float4*>(mr + 16 * kb + 4 * u);
#pragma unroll
            for (int i = 0; i < 16; ++i) s[kb][i] = (kSoftcap ? s[kb][i] : s[kb][i] * a.scale) + mv[i];
          }
        }
        // ---- masks (ragged key tail, causal diagonal, key ranges and invalid keys)
        if (kRanges) {
          // the tile's four valid-key words, loaded as scalars (wave-uniform address): no wait
          // on the vector-memory counter, which the in-flight DMA of the next tile also holds
          // (the constant address space: this kernel never writes key_bits)
          typedef const __attribute__((address_space(4))) uint32_t const_u32;
          const_u32* kw = (const_u32*)(a.key_bits + b * a.key_words + (key0 >> 5));
          const uint32_t kw0 = kw[0], kw1 = kw[1], kw2 = kw[2], kw3 = kw[3];
          if (!(lo_max <= key0 && key0 + kKeyTile - 1 <= hi_min) || (kw0 & kw1 & kw2 & kw3) != ~0u) {
            const bool hi_half = half != 0;
            const int base = key0 + (hi_half ? 64 : 0);
            const uint32_t m0 = bit_range32(rlo - base, rhi - base) & (hi_half ? kw2 : kw0);
            const uint32_t m1 = bit_range32(rlo - base - 32, rhi - base - 32) & (hi_half ? kw3 : kw1);
            // keep = all ones for an allowed key (sign-extended bit), else -inf: bfe + bfi
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                const int j = 16 * kb + i;
                const uint32_t keep = static_cast<uint32_t>(
                    __builtin_amdgcn_sbfe(static_cast<int>(j < 32 ? m0 : m1), static_cast<uint32_t>(j & 31), 1u));
                s[kb][i] = __uint_as_float((__float_as_uint(s[kb][i]) & keep) | (0xFF800000u & ~keep));
              }
          }
        } else if (kMask == 0 && ((key0 + kKeyTile > a.Lk) || (a.causal && key0 + kKeyTile - 1 > p0w + off))) {
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
        const float mx_row = halves_max(mx);
        if (a.mx_out) {
          // maxima pass: the tile's c1-scaled row maximum only
          if (row_live && half == 0) a.mx_out[row * a.mx_stride + t] = mx_row * a.c1;
          continue;
        }
        const float m_new = fmaxf(m_run, mx_row * a.c1);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float nm = -m_use;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        m_run = m_new;
        if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
          for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mb][i] *= alpha;
          l_run *= alpha;
          if (kDiag) {
            dq_run *= alpha;
            dp_run *= alpha;
          }
        }
        // ---- P, its HiF4 QDQ and the row sum, one 8-key chunk at a time; chunk c of this lane
        // is keys 64 half + 8c .. 8c+7, the B operand of PV k-chunk c.
        PQuant pq;
        if (kQuantP) {
          // group maximum = P of the lane's largest score (same fma and exp2)
          pq = pquant_setup<LV>(__builtin_amdgcn_exp2f(p_arg<kExactArg>(mx, a.c1, nm)));
        }
        // the probe's quantizer on the exact-argument P (the same as pq when the output path
        // takes that argument)
        PQuant pqx{};
        if (kDiag) pqx = kExactArg ? pq : pquant_setup<LV>(__builtin_amdgcn_exp2f(p_arg<true>(mx, a.c1, nm)));
        float rowsum = 0.0f, dq_sum = 0.0f, dp_sum = 0.0f;
        // Software pipeline over the eight 8-key chunks: iteration c computes chunk c's P^
        // (VALU) while the MFMAs of chunk c - 1 issue one at a time between those VALU
        // instructions.
        bf16x8 pprev, plprev;
#pragma unroll
        for (int c = 0; c <= 8; ++c) {
          if (c < 2) __builtin_amdgcn_s_setprio(3);
          else if (c < 4) __builtin_amdgcn_s_setprio(2);
          else if (c < 6) __builtin_amdgcn_s_setprio(1);
          else __builtin_amdgcn_s_setprio(0);
          bf16x8 va[4];
          if (c >= 1) {
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) va[mb] = lds_read_at(vp, mb * 32 * kRowUnits * 16 + (c - 1) * 16);
          }
          bf16x8 pcur, plcur;
          if (c < 8) {
            float pc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) pc[j] = __builtin_amdgcn_exp2f(p_arg<kExactArg>(s[c >> 1][8 * (c & 1) + j], a.c1, nm));
            if (!(kQuantP && kSame)) {
              // the normalizer sums P (unquantized mode, or no P quantization)
#pragma unroll
              for (int j = 0; j < 8; ++j) rowsum += pc[j];
            }
            if (kQuantP) {
              float pu[8];
              if (kDiag) {
#pragma unroll
                for (int j = 0; j < 8; ++j) pu[j] = pc[j];
              }
              pquant8<LV>(pc, pq);
              pcur = pack8<true>(pc);
              if (kSame) {
                uint32_t wv[4];
                __builtin_memcpy(wv, &pcur, 16);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  bf16x2_t pr;
                  __builtin_memcpy(&pr, &wv[i], 4);
                  rowsum = __builtin_amdgcn_fdot2_f32_bf16(pr, ones2, rowsum, false);
                }
              }
              if (kDiag) {
                // P and P^ of the exact exponent argument
                float pe[8], qe[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                  pe[j] = kExactArg ? pu[j] : __builtin_amdgcn_exp2f(p_arg<true>(s[c >> 1][8 * (c & 1) + j], a.c1, nm));
                  qe[j] = kExactArg ? pc[j] : pe[j];
                }
                if (!kExactArg) pquant8<LV>(qe, pqx);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                  const float d = qe[j] - pe[j];
                  dq_sum += qe[j];
                  dp_sum += pe[j];
                  dg_err = __builtin_fmaf(d, d, dg_err);
                  dg_ref = __builtin_fmaf(pe[j], pe[j], dg_ref);
                  dg_zero += (qe[j] == 0.0f && pe[j] > 0.0f) ? 1.0f : 0.0f;
                }
                if (a.p_dump && row_live) {
                  // this chunk's keys key0 + 64 half + 8c .. + 7 (within the padded row)
                  float* pd = a.p_dump + row * 2 * a.p_dump_stride + key0 + 64 * half + 8 * c;
#pragma unroll
                  for (int u = 0; u < 2; ++u) {
                    *reinterpret_cast<float4*>(pd + 4 * u) = make_float4(pu[4 * u], pu[4 * u + 1], pu[4 * u + 2], pu[4 * u + 3]);
                    *reinterpret_cast<float4*>(pd + a.p_dump_stride + 4 * u) =
                        make_float4(pc[4 * u], pc[4 * u + 1], pc[4 * u + 2], pc[4 * u + 3]);
                  }
                }
              }
            } else {
              // Unquantized P is not exact in bf16: it goes in as hi + lo bf16 parts
              // (16 significant bits) so PV keeps the fp32-operand accuracy of the reference.
              float r[8];
#pragma unroll
              for (int j = 0; j < 8; ++j) r[j] = pc[j] - bf16_rne(pc[j]);
              pcur = pack8<false>(pc);
              plcur = pack8<false>(r);
            }
          }
          if (c >= 1) {
            // ---- O^T += V^T P^T for chunk c - 1
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
              acc[mb] = mfma32(va[mb], pprev, acc[mb]);
              if (!kQuantP) acc[mb] = mfma32(va[mb], plprev, acc[mb]);
            }
            // issue order: the four LDS reads, ~20 VALU (read latency), then one MFMA per
            // ~12 VALU instructions
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            if (c < 8) {
              __builtin_amdgcn_sched_group_barrier(0x002, 20, 0);
#pragma unroll
              for (int i = 0; i < (kQuantP ? 4 : 8); ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, kQuantP ? 12 : 6, 0);
              }
              __builtin_amdgcn_sched_group_barrier(0x002, 200, 0);
            } else {
              __builtin_amdgcn_sched_group_barrier(0x008, kQuantP ? 4 : 8, 0);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          pprev = pcur;
          plprev = plcur;
        }
        l_run += halves_sum(rowsum);
        if (kDiag) {
          dq_run += halves_sum(dq_sum);
          dp_run += halves_sum(dp_sum);
        }
      } while (false);
    }

    // ---- epilogue of the item
    // bf16 rows go out through LDS: once every wave is done with the last tile's stage, each
    // wave stages its 32 output rows there (272-byte pitch) and stores whole 256-byte rows,
    // two per instruction.  Stored straight from the MFMA layout, a lane's 16 pieces of
    // 8 bytes land in 32 rows a position stride apart, each instruction touching 32
    // partially written cache lines.  (kernel-uniform condition: every wave takes the
    // barrier)
    const bool lds_out = !a.o_f32 && !a.mx_out && !a.part_o;
    uint16_t* const out_rows = reinterpret_cast<uint16_t*>(lds + ((step + 1) & 1) * kStageBytes) + w * (32 * kOutPitch);
    if (lds_out) __syncthreads();
    if (row_live && !a.mx_out) {
      if (a.part_o) {
        // partial pass: unnormalized O^T column of this row, its l and running maximum
        float* po = a.part_o + (static_cast<int64_t>(split) * a.rows_total + row) * kDim;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            *reinterpret_cast<float4*>(po + 32 * mb + 8 * j + 4 * half) =
                make_float4(acc[mb][4 * j], acc[mb][4 * j + 1], acc[mb][4 * j + 2], acc[mb][4 * j + 3]);
        if (half == 0) {
          float* lm = a.part_lm + (static_cast<int64_t>(split) * a.rows_total + row) * 2;
          lm[0] = l_run;
          lm[1] = m_run;
        }
      } else {
      const float l = l_run;
      if (kDiag) {
        // per row: sum P^, sum P, #(P^ = 0 < P), sum (P^ - P)^2, sum P^2
        const float zero = halves_sum(dg_zero), err = halves_sum(dg_err), ref = halves_sum(dg_ref);
        if (half == 0 && a.diag) {
          float* dg = a.diag + row * 5;
          dg[0] = dq_run;
          dg[1] = dp_run;
          dg[2] = zero;
          dg[3] = err;
          dg[4] = ref;
        }
      }
      const float inv_guard = fmaxf(l, 1.17549435e-38f);
      // acc / l as the reference divides: rl = RN(1 / l), then one correction step from
      // q0 = RN(acc rl) gives the correctly rounded quotient (Markstein's theorem)
      const float rl = 1.0f / inv_guard;
      if (a.row_den && half == 0) a.row_den[(static_cast<int64_t>(b) * a.Hq + hq) * a.Lq + pos] = l;
      // this lane's part of the output row: element 4 half, then constant offsets 32 mb + 8 j
      const int64_t orow = b * a.o_sb + hq * a.o_sh + static_cast<int64_t>(pos) * a.o_sl + 4 * half;
      char* const orow_p = static_cast<char*>(a.o) + orow * (a.o_f32 ? 4 : 2);
      // o = acc / l (0 for rows that saw no key), in the output dtype
      float val[4][4][4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float xa = acc[mb][4 * j + r];
            const float q0 = xa * rl;
            const float x = l > 0.0f ? __builtin_fmaf(__builtin_fmaf(-q0, inv_guard, xa), rl, q0) : 0.0f;
            val[mb][j][r] = a.o_f32 ? x : bf16_round_hw(x);
          }
      // the o_proj-input QDQ of the output row (qwen3.py:167-171), on the output-dtype values
      if (a.out_levels == 123) qdq_out_row<123>(val, half);
      else if (a.out_levels == 12) qdq_out_row<12>(val, half);
      else if (a.out_levels == 13) qdq_out_row<13>(val, half);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = 32 * mb + 8 * j;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = val[mb][j][r];
          if (a.o_f32) {
            *reinterpret_cast<float4*>(orow_p + d * 4) = make_float4(v[0], v[1], v[2], v[3]);
          } else {
            // the values are bf16 already (rounded above, or HiF4 values): pack the upper halves
            const uint32_t w0 = __builtin_amdgcn_perm(__float_as_uint(v[1]), __float_as_uint(v[0]), 0x07060302u);
            const uint32_t w1 = __builtin_amdgcn_perm(__float_as_uint(v[3]), __float_as_uint(v[2]), 0x07060302u);
            *reinterpret_cast<uint2*>(out_rows + n * kOutPitch + d + 4 * half) = make_uint2(w0, w1);
          }
        }
      }
      }

    }
    // bf16 rows through LDS: this wave's rows p0w .. p0w + 31, lane l takes 8 bytes (l % 32)
    // of row 2 it + l / 32, two whole rows per instruction (output rows need only 8-byte
    // alignment); each wave reads back only what it wrote, and the LDS wait orders its own
    // accesses.  All reads come before the stores: an LDS read may alias the in-flight
    // LDS-DMA of the next tile, so each one waits on the whole vector-memory counter, stores
    // included.
    const int piece = lane & 31;
    uint2 rows_v[16];
    if (lds_out) {
#pragma unroll
      for (int it = 0; it < 16; ++it)
        rows_v[it] = *reinterpret_cast<const uint2*>(out_rows + (2 * it + (lane >> 5)) * kOutPitch + 4 * piece);
    }
    if (lds_out) {
      uint16_t* const o16 = static_cast<uint16_t*>(a.o) + b * a.o_sb + hq * a.o_sh;
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        const int p = p0w + 2 * it + (lane >> 5);
        if (p < a.Lq) *reinterpret_cast<uint2*>(o16 + static_cast<int64_t>(p) * a.o_sl + 4 * piece) = rows_v[it];
      }
    }
    ++k_round;
    item = next_item;
    if (item >= n_items) break;
    g = ng;
  }
  if (pace && tid == 0) __hip_atomic_fetch_add(pace_ctr, kPaceDone, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch of the attention kernel for one masking form (kMask, see attn_fwd_kernel): picks
// the instantiation for the P levels, quant_p, norm_same and the probe (a.diag).  Defined,
// one kMask per object, in attn_instances.hip.
template <int kMask>
void launch_attention_mask(const AttnArgs& a, int quant_p, int p_levels, int norm_same, dim3 grid, hipStream_t st);

}  // namespace faq
