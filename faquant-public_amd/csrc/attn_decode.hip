// Decode-shaped HiF4 QK/PV attention on gfx950: a few query rows per KV head over a long
// key range (decode steps, short chunks), from bf16 or packed HiF4 K/V.
//
// Reference semantics: the same tiled recurrence as the prefill kernel
// (src/faquant/simulated_flash_attention.py:457-909, decode K/V cache sfa:243-289), with
// the key range cut into splits as faq_attention_fwd_split does: P of tile t uses the
// running maximum after tile t, so a split starts from the maximum of the tiles before
// it, and the per-split partials are combined at the end.
//
// Layout of the work: GQA packing.  The G query heads of a KV head share every K/V tile,
// so one wave's 32 MFMA columns hold G heads x 32 / G positions (column n: head n % G,
// position n / G of the row block).  At one decode position that is G live columns in
// one wave, where one wave per query head would repeat each tile's QK and PV MFMAs G
// times.  Each wave is an independent (row block, split); nothing is shared between the
// waves of a workgroup, so K/V tiles go straight from HBM to registers (non-temporal
// loads: every byte is read once).
//
// Two passes, so that K is read once:
//   scores  S = K Q^T per tile (the prefill kernel's MFMA chains, bit for bit), masked
//           keys -inf; S of the live rows, the lane maxima of each tile (the two 64-key
//           halves) and each split's row maximum go to the workspace;
//   values  the running maximum before the split from the split maxima, then per tile the
//           prefill kernel's recurrence on S: m' = max(m, rowmax c1), P = exp2(S c1 - m'),
//           HiF4 P^, l and acc = alpha acc + P^ V (same operations in the same order), and
//           the partial (acc, l, m) of the split.
// S costs 8 bytes per live row and key of HBM traffic, against 512 bytes per key of bf16
// K and V (144 packed), where a second K pass would cost 256 (72).
//
// Packed HiF4 K/V (4.5 bits per value): per key row of 128 values, 16 code words (dims
// 8u .. 8u + 7 in slot (u & 1) 8 + u / 2, dim 8u + i in nibble i as 8 + the signed code: a
// lane half's QK fragments, dims 16c + 8 half, are then 8 consecutive words, and a 64-dim
// group is two runs of 4) and 2 meta words
// (per 64-dim group: the E6M2 byte ((e + 48) << 2) | m, the level-2 bits << 8, the level-3
// bits << 16; the content of hif4.py:67-79).  A value is (nibble - 8) 2^(lv2 + lv3) s / 4,
// one fma of the nibble with per-4-group constants (exact: at most six significant
// bits), so the unpacked operands are bitwise the bf16 operands of the bf16 path and the
// outputs are bitwise equal.  K unpacks in registers straight into the QK fragments; V is
// unpacked per half tile into the wave's own LDS region in the transposed layout the PV
// fragments read (the HiF4 groups of V run along head_dim, the PV contraction along keys).
#include "attn_decode.h"
#include "hif4_attention.hip"

namespace faq {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  bf16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// The rows of a decode wave and its key tiles.
struct DecWave {
  int b, kvh, j;   // batch, KV head, key split (wave-uniform)
  int pmin;        // first position of the row block (wave-uniform)
  int t_lo, t_hi;  // key tiles of the split (wave-uniform)
  bool live;       // this lane's column is a row
  int pos, hq;
  int64_t row;
};

__device__ __forceinline__ DecWave dec_wave(const DecodeArgs& a, int wave_id, int n) {
  DecWave w;
  const int item = wave_id / a.nsplit;
  w.j = wave_id - item * a.nsplit;
  const int rb = item % a.n_rb;
  const int x = item / a.n_rb;
  w.kvh = x % a.Hkv;
  w.b = x / a.Hkv;
  const int pp = n / a.G;
  w.pmin = rb * a.pb;
  w.pos = w.pmin + pp;
  w.live = pp < a.pb && w.pos < a.Lq;
  w.hq = w.kvh * a.G + (n - pp * a.G);
  w.row = (static_cast<int64_t>(w.b) * a.Hq + w.hq) * a.Lq + (w.live ? w.pos : 0);
  // bottom-right causal: the block's last position sees keys <= pos + Lk - Lq
  const int pmax = min(w.pmin + a.pb, a.Lq) - 1;
  const int kend = a.causal ? max(0, min(a.Lk, pmax + (a.Lk - a.Lq) + 1)) : a.Lk;
  const int nt = (kend + kKeyTile - 1) / kKeyTile;
  w.t_lo = min(nt, w.j * a.tps);
  w.t_hi = min(nt, w.j * a.tps + a.tps);
  return w;
}

__device__ __forceinline__ int dec_wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kDecWaves + static_cast<int>(threadIdx.x >> 6));
}

// The 8 values of code word `word` (dims 8 g8 .. 8 g8 + 7 of one 64-dim group) as bf16:
// (nibble - 8) f = fma(nibble, f, -8 f) with f = 2^(lv2 + lv3) s / 4 of its 4-dim group.
// An E6M2 byte of 0xFF marks a group that held a NaN (its values are NaN).
__device__ __forceinline__ void hif4_unpack8(uint32_t word, uint32_t meta, int g8, float* v) {
  const uint32_t sb = meta & 0xFFu;
  const uint32_t base = (sb << 21) + (77u << 23);  // s / 4: exponent e - 2, mantissa m
  const uint32_t lv2 = (meta >> (8 + g8)) & 1u;
  const uint32_t lv3 = (meta >> (16 + 2 * g8)) & 3u;
  float fa = __uint_as_float(base + ((lv2 + (lv3 & 1u)) << 23));
  float fb = __uint_as_float(base + ((lv2 + (lv3 >> 1)) << 23));
  if (sb == 0xFFu) {
    fa = __builtin_nanf("");
    fb = fa;
  }
  const float na = fa * -8.0f, nb = fb * -8.0f;
  const uint32_t lo = word & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 as bytes
  const uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float f = i < 2 ? fa : fb;
    const float nf = i < 2 ? na : nb;
    v[2 * i] = __builtin_fmaf(static_cast<float>((lo >> (8 * i)) & 0xFFu), f, nf);
    v[2 * i + 1] = __builtin_fmaf(static_cast<float>((hi >> (8 * i)) & 0xFFu), f, nf);
  }
}

// ---------------------------------------------------------------------------------------
// Scores pass.  The K operand of a tile: bf16 fragments (key krow0 + 16 kb, dims
// 16 c + 8 half, the prefill kernel's QK A operand) or the packed words they unpack from.
template <bool kPacked>
struct KTile;

template <>
struct KTile<false> {
  bf16x8 f[4][8];
};

template <>
struct KTile<true> {
  uint32_t w[4][8];  // the lane half's code words: chunk c (dims 16c + 8 half) in w[kb][c]
  uint32_t m[4][2];  // meta words of the key's two 64-dim groups
};

template <bool kPacked>
__device__ __forceinline__ void load_k_block(const DecodeArgs& a, const DecWave& w, int t, int kb, int krow0,
                                             int half, KTile<kPacked>& k) {
  const int key = min(t * kKeyTile + krow0 + 16 * kb, a.Lk - 1);  // ragged tail: masked later
  if constexpr (kPacked) {
    const int64_t r = w.b * a.kp_sb + w.kvh * a.kp_sh + key;
    const uint32_t* cw = a.kc + r * 16 + 8 * half;  // slots 8 half + c
    const u32x4 x0 = ld_nt(cw), x1 = ld_nt(cw + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      k.w[kb][i] = x0[i];
      k.w[kb][4 + i] = x1[i];
    }
#pragma unroll
    for (int g = 0; g < 2; ++g) k.m[kb][g] = __builtin_nontemporal_load(a.km + r * 2 + g);
  } else {
    const uint16_t* kp = a.k + w.b * a.k_sb + w.kvh * a.k_sh + static_cast<int64_t>(key) * a.k_sl + 8 * half;
#pragma unroll
    for (int c = 0; c < 8; ++c) k.f[kb][c] = as_bf16x8(ld_nt(kp + 16 * c));
  }
}

template <bool kPacked>
__device__ __forceinline__ bf16x8 k_fragment(const KTile<kPacked>& k, int kb, int c, int half) {
  if constexpr (kPacked) {
    const int g = c >> 2, g8 = 2 * (c & 3) + half;  // 64-dim group, 8-dim group within it
    float v[8];
    hif4_unpack8(k.w[kb][c], k.m[kb][g], g8, v);
    return pack8<true>(v);
  } else {
    return k.f[kb][c];
  }
}

template <bool kPacked>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_scores_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int wave_id = dec_wave_id();
  if (wave_id >= a.B * a.Hkv * a.n_rb * a.nsplit) return;
  const DecWave w = dec_wave(a, wave_id, n);
  const int off = a.Lk - a.Lq;

  bf16x8 qf[8];
  {
    const uint16_t* qp = a.q + w.b * a.q_sb + w.hq * a.q_sh + static_cast<int64_t>(w.live ? w.pos : 0) * a.q_sl + 8 * half;
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = w.live ? *reinterpret_cast<const bf16x8*>(qp + 16 * c) : bf16x8{};
  }
  // QK A-operand row m of key block kb is key pi(kb, m) = krow0(m) + 16 kb, so lane (n, half)
  // ends with keys 64 half + 16 kb + i of row n (the prefill kernel's layout)
  const int krow0 = 64 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  float smax = -INFINITY;
  KTile<kPacked> k;
  if (w.t_lo < w.t_hi) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) load_k_block<kPacked>(a, w, w.t_lo, kb, krow0, half, k);
  }
  for (int t = w.t_lo; t < w.t_hi; ++t) {
    const int key0 = t * kKeyTile;
    floatx16 s[4];
    // each accumulator is the chain c = 0..7 of the prefill kernel; the block's registers
    // take the next tile's block as soon as its chain has issued
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      s[kb] = floatx16{};
#pragma unroll
      for (int c = 0; c < 8; ++c) s[kb] = mfma32(k_fragment<kPacked>(k, kb, c, half), qf[c], s[kb]);
      if (t + 1 < w.t_hi) load_k_block<kPacked>(a, w, t + 1, kb, krow0, half, k);
    }
    if (key0 + kKeyTile > a.Lk || (a.causal && key0 + kKeyTile - 1 > w.pmin + off)) {
      const int lim = a.causal ? min(a.Lk - 1, w.pos + off) : a.Lk - 1;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (key0 + 64 * half + 16 * kb + i > lim) s[kb][i] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    if (w.live) {
      float* sp = a.s + w.row * a.s_stride + key0 + 64 * half;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          *reinterpret_cast<float4*>(sp + 16 * kb + 4 * u) =
              make_float4(s[kb][4 * u], s[kb][4 * u + 1], s[kb][4 * u + 2], s[kb][4 * u + 3]);
      a.gmx[(w.row * a.ntiles + t) * 2 + half] = mx;
    }
    smax = fmaxf(smax, mx);
  }
  const float sm = halves_max(smax);
  if (w.live && half == 0) a.smx[w.row * a.nsplit + w.j] = sm;
}

// ---------------------------------------------------------------------------------------
// Values pass.

// The wave's LDS region for one unpacked half tile of V (packed V): V^T rows d = 0..127 of
// 64 keys (the keys 32 s + 0..31 and 64 + 32 s + 0..31 of half tile s, as local keys
// 0..63), a 144-byte pitch (16-byte aligned fragment reads) and rows 64..127 moved by 64
// bytes, so the two lane halves of a 4-byte store (dims d and d + 64) use other banks.
constexpr int kVPitch = 144;
constexpr int kVStageBytes = 18560;
static_assert(127 * kVPitch + 64 + 128 <= kVStageBytes, "V stage region");

__device__ __forceinline__ int vrow_byte(int d) { return d * kVPitch + (d >= 64 ? 64 : 0); }

// Raw packed V of one half tile for lane (p = lane % 32, h = lane / 32): keys 2p, 2p + 1
// of the half tile's local keys, dims 64 h .. 64 h + 63 (one group).
struct VRaw {
  uint32_t w[2][8];
  uint32_t m[2];
};

__device__ __forceinline__ void load_v_raw(const DecodeArgs& a, const DecWave& w, int t, int s, int lane, VRaw& r) {
  const int p = lane & 31, h = lane >> 5;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int lk = 2 * p + e;  // local key
    const int key = t * kKeyTile + (lk < 32 ? 32 * s + lk : 64 + 32 * s + lk - 32);
    const int64_t row = w.b * a.vp_sb + w.kvh * a.vp_sh + min(key, a.Lk - 1);
    // dims 64 h + 8 u: u even in slots 4 h + u / 2, u odd in slots 8 + 4 h + u / 2
    const u32x4 x0 = ld_nt(a.vc + row * 16 + 4 * h), x1 = ld_nt(a.vc + row * 16 + 8 + 4 * h);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.w[e][2 * i] = x0[i];
      r.w[e][2 * i + 1] = x1[i];
    }
    // keys past Lk are zeros, as the bf16 V^T padding is (their P is 0, and 0 times a
    // stale value could be NaN)
    r.m[e] = key < a.Lk ? __builtin_nontemporal_load(a.vm + row * 2 + h) : 0u;
    if (key >= a.Lk) {
#pragma unroll
      for (int i = 0; i < 8; ++i) r.w[e][i] = 0x88888888u;
    }
  }
}

// Unpack a half tile into the LDS region: dim d = 64 h + 8 u + i, local keys 2p, 2p + 1 as
// one 4-byte store.
__device__ __forceinline__ void store_v_stage(const VRaw& r, int lane, uint8_t* region) {
  const int p = lane & 31, h = lane >> 5;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    float v0[8], v1[8];
    hif4_unpack8(r.w[0][u], r.m[0], u, v0);
    hif4_unpack8(r.w[1][u], r.m[1], u, v1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t pair = __builtin_amdgcn_perm(__float_as_uint(v1[i]), __float_as_uint(v0[i]), 0x07060302u);
      *reinterpret_cast<uint32_t*>(region + vrow_byte(64 * h + 8 * u + i) + 4 * p) = pair;
    }
  }
}

// Orders this wave's LDS accesses around a stage change (the LDS unit runs one wave's
// accesses in order; this keeps the compiler from moving them across).
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

template <int LV, bool kQuantP, bool kSame, bool kPacked>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_values_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(128))) uint8_t lds[kPacked ? kDecWaves * kVStageBytes : 16];
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int wave_id = dec_wave_id();
  if (wave_id >= a.B * a.Hkv * a.n_rb * a.nsplit) return;
  const DecWave w = dec_wave(a, wave_id, n);
  uint8_t* const region = lds + (threadIdx.x >> 6) * (kPacked ? kVStageBytes : 0);

  // running maximum before the split: the largest split maximum of the splits before it
  // (raw scores; c1 > 0 and rounding is monotonic, so scaling the maximum once equals the
  // maximum of the c1-scaled tile maxima)
  float ms = -INFINITY;
  if (w.live) {
    for (int jj = half; jj < w.j; jj += 2) ms = fmaxf(ms, a.smx[w.row * a.nsplit + jj]);
  }
  float m_run = halves_max(ms) * a.c1;
  float l_run = 0.0f;
  floatx16 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = floatx16{};

  bf16x2_t ones2;
  {
    const uint32_t one2 = 0x3F803F80u;
    __builtin_memcpy(&ones2, &one2, 4);
  }
  const float* srow = a.s + w.row * a.s_stride + 64 * half;
  const uint16_t* vbase = a.vt + w.b * a.v_sb + w.kvh * a.v_sh + static_cast<int64_t>(n) * a.v_sd + 64 * half;

  // S of chunk c (keys 64 half + 8 c .. + 7 of tile t) in a ring of four chunks and, with
  // bf16 V, its V^T fragments in a ring of two (the register budget of two waves per SIMD)
  float sv[4][8];
  bf16x8 vv[2][4];
  auto load_s = [&](int t, int c, int slot) {
    if (w.live) {
      const float* sp = srow + t * kKeyTile + 8 * c;
      const u32x4 x0 = ld_nt(sp), x1 = ld_nt(sp + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[slot][i] = __uint_as_float(x0[i]);
        sv[slot][4 + i] = __uint_as_float(x1[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[slot][i] = -INFINITY;
    }
  };
  auto load_v = [&](int t, int c, int slot) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
      vv[slot][mb] = as_bf16x8(ld_nt(vbase + static_cast<int64_t>(32 * mb) * a.v_sd + t * kKeyTile + 8 * c));
  };
  VRaw vr;
  if (w.t_lo < w.t_hi) {
#pragma unroll
    for (int c = 0; c < 4; ++c) load_s(w.t_lo, c, c);
    if constexpr (kPacked) {
      load_v_raw(a, w, w.t_lo, 0, lane, vr);
    } else {
      load_v(w.t_lo, 0, 0);
      load_v(w.t_lo, 1, 1);
    }
  }
  float2 gnext = make_float2(-INFINITY, -INFINITY);
  if (w.live && w.t_lo < w.t_hi) gnext = *reinterpret_cast<const float2*>(a.gmx + (w.row * a.ntiles + w.t_lo) * 2);

  for (int t = w.t_lo; t < w.t_hi; ++t) {
    const float2 g = gnext;
    if (w.live && t + 1 < w.t_hi) gnext = *reinterpret_cast<const float2*>(a.gmx + (w.row * a.ntiles + t + 1) * 2);
    // the prefill kernel's tile recurrence: g.x, g.y are the lane maxima of the two halves
    const float mx = half ? g.y : g.x;
    const float mx_row = fmaxf(g.x, g.y);
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
    }
    PQuant pq;
    if (kQuantP) pq = pquant_setup<LV>(__builtin_amdgcn_exp2f(__builtin_fmaf(mx, a.c1, nm)));
    float rowsum = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int slot = c & 3;
      bf16x8 va[4];
      if constexpr (kPacked) {
        if ((c & 3) == 0) {
          // unpack half tile c / 4 (the previous one's fragment reads were issued before)
          wave_lds_order();
          store_v_stage(vr, lane, region);
          wave_lds_order();
          const int s_next = (c >> 2) ^ 1;
          const int t_next = (c >> 2) ? t + 1 : t;
          if (t_next < w.t_hi) load_v_raw(a, w, t_next, s_next, lane, vr);
        }
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
          va[mb] = *reinterpret_cast<const bf16x8*>(region + vrow_byte(32 * mb + n) + 64 * half + 16 * (c & 3));
      } else {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) va[mb] = vv[c & 1][mb];
        // the slot takes chunk c + 2 (of this tile or the next)
        if (c < 6) load_v(t, c + 2, c & 1);
        else if (t + 1 < w.t_hi) load_v(t + 1, c - 6, c & 1);
      }
      float pc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pc[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[slot][j], a.c1, nm));
      // the S slot takes chunk c + 4 (of this tile or the next)
      if (c < 4) load_s(t, c + 4, slot);
      else if (t + 1 < w.t_hi) load_s(t + 1, c - 4, slot);
      if (!(kQuantP && kSame)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) rowsum += pc[j];
      }
      bf16x8 pcur, plcur;
      if (kQuantP) {
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
      } else {
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = pc[j] - bf16_rne(pc[j]);
        pcur = pack8<false>(pc);
        plcur = pack8<false>(r);
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        acc[mb] = mfma32(va[mb], pcur, acc[mb]);
        if (!kQuantP) acc[mb] = mfma32(va[mb], plcur, acc[mb]);
      }
    }
    l_run += halves_sum(rowsum);
  }

  if (w.live) {
    float* po = a.part_o + (static_cast<int64_t>(w.j) * a.rows_total + w.row) * kDim;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<float4*>(po + 32 * mb + 8 * j + 4 * half) =
            make_float4(acc[mb][4 * j], acc[mb][4 * j + 1], acc[mb][4 * j + 2], acc[mb][4 * j + 3]);
    if (half == 0) {
      float* lm = a.part_lm + (static_cast<int64_t>(w.j) * a.rows_total + w.row) * 2;
      lm[0] = l_run;
      lm[1] = m_run;
    }
  }
}

template <int LV, bool kQuantP, bool kSame>
void launch_values(const DecodeArgs& a, int packed, dim3 grid, hipStream_t st) {
  if (packed) hipLaunchKernelGGL((dec_values_kernel<LV, kQuantP, kSame, true>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((dec_values_kernel<LV, kQuantP, kSame, false>), grid, dim3(256), 0, st, a);
}

template <int LV>
void launch_values_lv(const DecodeArgs& a, int packed, int quant_p, int same, dim3 grid, hipStream_t st) {
  if (quant_p && same) launch_values<LV, true, true>(a, packed, grid, st);
  else if (quant_p) launch_values<LV, true, false>(a, packed, grid, st);
  else launch_values<123, false, false>(a, packed, grid, st);
}

}  // namespace

void launch_decode(const DecodeArgs& a, int packed, int quant_p, int p_levels, int norm_same, hipStream_t st) {
  const int64_t waves = static_cast<int64_t>(a.B) * a.Hkv * a.n_rb * a.nsplit;
  const dim3 grid(static_cast<unsigned>((waves + kDecWaves - 1) / kDecWaves));
  if (packed) hipLaunchKernelGGL((dec_scores_kernel<true>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((dec_scores_kernel<false>), grid, dim3(256), 0, st, a);
  const int lv = quant_p ? p_levels : 123;
  if (lv == 12) launch_values_lv<12>(a, packed, quant_p, norm_same, grid, st);
  else if (lv == 13) launch_values_lv<13>(a, packed, quant_p, norm_same, grid, st);
  else launch_values_lv<123>(a, packed, quant_p, norm_same, grid, st);
}

}  // namespace faq
