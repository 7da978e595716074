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
// times.  Each wave is an independent (row block, split) with its own LDS region: K and V
// come as natural [key][dim] rows (a tile is 32 KiB of contiguous bf16, or 9 KiB packed),
// loaded with coalesced row reads and staged half a tile at a time in the layout the MFMA
// fragments read (V transposed), the next half tile's loads in flight meanwhile.
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
// K and V (144 packed), where a second K pass would cost 256 (72).  With at most 4 or 8
// live columns (a decode step) and P summed as P^, the values pass computes P and P^ in
// a compact layout (dec_values_compact_kernel) and moves P^ into the MFMA layout through
// LDS, with the same results.
//
// Packed HiF4 K/V (4.5 bits per value): per key row of 128 values, 16 code words (dims
// 8u .. 8u + 7 in slot (u & 1) 8 + u / 2, dim 8u + i in nibble i as 8 + the signed code: a
// lane half's QK fragments, dims 16c + 8 half, are then 8 consecutive words, and a 64-dim
// group is two runs of 4) and 2 meta words
// (per 64-dim group: the E6M2 byte ((e + 48) << 2) | m, the level-2 bits << 8, the level-3
// bits << 16; the content of hif4.py:67-79).  A value is (nibble - 8) 2^(lv2 + lv3) s / 4,
// one fma of the nibble with per-4-group constants (exact: at most six significant
// bits), so the unpacked operands are bitwise the bf16 operands of the bf16 path and the
// outputs are bitwise equal.  Both unpack per key row on their way into LDS.
#include <cstdlib>
#include <cstring>

#include "attn_decode.h"
#include "hif4_attention.hip"
#include "hif4_packed.h"

namespace faq {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// The rows of a decode wave and its key tiles.
struct DecWave {
  int item;        // work item: (batch, KV head, row block) (wave-uniform)
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
  w.item = item;
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

// One DPP step of a maximum: x and lane (ctrl's source lane) of x.
template <int kCtrl>
__device__ __forceinline__ float dpp_max(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false);
  return fmaxf(x, __int_as_float(y));
}

// Maximum over the 64 lanes, wave-uniform: within each row of 16 lanes by DPP (lane pairs,
// quads, the two halves of a row mirrored, the row mirrored), then the four row maxima read
// from lanes 0, 16, 32, 48.  No LDS round trips; a maximum does not depend on the order.
__device__ __forceinline__ float wave_max_f32(float x) {
  x = dpp_max<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x = dpp_max<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x = dpp_max<0x141>(x);  // row_half_mirror
  x = dpp_max<0x140>(x);  // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ int dec_wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kDecWaves + static_cast<int>(threadIdx.x >> 6));
}

// Orders this wave's LDS accesses around a stage change (the LDS unit runs one wave's
// accesses in order; this keeps the compiler from moving them across).
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Half tiles.  Half tile s of a 128-key tile holds the keys 32 s + 0..31 and 64 + 32 s +
// 0..31 as local keys r = 0..63: the QK key blocks kb = 2 s, 2 s + 1 (keys pi(kb, m)) and
// the PV chunks c = 4 s .. 4 s + 3 (keys 64 half + 8 c + 0..7) of the prefill layout.
__device__ __forceinline__ int stage_key(int r, int s) { return (r & 31) + 32 * s + 64 * (r >> 5); }

// ---------------------------------------------------------------------------------------
// Half tiles of K and of V are staged in the wave's LDS region the same way: bf16 rows of the
// 64 local keys at a pitch of 17 16-byte units, from coalesced row loads: bf16 rows
// (instruction i, lane l: unit l % 16 of local key 4 i + l / 16, 1 KiB contiguous per
// instruction) or packed rows (lane l: the 72 bytes of local key l, unpacked in registers).
// The QK fragments are plain 16-byte reads of that layout (the prefill kernel's
// conflict-free pitch); the PV fragments are transposing reads (ds_read_b64_tr_b16).
constexpr int kStageBytes = 64 * kRowUnits * 16;  // 17408
constexpr int kRowBytes = kRowUnits * 16;

// One operand's rows of a (batch, KV head): bf16 rows (key 0's row, row stride in bytes) or
// packed rows (key 0's 16 code words and its 2 meta words).
struct RowSrc {
  const uint8_t* base;
  const uint8_t* meta;
  uint32_t row_bytes;
};

template <bool kPacked>
struct RowsRaw;

template <>
struct RowsRaw<false> {
  u32x4 x[16];
};

template <>
struct RowsRaw<true> {
  u32x4 c[4];     // the 16 code words of the key
  uint32_t m[2];  // its two meta words
};

// Per-lane byte offsets of the row loads from a half tile's first key (loop-invariant).  bf16
// rows: instruction i, lane l reads unit l % 16 of local row 4 i + l / 16, which is key
// 4 i + l / 16 + 32 [i >= 8] of the half tile; packed rows: lane l reads local key l, key
// (l % 32) + 64 (l / 32).
template <bool kPacked>
struct RowOffs;

template <>
struct RowOffs<false> {
  uint32_t v[16];
};

template <>
struct RowOffs<true> {
  uint32_t c, m;
};

template <bool kPacked>
__device__ __forceinline__ RowOffs<kPacked> row_offsets(const RowSrc& src, int lane) {
  RowOffs<kPacked> o;
  if constexpr (kPacked) {
    const uint32_t k = static_cast<uint32_t>((lane & 31) + 64 * (lane >> 5));
    o.c = 64u * k;
    o.m = 8u * k;
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      o.v[i] = static_cast<uint32_t>(4 * i + (lane >> 4) + (i >= 8 ? 32 : 0)) * src.row_bytes + 16u * (lane & 15);
  }
  return o;
}

// Raw buffer resource over the `keys` rows of `row_bytes` each from `base` (empty when keys
// <= 0).  32-bit arithmetic: one head's rows span less than 4 GiB.  The arguments are
// wave-uniform; they are read from the first lane so that the resource is built in scalar
// registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const uint8_t* base, int keys, uint32_t row_bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32));
  const uint32_t bytes = __builtin_amdgcn_readfirstlane(keys > 0 ? static_cast<uint32_t>(keys) * row_bytes : 0u);
  return make_rsrc(reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo), bytes);
}

// Loads of half tile s of tile t (local keys 0..31 are keys 32 s + 0..31 of the tile, local keys
// 32..63 keys 64 + 32 s + 0..31) through buffer resources that start at the half tile's first
// key and end at key Lk: the address arithmetic is scalar, and rows past Lk read as zeros
// without a memory access (K: masked later; V: zeroed in LDS by zero_tail_rows, since packed
// zeros do not decode to zero).  `valid` false (wave-uniform: a prefetch past the split's last
// tile) gives an empty resource.  The loads are unconditional, so the memory counter the
// waits use sees the same sequence on every iteration (a wait then covers only the loads it
// needs: the counter completes in order).
template <bool kPacked>
__device__ __forceinline__ void load_rows(const RowSrc& src, const RowOffs<kPacked>& off, int Lk, int t, int s,
                                          RowsRaw<kPacked>& raw, bool valid = true) {
  const int key0 = valid ? t * kKeyTile + 32 * s : 0;
  const int keys = valid ? Lk - key0 : 0;
  if constexpr (kPacked) {
    const __amdgpu_buffer_rsrc_t rc = rows_rsrc(src.base + static_cast<int64_t>(key0) * 64, keys, 64u);
    const __amdgpu_buffer_rsrc_t rm = rows_rsrc(src.meta + static_cast<int64_t>(key0) * 8, keys, 8u);
#pragma unroll
    for (int i = 0; i < 4; ++i) raw.c[i] = __builtin_amdgcn_raw_buffer_load_b128(rc, off.c + 16u * i, 0, 0);
    const auto mm = __builtin_amdgcn_raw_buffer_load_b64(rm, off.m, 0, 0);
    raw.m[0] = mm[0];
    raw.m[1] = mm[1];
  } else {
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(src.base + static_cast<int64_t>(key0) * src.row_bytes, keys, src.row_bytes);
#pragma unroll
    for (int i = 0; i < 16; ++i) raw.x[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off.v[i], 0, 0);
  }
}

// Zeros of the staged rows past Lk (the zero padding of the bf16 V^T layout: P is 0 there,
// and 0 times a repeated NaN must not reach PV).  Lane l clears local key l.
__device__ __forceinline__ void zero_tail_rows(int Lk, int t, int s, int lane, uint8_t* region) {
  if (t * kKeyTile + stage_key(lane, s) >= Lk) {
#pragma unroll
    for (int u = 0; u < 16; ++u) *reinterpret_cast<u32x4*>(region + lane * kRowBytes + u * 16) = u32x4{0u, 0u, 0u, 0u};
  }
}

template <bool kPacked>
__device__ __forceinline__ void store_rows(const RowsRaw<kPacked>& raw, int lane, uint8_t* region) {
  if constexpr (kPacked) {
    const float s4[2] = {hif4_group_s4(raw.m[0]), hif4_group_s4(raw.m[1])};
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int slot = (u & 1) * 8 + (u >> 1);  // dims 8u .. 8u + 7
      float v[8];
      hif4_unpack8(raw.c[slot >> 2][slot & 3], s4[u >> 3], raw.m[u >> 3], u & 7, v);
      *reinterpret_cast<bf16x8*>(region + lane * kRowBytes + u * 16) = pack8<true>(v);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      *reinterpret_cast<u32x4*>(region + (4 * i + (lane >> 4)) * kRowBytes + (lane & 15) * 16) = raw.x[i];
  }
}

template <bool kPacked>
__device__ __forceinline__ RowSrc k_source(const DecodeArgs& a, const DecWave& w) {
  if constexpr (kPacked) {
    const int64_t row0 = w.b * a.kp_sb + w.kvh * a.kp_sh;
    return RowSrc{reinterpret_cast<const uint8_t*>(a.kc + row0 * 16), reinterpret_cast<const uint8_t*>(a.km + row0 * 2), 0u};
  } else {
    return RowSrc{reinterpret_cast<const uint8_t*>(a.k + w.b * a.k_sb + w.kvh * a.k_sh), nullptr,
                  static_cast<uint32_t>(2 * a.k_sl)};
  }
}

template <bool kPacked>
__device__ __forceinline__ RowSrc v_source(const DecodeArgs& a, const DecWave& w) {
  if constexpr (kPacked) {
    const int64_t row0 = w.b * a.vp_sb + w.kvh * a.vp_sh;
    return RowSrc{reinterpret_cast<const uint8_t*>(a.vc + row0 * 16), reinterpret_cast<const uint8_t*>(a.vm + row0 * 2), 0u};
  } else {
    return RowSrc{reinterpret_cast<const uint8_t*>(a.v + w.b * a.v_sb + w.kvh * a.v_sh), nullptr,
                  static_cast<uint32_t>(2 * a.v_sl)};
  }
}

// Scores pass.
template <bool kPacked>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_scores_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(128))) uint8_t lds[kDecWaves * kStageBytes];
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int wave_id = dec_wave_id();
  if (wave_id >= a.B * a.Hkv * a.n_rb * a.nsplit) return;
  const DecWave w = dec_wave(a, wave_id, n);
  uint8_t* const region = lds + (threadIdx.x >> 6) * kStageBytes;
  const int off = a.Lk - a.Lq;
  const RowSrc ksrc = k_source<kPacked>(a, w);
  const RowOffs<kPacked> koff = row_offsets<kPacked>(ksrc, lane);

  bf16x8 qf[8];
  {
    const uint16_t* qp = a.q + w.b * a.q_sb + w.hq * a.q_sh + static_cast<int64_t>(w.live ? w.pos : 0) * a.q_sl + 8 * half;
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = w.live ? *reinterpret_cast<const bf16x8*>(qp + 16 * c) : bf16x8{};
  }
  // QK A-operand row m of key block kb is key pi(kb, m) = krow0(m) + 16 kb, so lane (n, half)
  // ends with keys 64 half + 16 kb + i of row n (the prefill kernel's layout); as a local key
  // of half tile kb / 2 that is (pi & 31) + 32 (pi >> 6)
  const int krow0 = 64 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  float smax = -INFINITY;
  RowsRaw<kPacked> raw;
  if (w.t_lo < w.t_hi) load_rows<kPacked>(ksrc, koff, a.Lk, w.t_lo, 0, raw);
  for (int t = w.t_lo; t < w.t_hi; ++t) {
    const int key0 = t * kKeyTile;
    floatx16 s[4];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      wave_lds_order();  // the previous half tile's fragment reads are issued
      store_rows<kPacked>(raw, lane, region);
      wave_lds_order();
      // the next half tile's loads fly during this one's MFMAs (past the split's last tile:
      // an empty resource)
      load_rows<kPacked>(ksrc, koff, a.Lk, t + st, st ^ 1, raw, st == 0 || t + 1 < w.t_hi);
#pragma unroll
      for (int kb = 2 * st; kb < 2 * st + 2; ++kb) {
        const int pi = krow0 + 16 * kb;
        const uint8_t* kp = region + (((pi & 31) + 32 * (pi >> 6)) * kRowUnits + half) * 16;
        // each accumulator is the chain c = 0..7 of the prefill kernel
        s[kb] = floatx16{};
#pragma unroll
        for (int c = 0; c < 8; ++c) s[kb] = mfma32(lds_read_at(kp, 32 * c), qf[c], s[kb]);
      }
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

// Scores pass over packed rows without LDS: lane (n, half) unpacks the A operand of its MFMA
// rows itself.  Key block kb's row n is key pi = krow0 + 16 kb of the tile (the prefill
// layout above), and the lane's chunk c is dims 16 c + 8 half .. + 7 of that key: code word
// 8 half + c (the lane's 32 code bytes are contiguous) unpacked with its 64-dim group's meta
// word, exactly as store_rows unpacks it.  The loads go through buffer resources that end at
// key Lk (rows past it read as zeros and are masked), and the MFMAs take the same operands
// in the same order as the staged form, so the scores are bitwise equal.  Same-box decode
// steps: 61.2 -> 60.3 us at 128k keys, 29.3 -> 28.0 us at 32k read from HBM.  (The same
// form over bf16 rows was slower, 139 against 120 us at 128k: its 16-byte loads touch 32
// rows each, where the staged form reads 1 KiB runs.)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_scores_packed_direct_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int wave_id = dec_wave_id();
  if (wave_id >= a.B * a.Hkv * a.n_rb * a.nsplit) return;
  const DecWave w = dec_wave(a, wave_id, n);
  const int off = a.Lk - a.Lq;
  const RowSrc ksrc = k_source<true>(a, w);

  bf16x8 qf[8];
  {
    const uint16_t* qp = a.q + w.b * a.q_sb + w.hq * a.q_sh + static_cast<int64_t>(w.live ? w.pos : 0) * a.q_sl + 8 * half;
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = w.live ? *reinterpret_cast<const bf16x8*>(qp + 16 * c) : bf16x8{};
  }
  const int krow0 = 64 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  float smax = -INFINITY;
  for (int t = w.t_lo; t < w.t_hi; ++t) {
    const int key0 = t * kKeyTile;
    floatx16 s[4];
    {
      const __amdgpu_buffer_rsrc_t rc = rows_rsrc(ksrc.base + static_cast<int64_t>(key0) * 64, a.Lk - key0, 64u);
      const __amdgpu_buffer_rsrc_t rm = rows_rsrc(ksrc.meta + static_cast<int64_t>(key0) * 8, a.Lk - key0, 8u);
      u32x4 cw[4][2];
      uint32_t mw[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const uint32_t pi = static_cast<uint32_t>(krow0 + 16 * kb);
        cw[kb][0] = __builtin_amdgcn_raw_buffer_load_b128(rc, pi * 64u + 32u * half, 0, 0);
        cw[kb][1] = __builtin_amdgcn_raw_buffer_load_b128(rc, pi * 64u + 32u * half + 16u, 0, 0);
        const auto mm = __builtin_amdgcn_raw_buffer_load_b64(rm, pi * 8u, 0, 0);
        mw[kb][0] = mm[0];
        mw[kb][1] = mm[1];
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const float s4[2] = {hif4_group_s4(mw[kb][0]), hif4_group_s4(mw[kb][1])};
        s[kb] = floatx16{};
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float v[8];
          hif4_unpack8(cw[kb][c >> 2][c & 3], s4[c >> 2], mw[kb][c >> 2], 2 * (c & 3) + half, v);
          s[kb] = mfma32(pack8<true>(v), qf[c], s[kb]);
        }
      }
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
// Values pass.  The PV A operand of chunk c (V^T rows 32 mb + m, keys 64 half + 8 c + 0..7)
// comes from the natural half tile by two transposing reads: within each 16-lane group,
// lane i of ds_read_b64_tr_b16 receives element i % 4 of the 8 bytes addressed by lanes
// 4k + i / 4, k = 0..3.  Lane jj of group g addresses local key 32 (g / 2) + 8 (c % 4) + jj / 4
// (+ 4 for the second read), dims 32 mb + 16 (g % 2) + 4 (jj % 4) .. + 3, so lane i receives
// dim 32 mb + 16 (g % 2) + i of four consecutive keys.
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ __forceinline__ bf16x8 vt_fragment(const uint8_t* region, int lane, int mb, int cc) {
  const int g = lane >> 4, jj = lane & 15;
  const int row = 32 * (g >> 1) + 8 * cc + (jj >> 2);
  const int dim = 32 * mb + 16 * (g & 1) + 4 * (jj & 3);
  const uint8_t* p = region + row * kRowBytes + 2 * dim;
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 4 * kRowBytes));
  bf16x8 r;
  __builtin_memcpy(&r, &lo, 8);
  __builtin_memcpy(reinterpret_cast<char*>(&r) + 8, &hi, 8);
  return r;
}

// Running maximum before split w.j of column n, c1-scaled: the largest split maximum of
// the splits before it (raw scores; c1 > 0 and rounding is monotonic, so scaling the
// maximum once equals the maximum of the c1-scaled tile maxima).  The 64 lanes read 64
// splits of every live column (at most kCols) at a time, two such chunks per round (all
// their loads in flight together), then each column's maximum is reduced across the wave.
template <int kCols>
__device__ __forceinline__ float running_max_before(const DecodeArgs& a, const DecWave& w, int lane, int n) {
  float m_run = -INFINITY;
  const int nrows = min(min(a.G * a.pb, a.G * (a.Lq - w.pmin)), kCols);  // live columns 0 .. nrows - 1
  float mr[kCols];
#pragma unroll
  for (int r = 0; r < kCols; ++r) mr[r] = -INFINITY;
  const int64_t row0 = (static_cast<int64_t>(w.b) * a.Hq + w.kvh * a.G) * a.Lq + w.pmin;
  for (int j0 = 0; j0 < w.j; j0 += 128) {
    float x[2][kCols];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int jj = j0 + 64 * q + lane;
#pragma unroll
      for (int r = 0; r < kCols; ++r) {
        // column r: head r % G, position pmin + r / G
        x[q][r] = -INFINITY;
        if (r < nrows && jj < w.j)
          x[q][r] = a.smx[(row0 + static_cast<int64_t>(r % a.G) * a.Lq + r / a.G) * a.nsplit + jj];
      }
    }
#pragma unroll
    for (int r = 0; r < kCols; ++r) mr[r] = fmaxf(mr[r], fmaxf(x[0][r], x[1][r]));
  }
#pragma unroll
  for (int r = 0; r < kCols; ++r) {
    if (r < nrows) {
      const float m = wave_max_f32(mr[r]);
      if (n == r) m_run = m * a.c1;
    }
  }
  return m_run;
}

// The same maximum in two steps, for a few columns: rmax_issue loads the maxima of splits
// 0..127 (unconditional loads of clamped indices) before the first tile's loads are issued,
// so that waiting for them does not wait for the tile; rmax_finish drops the lanes outside
// [0, w.j), reads the splits from 128 on, and reduces each live column across the wave.
template <int kCols>
__device__ __forceinline__ const float* rmax_row(const DecodeArgs& a, const DecWave& w, int r, int nrows) {
  const int rr = min(r, nrows - 1);  // column rr: head rr % G, position pmin + rr / G
  const int64_t row0 = (static_cast<int64_t>(w.b) * a.Hq + w.kvh * a.G) * a.Lq + w.pmin;
  return a.smx + (row0 + static_cast<int64_t>(rr % a.G) * a.Lq + rr / a.G) * a.nsplit;
}

template <int kCols>
__device__ __forceinline__ int rmax_rows(const DecodeArgs& a, const DecWave& w) {
  return min(min(a.G * a.pb, a.G * (a.Lq - w.pmin)), kCols);  // live columns 0 .. nrows - 1
}

template <int kCols>
__device__ __forceinline__ void rmax_issue(const DecodeArgs& a, const DecWave& w, int lane, uint32_t (&x)[2][kCols]) {
  const int nrows = rmax_rows<kCols>(a, w);
  const int jmax = max(w.j - 1, 0);
#pragma unroll
  for (int r = 0; r < kCols; ++r) {
    const float* sm = rmax_row<kCols>(a, w, r, nrows);
#pragma unroll
    for (int q = 0; q < 2; ++q) x[q][r] = __float_as_uint(sm[min(64 * q + lane, jmax)]);
  }
}

template <int kCols>
__device__ __forceinline__ float rmax_finish(const DecodeArgs& a, const DecWave& w, int lane, int n,
                                             const uint32_t (&x)[2][kCols]) {
  const int nrows = rmax_rows<kCols>(a, w);
  float mr[kCols];
#pragma unroll
  for (int r = 0; r < kCols; ++r)
    mr[r] = fmaxf(lane < w.j ? __uint_as_float(x[0][r]) : -INFINITY, 64 + lane < w.j ? __uint_as_float(x[1][r]) : -INFINITY);
  for (int j0 = 128; j0 < w.j; j0 += 128) {
    float y[2][kCols];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int jj = j0 + 64 * q + lane;
#pragma unroll
      for (int r = 0; r < kCols; ++r) y[q][r] = jj < w.j ? rmax_row<kCols>(a, w, r, nrows)[jj] : -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < kCols; ++r) mr[r] = fmaxf(mr[r], fmaxf(y[0][r], y[1][r]));
  }
  float m_run = -INFINITY;
#pragma unroll
  for (int r = 0; r < kCols; ++r) {
    if (r < nrows) {
      const float m = wave_max_f32(mr[r]);
      if (n == r) m_run = m * a.c1;
    }
  }
  return m_run;
}

template <int LV, bool kQuantP, bool kSame, bool kPacked>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_values_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(128))) uint8_t lds[kDecWaves * kStageBytes];
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int wave_id = dec_wave_id();
  if (wave_id >= a.B * a.Hkv * a.n_rb * a.nsplit) return;
  const DecWave w = dec_wave(a, wave_id, n);
  uint8_t* const region = lds + (threadIdx.x >> 6) * kStageBytes;
  const RowSrc vsrc = v_source<kPacked>(a, w);
  const RowOffs<kPacked> voff = row_offsets<kPacked>(vsrc, lane);

  const float* srow = a.s + w.row * a.s_stride + 64 * half;
  // S of chunk c (keys 64 half + 8 c .. + 7 of tile t) in a ring of four chunks, kept as
  // loaded (unconditional loads: lanes without a row read a row of this KV head, and their
  // scores and lane maxima are made -inf where they are used, so that no select right after
  // a load makes the wave wait for it)
  u32x4 sv[4][2];
  auto load_s = [&](int t, int c, int slot) {
    const float* sp = srow + t * kKeyTile + 8 * c;
    sv[slot][0] = ld16(sp);
    sv[slot][1] = ld16(sp + 4);
  };
  auto load_g = [&](int t) { return *reinterpret_cast<const float2*>(a.gmx + (w.row * a.ntiles + t) * 2); };
  // the first tile's lane maxima, V half tile and S chunks are in flight (in the order they
  // are used) while the maximum below is read
  RowsRaw<kPacked> vr;
  float2 gnext = make_float2(-INFINITY, -INFINITY);
  if (w.t_lo < w.t_hi) {
    gnext = load_g(w.t_lo);
    load_rows<kPacked>(vsrc, voff, a.Lk, w.t_lo, 0, vr);
#pragma unroll
    for (int c = 0; c < 4; ++c) load_s(w.t_lo, c, c);
  }

  // running maximum before the split (the first tile's loads fly meanwhile)
  float m_run = running_max_before<32>(a, w, lane, n);
  float l_run = 0.0f;
  floatx16 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = floatx16{};

  bf16x2_t ones2;
  {
    const uint32_t one2 = 0x3F803F80u;
    __builtin_memcpy(&ones2, &one2, 4);
  }
  for (int t = w.t_lo; t < w.t_hi; ++t) {
    const int tn = min(t + 1, w.t_hi - 1);  // the next tile (past the last: a repeat, unused)
    const float2 g = w.live ? gnext : make_float2(-INFINITY, -INFINITY);
    gnext = load_g(tn);
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
    if (kQuantP) pq = pquant_setup<LV>(__builtin_amdgcn_exp2f(p_arg<!(kQuantP && kSame)>(mx, a.c1, nm)));
    float rowsum = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int slot = c & 3;
      bf16x8 va[4];
      if ((c & 3) == 0) {
        // stage half tile c / 4 (the previous one's fragment reads were issued before), then
        // load the next one
        wave_lds_order();
        store_rows<kPacked>(vr, lane, region);
        if ((t + 1) * kKeyTile > a.Lk) zero_tail_rows(a.Lk, t, c >> 2, lane, region);
        wave_lds_order();
        load_rows<kPacked>(vsrc, voff, a.Lk, t + (c >> 2), (c >> 2) ^ 1, vr, c == 0 || t + 1 < w.t_hi);
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) va[mb] = vt_fragment(region, lane, mb, c & 3);
      float pc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sj = w.live ? __uint_as_float(sv[slot][j >> 2][j & 3]) : -INFINITY;
        pc[j] = __builtin_amdgcn_exp2f(p_arg<!(kQuantP && kSame)>(sj, a.c1, nm));
      }
      // the S slot takes chunk c + 4 (of this tile or the next)
      load_s(c < 4 ? t : tn, (c + 4) & 7, slot);
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

// Values pass for at most kCols = 4 or 8 live columns (G x query positions <= kCols: a
// decode step of up to eight heads per KV head), P quantized and summed as P^ (the
// quantized-same normalizer).  The recurrence of the full values pass, with P and P^
// computed in a compact layout: unit u = l + 64 i (i < kCols / 4) of lane l holds the 8
// keys 64 h + 8 c .. + 7 of column u / 16 (h = (u / 8) & 1, c = u & 7), kCols / 4 pquant8
// per lane and tile instead of eight for 32 columns of which 32 - kCols are empty.  The
// P^ chunks go through LDS into the PV B operand layout of the full pass (lane (n, half),
// chunk c), where the row sum and PV run as there, so every output bit is the same.
template <int LV, bool kPacked, int kCols>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_values_compact_kernel(DecodeArgs a) {
  static_assert(kCols == 4 || kCols == 8, "compact columns");
  constexpr int kUnits = kCols / 4;                   // compact units per lane
  constexpr int kRegion = kStageBytes + kCols * 256;  // V half tile, then 16 kCols P^ chunks
  __shared__ __attribute__((aligned(128))) uint8_t lds[kDecWaves * kRegion];
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int wave_id = dec_wave_id();
  if (wave_id >= a.B * a.Hkv * a.n_rb * a.nsplit) return;
  const DecWave w = dec_wave(a, wave_id, n);
  uint8_t* const region = lds + (threadIdx.x >> 6) * kRegion;
  uint8_t* const pslots = region + kStageBytes;
  const RowSrc vsrc = v_source<kPacked>(a, w);
  const RowOffs<kPacked> voff = row_offsets<kPacked>(vsrc, lane);

  // this lane's compact units: columns cr + 4 i, key half ch, chunk cc
  const int cr = lane >> 4, ch = (lane >> 3) & 1, cc = lane & 7;
  bool clive[kUnits];
  const float* sc[kUnits];
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    const DecWave wc = dec_wave(a, wave_id, cr + 4 * i);
    clive[i] = wc.live;
    sc[i] = a.s + wc.row * a.s_stride + 64 * ch + 8 * cc;
  }
  // S chunks and lane maxima are kept as loaded and made -inf for lanes without a row where
  // they are used (in the tile loop): a select right after the loads would make the wave
  // wait for them early
  auto load_sc = [&](int t, u32x4 (&x)[kUnits][2]) {
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      x[u][0] = ld16(sc[u] + t * kKeyTile);
      x[u][1] = ld16(sc[u] + t * kKeyTile + 4);
    }
  };
  auto load_g = [&](int t) { return *reinterpret_cast<const float2*>(a.gmx + (w.row * a.ntiles + t) * 2); };
  if (w.t_lo >= w.t_hi) {
    // an empty split (past a causal row block's last key): a zero partial, which the combine
    // weighs 0 (the split maximum does not matter then)
    if (w.live) {
      float* po = a.part_o + (static_cast<int64_t>(w.j) * a.rows_total + w.row) * kDim;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<float4*>(po + 32 * mb + 8 * j + 4 * half) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (half == 0) {
        float* lm = a.part_lm + (static_cast<int64_t>(w.j) * a.rows_total + w.row) * 2;
        lm[0] = 0.0f;
        lm[1] = -INFINITY;
      }
    }
    return;
  }
  // the split maxima before this split first, then the first tile's lane maxima, V half tile
  // and S chunks, all in flight together (unconditional, so that the waits count them exactly)
  uint32_t rmx[2][kCols];
  rmax_issue<kCols>(a, w, lane, rmx);
  RowsRaw<kPacked> vr;
  u32x4 snext[kUnits][2];
  float2 gnext = load_g(w.t_lo);
  load_rows<kPacked>(vsrc, voff, a.Lk, w.t_lo, 0, vr);
  load_sc(w.t_lo, snext);
  float m_run = rmax_finish<kCols>(a, w, lane, n, rmx);
  float l_run = 0.0f;
  floatx16 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = floatx16{};
  bf16x2_t ones2;
  {
    const uint32_t one2 = 0x3F803F80u;
    __builtin_memcpy(&ones2, &one2, 4);
  }
  for (int t = w.t_lo; t < w.t_hi; ++t) {
    const int tn = min(t + 1, w.t_hi - 1);  // the next tile (past the last: a repeat, unused)
    const float2 g = w.live ? gnext : make_float2(-INFINITY, -INFINITY);
    gnext = load_g(tn);
    float sx[kUnits][8];
#pragma unroll
    for (int u = 0; u < kUnits; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) sx[u][j] = clive[u] ? __uint_as_float(snext[u][j >> 2][j & 3]) : -INFINITY;
    load_sc(tn, snext);
    // the full pass's tile recurrence, per column n
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
    wave_lds_order();  // the previous tile's chunk reads are issued
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      // P and P^ of this unit's chunk, with its column's offset and group maximum
      const int col = cr + 4 * u;
      const float nmc = __shfl(nm, col, 64);
      const float gx = __shfl(g.x, col, 64), gy = __shfl(g.y, col, 64);
      const PQuant pq = pquant_setup<LV>(__builtin_amdgcn_exp2f(p_arg<false>(ch ? gy : gx, a.c1, nmc)));
      float pc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pc[j] = __builtin_amdgcn_exp2f(p_arg<false>(sx[u][j], a.c1, nmc));
      pquant8<LV>(pc, pq);
      *reinterpret_cast<bf16x8*>(pslots + (lane + 64 * u) * 16) = pack8<true>(pc);
    }
    wave_lds_order();
    // the PV B operand of lane (n, half), chunk c: column n's chunk (zero past the compact
    // columns), and the row sum over it in the full pass's order
    bf16x8 pb[8];
    float rowsum = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const bf16x8 x = *reinterpret_cast<const bf16x8*>(pslots + (16 * (n & (kCols - 1)) + 8 * half + c) * 16);
      pb[c] = n < kCols ? x : bf16x8{};
      uint32_t wv[4];
      __builtin_memcpy(wv, &pb[c], 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x2_t pr;
        __builtin_memcpy(&pr, &wv[i], 4);
        rowsum = __builtin_amdgcn_fdot2_f32_bf16(pr, ones2, rowsum, false);
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      if ((c & 3) == 0) {
        // stage half tile c / 4 (the previous one's fragment reads were issued before), then
        // load the next one
        wave_lds_order();
        store_rows<kPacked>(vr, lane, region);
        if ((t + 1) * kKeyTile > a.Lk) zero_tail_rows(a.Lk, t, c >> 2, lane, region);
        wave_lds_order();
        load_rows<kPacked>(vsrc, voff, a.Lk, t + (c >> 2), (c >> 2) ^ 1, vr, c == 0 || t + 1 < w.t_hi);
      }
      bf16x8 va[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) va[mb] = vt_fragment(region, lane, mb, c & 3);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) acc[mb] = mfma32(va[mb], pb[c], acc[mb]);
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

// ---------------------------------------------------------------------------------------
// One-pass decode for at most kCols = 4 or 8 live columns (the compact values pass's cases)
// and one key tile per split: each wave computes its split's scores (kept in registers, in
// the compact layout), publishes its split maxima, finds the running maximum before its
// split from the maxima that the earlier splits of its row block published (a look-back
// across waves), then runs the compact values pass on those scores.  K and V are read in
// one launch and S never goes to memory; the arithmetic is the two passes', so the outputs
// are the same bits.
//
// The published maxima live in a file-scope array of 64-bit words (value bits, and the
// call's epoch in the high half: a word from another call never matches), slot
// (item nsplit + split) kCols + column.  Waiting is bounded: after spin_limit rounds a wave
// computes the maxima it still lacks itself, from K (spin_limit < 0: always), so a split
// whose predecessors never run still finishes, with the same result.
constexpr int kDecFlagSlots = 1 << 19;
constexpr int kFusedMaxTps = 1;  // key tiles per split
// The one pass is taken up to 64 key tiles (8192 keys): measured against the two passes
// (Qwen3-8B heads, one tile per split), 8k 16.7 against 19.0 us (bf16) and 17.9 against
// 19.9 (packed); 16k and 32k within +-0.5 us either way.
constexpr int kFusedMaxTiles = 64;
__device__ unsigned long long dec_flags[kDecFlagSlots];

__device__ __forceinline__ void flag_publish(int64_t slot, uint32_t epoch, float v) {
  const unsigned long long word = (static_cast<unsigned long long>(epoch) << 32) | __float_as_uint(v);
  __hip_atomic_store(&dec_flags[slot], word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long flag_read(int64_t slot) {
  return __hip_atomic_load(&dec_flags[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The maximum of split w's scores (key tiles [t_lo, t_hi)) in lane (n, half) (column n, keys
// 64 half + 0..63 of each tile), with the scores pass's loads, staging, MFMA chains and
// masking: the look-back's own computation of a split maximum that did not arrive.
template <bool kPacked>
__device__ __forceinline__ float split_scores_max(const DecodeArgs& a, const DecWave& w, const bf16x8 (&qf)[8],
                                                  const RowSrc& ksrc, const RowOffs<kPacked>& koff, uint8_t* region,
                                                  int lane) {
  const int n = lane & 31, half = lane >> 5;
  const int off = a.Lk - a.Lq;
  const int krow0 = 64 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  float smax = -INFINITY;
  RowsRaw<kPacked> raw;
  load_rows<kPacked>(ksrc, koff, a.Lk, w.t_lo, 0, raw);
  for (int t = w.t_lo; t < w.t_hi; ++t) {
    const int key0 = t * kKeyTile;
    floatx16 s[4];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      wave_lds_order();
      store_rows<kPacked>(raw, lane, region);
      wave_lds_order();
      load_rows<kPacked>(ksrc, koff, a.Lk, t + st, st ^ 1, raw, st == 0 || t + 1 < w.t_hi);
#pragma unroll
      for (int kb = 2 * st; kb < 2 * st + 2; ++kb) {
        const int pi = krow0 + 16 * kb;
        const uint8_t* kp = region + (((pi & 31) + 32 * (pi >> 6)) * kRowUnits + half) * 16;
        s[kb] = floatx16{};
#pragma unroll
        for (int c = 0; c < 8; ++c) s[kb] = mfma32(lds_read_at(kp, 32 * c), qf[c], s[kb]);
      }
    }
    if (key0 + kKeyTile > a.Lk || (a.causal && key0 + kKeyTile - 1 > w.pmin + off)) {
      const int lim = a.causal ? min(a.Lk - 1, w.pos + off) : a.Lk - 1;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (key0 + 64 * half + 16 * kb + i > lim) s[kb][i] = -INFINITY;
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) smax = fmaxf(smax, s[kb][i]);
  }
  return smax;
}

// Running maximum before split w.j (c1-scaled, in lane n for column n) from the published
// split maxima of splits 0 .. w.j - 1 of the row block: lane l waits for split j0 + l.
template <bool kPacked, int kCols>
__device__ __forceinline__ float lookback_max(const DecodeArgs& a, const DecWave& w, const bf16x8 (&qf)[8],
                                              const RowSrc& ksrc, const RowOffs<kPacked>& koff, uint8_t* region,
                                              int wave_id, int lane, uint32_t epoch, int spin_limit) {
  const int n = lane & 31;
  const int nrows = rmax_rows<kCols>(a, w);
  const int64_t slot0 = static_cast<int64_t>(w.item) * a.nsplit * kCols;
  float mr[kCols];
#pragma unroll
  for (int r = 0; r < kCols; ++r) mr[r] = -INFINITY;
  for (int j0 = 0; j0 < w.j; j0 += 64) {
    const int jj = j0 + lane;
    const bool in = jj < w.j;
    float x[kCols];
    bool ok[kCols];
#pragma unroll
    for (int r = 0; r < kCols; ++r) {
      x[r] = -INFINITY;
      ok[r] = !in || r >= nrows;
    }
    if (spin_limit >= 0) {
      for (int it = 0;; ++it) {
        bool all = true;
#pragma unroll
        for (int r = 0; r < kCols; ++r) {
          if (!ok[r]) {
            const unsigned long long v = flag_read(slot0 + static_cast<int64_t>(jj) * kCols + r);
            if (static_cast<uint32_t>(v >> 32) == epoch) {
              x[r] = __uint_as_float(static_cast<uint32_t>(v));
              ok[r] = true;
            }
          }
          all = all && ok[r];
        }
        if (__ballot(!all) == 0 || it >= spin_limit) break;
        __builtin_amdgcn_s_sleep(1);
      }
    }
    bool all = true;
#pragma unroll
    for (int r = 0; r < kCols; ++r) all = all && ok[r];
    // splits whose maxima did not arrive: computed here, from K (wave-uniform loop)
    uint64_t pending = __ballot(!all);
    while (pending != 0) {
      const int l = __builtin_ctzll(pending);
      pending &= pending - 1;
      const DecWave wp = dec_wave(a, wave_id - w.j + j0 + l, n);
      const float mp = halves_max(split_scores_max<kPacked>(a, wp, qf, ksrc, koff, region, lane));
#pragma unroll
      for (int r = 0; r < kCols; ++r) {
        const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mp), r));
        if (lane == l && r < nrows) x[r] = v;
      }
    }
#pragma unroll
    for (int r = 0; r < kCols; ++r) mr[r] = fmaxf(mr[r], in && r < nrows ? x[r] : -INFINITY);
  }
  float m_run = -INFINITY;
#pragma unroll
  for (int r = 0; r < kCols; ++r) {
    if (r < nrows) {
      const float m = wave_max_f32(mr[r]);
      if (n == r) m_run = m * a.c1;
    }
  }
  return m_run;
}

template <int LV, bool kPacked, int kCols>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_fused_kernel(DecodeArgs a, uint32_t epoch, int spin_limit) {
  static_assert(kCols == 4 || kCols == 8, "compact columns");
  constexpr int kUnits = kCols / 4;
  constexpr int kRegion = kStageBytes + kCols * 256;  // K or V half tile (and the scores' transfer), P^ chunks
  __shared__ __attribute__((aligned(128))) uint8_t lds[kDecWaves * kRegion];
  const int lane = threadIdx.x & 63;
  const int n = lane & 31;
  const int half = lane >> 5;
  const int wave_id = dec_wave_id();
  if (wave_id >= a.B * a.Hkv * a.n_rb * a.nsplit) return;
  const DecWave w = dec_wave(a, wave_id, n);
  uint8_t* const region = lds + (threadIdx.x >> 6) * kRegion;
  uint8_t* const pslots = region + kStageBytes;
  const RowSrc ksrc = k_source<kPacked>(a, w);
  const int64_t slot = (static_cast<int64_t>(w.item) * a.nsplit + w.j) * kCols + n;
  const bool publisher = w.live && half == 0 && n < kCols;

  if (w.t_lo >= w.t_hi) {
    // an empty split: its maxima are -inf, and its zero partial weighs 0 in the combine
    if (publisher) flag_publish(slot, epoch, -INFINITY);
    if (w.live) {
      float* po = a.part_o + (static_cast<int64_t>(w.j) * a.rows_total + w.row) * kDim;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<float4*>(po + 32 * mb + 8 * j + 4 * half) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (half == 0) {
        float* lm = a.part_lm + (static_cast<int64_t>(w.j) * a.rows_total + w.row) * 2;
        lm[0] = 0.0f;
        lm[1] = -INFINITY;
      }
    }
    return;
  }

  bf16x8 qf[8];
  {
    // (columns without a row read row 0 of their head: their scores are not used)
    const uint16_t* qp = a.q + w.b * a.q_sb + w.hq * a.q_sh + static_cast<int64_t>(w.live ? w.pos : 0) * a.q_sl + 8 * half;
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = *reinterpret_cast<const bf16x8*>(qp + 16 * c);
  }
  // the split's one tile: S, masked, the lane maxima g (x: keys 0-63, y: 64-127 of column n)
  const int t = w.t_lo;
  const int key0 = t * kKeyTile;
  floatx16 s[4];
  {
    const RowOffs<kPacked> koff = row_offsets<kPacked>(ksrc, lane);
    const int krow0 = 64 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
    RowsRaw<kPacked> raw;
    load_rows<kPacked>(ksrc, koff, a.Lk, t, 0, raw);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      wave_lds_order();
      store_rows<kPacked>(raw, lane, region);
      wave_lds_order();
      if (st == 0) load_rows<kPacked>(ksrc, koff, a.Lk, t, 1, raw);
#pragma unroll
      for (int kb = 2 * st; kb < 2 * st + 2; ++kb) {
        const int pi = krow0 + 16 * kb;
        const uint8_t* kp = region + (((pi & 31) + 32 * (pi >> 6)) * kRowUnits + half) * 16;
        s[kb] = floatx16{};
#pragma unroll
        for (int c = 0; c < 8; ++c) s[kb] = mfma32(lds_read_at(kp, 32 * c), qf[c], s[kb]);
      }
    }
  }
  const int off = a.Lk - a.Lq;
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
  float2 g;
  {
    const uint32_t u = __float_as_uint(mx);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    g = make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  // the live columns' scores to the compact layout (unit: column cr + 4 u, key half ch,
  // chunk cc) through the staged half tile's LDS, whose fragment reads were issued before
  const int cr = lane >> 4, ch = (lane >> 3) & 1, cc = lane & 7;
  float sx[kUnits][8];
  {
    float* sb = reinterpret_cast<float*>(region);
    wave_lds_order();
    if (n < kCols) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          *reinterpret_cast<float4*>(sb + n * kKeyTile + 64 * half + 16 * kb + 4 * u) =
              make_float4(s[kb][4 * u], s[kb][4 * u + 1], s[kb][4 * u + 2], s[kb][4 * u + 3]);
    }
    wave_lds_order();
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      const bool live = dec_wave(a, wave_id, cr + 4 * u).live;
      const float* sp = sb + (cr + 4 * u) * kKeyTile + 64 * ch + 8 * cc;
      const float4 x0 = *reinterpret_cast<const float4*>(sp), x1 = *reinterpret_cast<const float4*>(sp + 4);
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) sx[u][j] = live ? xs[j] : -INFINITY;
    }
  }
  if (publisher) flag_publish(slot, epoch, fmaxf(g.x, g.y));
  float m_run;
  {
    const RowOffs<kPacked> koff = row_offsets<kPacked>(ksrc, lane);
    m_run = lookback_max<kPacked, kCols>(a, w, qf, ksrc, koff, region, wave_id, lane, epoch, spin_limit);
  }
  // (V loads after the look-back: its fallback needs the registers a V half tile would hold)
  const RowSrc vsrc = v_source<kPacked>(a, w);
  const RowOffs<kPacked> voff = row_offsets<kPacked>(vsrc, lane);
  RowsRaw<kPacked> vr;
  load_rows<kPacked>(vsrc, voff, a.Lk, t, 0, vr);

  // the compact values pass on the tile
  if (!w.live) g = make_float2(-INFINITY, -INFINITY);
  const float m_new = fmaxf(m_run, fmaxf(g.x, g.y) * a.c1);
  const float m_use = m_new == -INFINITY ? 0.0f : m_new;
  const float nm = -m_use;
  // the two passes' first-tile rescale of the (zero) accumulator and l, kept so that a NaN
  // maximum propagates the same way
  const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
  m_run = m_new;
  floatx16 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = floatx16{};
  float l_run = 0.0f;
  if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mb][i] *= alpha;
    l_run *= alpha;
  }
  wave_lds_order();
#pragma unroll
  for (int u = 0; u < kUnits; ++u) {
    const int col = cr + 4 * u;
    const float nmc = __shfl(nm, col, 64);
    const float gx = __shfl(g.x, col, 64), gy = __shfl(g.y, col, 64);
    const PQuant pq = pquant_setup<LV>(__builtin_amdgcn_exp2f(p_arg<false>(ch ? gy : gx, a.c1, nmc)));
    float pc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pc[j] = __builtin_amdgcn_exp2f(p_arg<false>(sx[u][j], a.c1, nmc));
    pquant8<LV>(pc, pq);
    *reinterpret_cast<bf16x8*>(pslots + (lane + 64 * u) * 16) = pack8<true>(pc);
  }
  wave_lds_order();
  bf16x2_t ones2;
  {
    const uint32_t one2 = 0x3F803F80u;
    __builtin_memcpy(&ones2, &one2, 4);
  }
  bf16x8 pb[8];
  float rowsum = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(pslots + (16 * (n & (kCols - 1)) + 8 * half + c) * 16);
    pb[c] = n < kCols ? x : bf16x8{};
    uint32_t wv[4];
    __builtin_memcpy(wv, &pb[c], 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x2_t pr;
      __builtin_memcpy(&pr, &wv[i], 4);
      rowsum = __builtin_amdgcn_fdot2_f32_bf16(pr, ones2, rowsum, false);
    }
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if ((c & 3) == 0) {
      wave_lds_order();
      store_rows<kPacked>(vr, lane, region);
      if ((t + 1) * kKeyTile > a.Lk) zero_tail_rows(a.Lk, t, c >> 2, lane, region);
      wave_lds_order();
      if (c == 0) load_rows<kPacked>(vsrc, voff, a.Lk, t, 1, vr);
    }
    bf16x8 va[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) va[mb] = vt_fragment(region, lane, mb, c & 3);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[mb] = mfma32(va[mb], pb[c], acc[mb]);
  }
  l_run += halves_sum(rowsum);

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
  if (quant_p && same && a.G * a.Lq <= 4) {
    if (packed) hipLaunchKernelGGL((dec_values_compact_kernel<LV, true, 4>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((dec_values_compact_kernel<LV, false, 4>), grid, dim3(256), 0, st, a);
    return;
  }
  if (quant_p && same && a.G * a.Lq <= 8) {
    if (packed) hipLaunchKernelGGL((dec_values_compact_kernel<LV, true, 8>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((dec_values_compact_kernel<LV, false, 8>), grid, dim3(256), 0, st, a);
    return;
  }
  if (quant_p && same) launch_values<LV, true, true>(a, packed, grid, st);
  else if (quant_p) launch_values<LV, true, false>(a, packed, grid, st);
  else launch_values<123, false, false>(a, packed, grid, st);
}

}  // namespace

bool decode_fused_fits(const DecodeArgs& a, int quant_p, int norm_same) {
  return quant_p && norm_same && a.G * a.Lq <= 8 && a.tps <= kFusedMaxTps && a.ntiles <= kFusedMaxTiles &&
         static_cast<int64_t>(a.B) * a.Hkv * a.n_rb * a.nsplit * (a.G * a.Lq <= 4 ? 4 : 8) <= kDecFlagSlots;
}

void launch_decode_fused(const DecodeArgs& a, int packed, int p_levels, uint32_t epoch, int spin_limit, hipStream_t st) {
  const int64_t waves = static_cast<int64_t>(a.B) * a.Hkv * a.n_rb * a.nsplit;
  const dim3 grid(static_cast<unsigned>((waves + kDecWaves - 1) / kDecWaves));
  const bool four = a.G * a.Lq <= 4;
  auto go = [&](auto lv) {
    constexpr int LV = decltype(lv)::value;
    if (packed) {
      if (four) hipLaunchKernelGGL((dec_fused_kernel<LV, true, 4>), grid, dim3(256), 0, st, a, epoch, spin_limit);
      else hipLaunchKernelGGL((dec_fused_kernel<LV, true, 8>), grid, dim3(256), 0, st, a, epoch, spin_limit);
    } else {
      if (four) hipLaunchKernelGGL((dec_fused_kernel<LV, false, 4>), grid, dim3(256), 0, st, a, epoch, spin_limit);
      else hipLaunchKernelGGL((dec_fused_kernel<LV, false, 8>), grid, dim3(256), 0, st, a, epoch, spin_limit);
    }
  };
  if (p_levels == 12) go(std::integral_constant<int, 12>{});
  else if (p_levels == 13) go(std::integral_constant<int, 13>{});
  else go(std::integral_constant<int, 123>{});
}

void launch_decode(const DecodeArgs& a, int packed, int quant_p, int p_levels, int norm_same, hipStream_t st) {
  const int64_t waves = static_cast<int64_t>(a.B) * a.Hkv * a.n_rb * a.nsplit;
  const dim3 grid(static_cast<unsigned>((waves + kDecWaves - 1) / kDecWaves));
  // packed rows: the scores pass without LDS (test hook: FAQ_DEC_SCORES=lds stages them)
  const char* sc_env = std::getenv("FAQ_DEC_SCORES");
  const bool staged = sc_env && std::strcmp(sc_env, "lds") == 0;
  if (packed && !staged) hipLaunchKernelGGL(dec_scores_packed_direct_kernel, grid, dim3(256), 0, st, a);
  else if (packed) hipLaunchKernelGGL((dec_scores_kernel<true>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((dec_scores_kernel<false>), grid, dim3(256), 0, st, a);
  const int lv = quant_p ? p_levels : 123;
  if (lv == 12) launch_values_lv<12>(a, packed, quant_p, norm_same, grid, st);
  else if (lv == 13) launch_values_lv<13>(a, packed, quant_p, norm_same, grid, st);
  else launch_values_lv<123>(a, packed, quant_p, norm_same, grid, st);
}

}  // namespace faq
