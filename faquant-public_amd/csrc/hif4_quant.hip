// HBM-bound kernels of the HiF4 attention path on gfx950:
//   qdq_rows_kernel        fake_quantize_hif4 / fit_hif4_compact_parameters / packed encode
//                          (reference: src/faquant/hif4.py:143-271, 346-390)
//   hadamard_rows_kernel   hadamard_transform / chunked_block_hadamard_transform
//                          (reference: src/faquant/rotation.py:14-29, 117-135)
//   operand_prep_kernel    post-RoPE Q/K excursion (key offset, Smooth-QK, Hadamard, one
//                          cast) fused with the operand QDQ, writing the attention operand
//                          (reference: src/faquant/qwen3.py:97-136,
//                          src/faquant/simulated_flash_attention.py:588-619,
//                          src/faquant/wan22_attention.py:186-192, 219-221)
//   operand_prep_vt_kernel V QDQ written transposed ([d][key], keys padded with zeros to
//                          a multiple of 128) for the attention kernel's PV operand.
//   act_qdq_rows_kernel    the quantized Linear's input prologue: input scale, block
//                          Hadamard up to 512, HiF4 QDQ (reference: quantization.py:199-276)
//   act_row_kernel         the whole Linear activation path, one workgroup per row: HiSQ
//                          rotation, clamp, companding, block or generalized Hadamard, QDQ
//                          (reference: quantization.py:199-276, hisq_rotation.py:50-71,
//                          rotation.py:53-69, 117-135)
//
// Layout: one lane owns 8 consecutive values of a row (one 16-byte bf16 vector); a
// 64-value HiF4 group spans 8 adjacent lanes and its maxima reduce with xor shuffles
// inside those 8 lanes.  A Hadamard butterfly of stride 8*m pairs lane l with lane l^m.
#include "hif4_device.h"

namespace faq {

template <typename T>
struct Io;

template <>
struct Io<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
  static __device__ __forceinline__ float round(float v) { return v; }
  static __device__ __forceinline__ void load8(const float* p, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store8(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
  // 8 values as loaded, unpacked later (a load kept in flight across other work)
  struct Raw {
    float4 a, b;
  };
  static __device__ __forceinline__ Raw load_raw8(const float* p) {
    return Raw{*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4)};
  }
  static __device__ __forceinline__ void unpack8(const Raw& w, float* v) {
    v[0] = w.a.x; v[1] = w.a.y; v[2] = w.a.z; v[3] = w.a.w;
    v[4] = w.b.x; v[5] = w.b.y; v[6] = w.b.z; v[7] = w.b.w;
  }
};

template <>
struct Io<__hip_bfloat16> {
  using T = __hip_bfloat16;
  static __device__ __forceinline__ float load(const T* p) {
    return bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p));
  }
  static __device__ __forceinline__ void store(T* p, float v) {
    *reinterpret_cast<uint16_t*>(p) = f32_to_bf16_bits_rne(v);
  }
  static __device__ __forceinline__ float round(float v) { return bf16_round_hw(v); }
  static __device__ __forceinline__ void load8(const T* p, float* v) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
  static __device__ __forceinline__ void store8(T* p, const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack2_bf16_hw(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  using Raw = uint4;
  static __device__ __forceinline__ Raw load_raw8(const T* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ void unpack8(const Raw& a, float* v) {
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
};

// fp32 -> fp16, round to nearest even, of a value already rounded to fp32.  The empty asm
// keeps the compiler from fusing the multiply or add that produced v into the conversion as
// one mixed-precision fma (v_fma_mixlo_f16 a, b, 0): that rounds the exact a * b once to fp16
// instead of rounding to fp32 first, as torch does, and its +0 addend turns a -0 product
// into +0.
__device__ __forceinline__ __half f16_rn(float v) {
  asm volatile("" : "+v"(v));
  return __float2half_rn(v);
}

template <>
struct Io<__half> {
  using T = __half;
  static __device__ __forceinline__ float load(const T* p) { return __half2float(*p); }
  static __device__ __forceinline__ void store(T* p, float v) { *p = f16_rn(v); }
  static __device__ __forceinline__ float round(float v) { return __half2float(f16_rn(v)); }
  static __device__ __forceinline__ void load8(const T* p, float* v) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __half2float(p[i]);
  }
  static __device__ __forceinline__ void store8(T* p, const float* v) {
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = f16_rn(v[i]);
  }
  using Raw = uint4;
  static __device__ __forceinline__ Raw load_raw8(const T* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ void unpack8(const Raw& a, float* v) {
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] & 0xFFFFu)));
      v[2 * i + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] >> 16)));
    }
  }
};

// Value of lane l ^ M, as VALU lane moves instead of LDS permutes: DPP quad_perm for
// M = 1, 2; row_half_mirror (l ^ 7) then quad_perm [3,2,1,0] (l ^ 3) for M = 4;
// row_mirror (l ^ 15) then row_half_mirror for M = 8; v_permlane16_swap /
// v_permlane32_swap of a register with itself for M = 16, 32 (results 0 / 1 are the
// lower / upper lane's copy).
template <int M>
__device__ __forceinline__ int lane_xor(int u) {
  if constexpr (M == 1) {
    return __builtin_amdgcn_mov_dpp(u, 0xB1, 0xF, 0xF, false);
  } else if constexpr (M == 2) {
    return __builtin_amdgcn_mov_dpp(u, 0x4E, 0xF, 0xF, false);
  } else if constexpr (M == 4) {
    const int h = __builtin_amdgcn_mov_dpp(u, 0x141, 0xF, 0xF, false);
    return __builtin_amdgcn_mov_dpp(h, 0x1B, 0xF, 0xF, false);
  } else if constexpr (M == 8) {
    const int h = __builtin_amdgcn_mov_dpp(u, 0x140, 0xF, 0xF, false);
    return __builtin_amdgcn_mov_dpp(h, 0x141, 0xF, 0xF, false);
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return (threadIdx.x & 16) ? static_cast<int>(r[0]) : static_cast<int>(r[1]);
  } else {
    static_assert(M == 32, "lane_xor: M must be a power of two <= 32");
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return (threadIdx.x & 32) ? static_cast<int>(r[0]) : static_cast<int>(r[1]);
  }
}

template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  return __int_as_float(lane_xor<M>(__float_as_int(v)));
}

template <int M>
struct LaneMask {
  static constexpr int value = M;
};

// Block maximum over the 8 lanes holding one 64-value group of non-negative values
// (integer max of the bit patterns: no float canonicalization of the lane moves).
__device__ __forceinline__ float group_max8(float v) {
  int u = __float_as_int(v);
  u = max(u, lane_xor<1>(u));
  u = max(u, lane_xor<2>(u));
  u = max(u, lane_xor<4>(u));
  return __int_as_float(u);
}

// HiF4 QDQ of the 8 values a lane owns (signed, |x| based).  Lanes 8j..8j+7 must hold
// one 64-value group in order.  `nan_in_group` reproduces the reference's NaN
// propagation: a NaN anywhere in a block makes the whole block NaN.
template <int LV>
__device__ __forceinline__ void qdq8(float* v, float* s_out = nullptr, float* rec_out = nullptr,
                                     int* ka_out = nullptr, int* kb_out = nullptr, uint32_t* codes = nullptr) {
  float m3a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  float m3b = fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7])));
  int nan = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) nan |= v[i] != v[i];
  nan = lane_xor<1>(nan) | nan;
  nan = lane_xor<2>(nan) | nan;
  nan = lane_xor<4>(nan) | nan;
  const float m1 = group_max8(fmaxf(m3a, m3b));
  float s, rec;
  hif4_scale<LV>(m1, s, rec);
  int ka, kb;
  hif4_micro<LV>(m3a, m3b, rec, ka, kb);
  float qa, da, qb, db;
  hif4_group_mults(s, rec, ka, qa, da);
  hif4_group_mults(s, rec, kb, qb, db);
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float qm4 = i < 4 ? qa : qb;
    const float dq = i < 4 ? da : db;
    const float a = fabsf(v[i]);
    if (codes) {
      const uint32_t c = hif4_code(a, qm4);
      packed |= ((v[i] < 0.0f ? 8u : 0u) | c) << (4 * i);
    }
    const float y = hif4_element(a, qm4, dq);
    v[i] = nan ? __builtin_nanf("") : (v[i] < 0.0f ? -y : y);
  }
  if (s_out) *s_out = s;
  if (rec_out) *rec_out = rec;
  if (ka_out) *ka_out = ka;
  if (kb_out) *kb_out = kb;
  if (codes) *codes = packed;
}

// ------------------------------------------------------------------ qdq_rows

struct QdqRowsArgs {
  const void* x;
  void* y;
  int64_t rows;
  int64_t cols;
  int vec;  // 1: rows are 16-byte aligned and cols % 8 == 0
  float* scale;      // [rows, groups] or null
  float* rec;        // [rows, groups] or null
  int8_t* lv2;       // [rows, groups, 8] or null
  int8_t* lv3;       // [rows, groups, 16] or null
  uint8_t* codes;    // [rows, cols / 2] or null (cols % 64 == 0)
  uint8_t* scale_byte;   // [rows, groups] or null
  uint8_t* lv2_bits;     // [rows, groups] or null
  uint16_t* lv3_bits;    // [rows, groups] or null
};

template <typename T, int LV>
__global__ __launch_bounds__(256) void qdq_rows_kernel(QdqRowsArgs a) {
  const int64_t groups = (a.cols + 63) / 64;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t unit = tid >> 3;  // one (row, group)
  const int part = threadIdx.x & 7;
  // Lanes past the end still take part in the shuffles (with zeros) but store nothing.
  const bool live = unit < a.rows * groups;
  const int64_t row = live ? unit / groups : 0;
  const int64_t g = live ? unit % groups : 0;
  const int64_t c0 = g * 64 + part * 8;
  const T* x = static_cast<const T*>(a.x) + row * a.cols;
  T* y = static_cast<T*>(a.y) + row * a.cols;
  float v[8];
  if (live && a.vec && c0 < a.cols) {
    Io<T>::load8(x + c0, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (live && c0 + i < a.cols) ? Io<T>::load(x + c0 + i) : 0.0f;
  }
  float s, rec;
  int ka, kb;
  uint32_t codes = 0;
  qdq8<LV>(v, &s, &rec, &ka, &kb, a.codes ? &codes : nullptr);
  if (!live) return;
  if (a.vec && c0 < a.cols) {
    Io<T>::store8(y + c0, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (c0 + i < a.cols) Io<T>::store(y + c0 + i, v[i]);
  }
  const int64_t gi = row * groups + g;
  // k = lv2 + lv3 per 4-group.  For levels 123, lv2 = 1 forces the larger 4-group to
  // lv3 = 1 (its m3 rec is the 8-group's m2 rec >= 4), so lv2 = [ka == 2 or kb == 2].
  const int e2 = LV == 123 ? (ka == 2 || kb == 2) : (LV == 12 ? ka : 0);
  const int e3a = ka - e2;
  const int e3b = kb - e2;
  if (a.lv2) a.lv2[gi * 8 + part] = static_cast<int8_t>(e2);
  if (a.lv3) {
    a.lv3[gi * 16 + 2 * part] = static_cast<int8_t>(e3a);
    a.lv3[gi * 16 + 2 * part + 1] = static_cast<int8_t>(e3b);
  }
  if (a.scale && part == 0) a.scale[gi] = s;
  if (a.rec && part == 0) a.rec[gi] = rec;
  if (a.codes) *reinterpret_cast<uint32_t*>(a.codes + row * (a.cols / 2) + c0 / 2) = codes;
  if (a.scale_byte || a.lv2_bits || a.lv3_bits) {
    // The 8 lanes of a group share one byte of lv2 bits and 16 lv3 bits.
    uint32_t b2 = static_cast<uint32_t>(e2) << part;
    uint32_t b3 = (static_cast<uint32_t>(e3a) | (static_cast<uint32_t>(e3b) << 1)) << (2 * part);
    // (reductions run on live lanes only; a group's 8 lanes are all live or all dead)
    b2 |= static_cast<uint32_t>(lane_xor<1>(static_cast<int>(b2)));
    b2 |= static_cast<uint32_t>(lane_xor<2>(static_cast<int>(b2)));
    b2 |= static_cast<uint32_t>(lane_xor<4>(static_cast<int>(b2)));
    b3 |= static_cast<uint32_t>(lane_xor<1>(static_cast<int>(b3)));
    b3 |= static_cast<uint32_t>(lane_xor<2>(static_cast<int>(b3)));
    b3 |= static_cast<uint32_t>(lane_xor<4>(static_cast<int>(b3)));
    if (part == 0) {
      if (a.lv2_bits) a.lv2_bits[gi] = static_cast<uint8_t>(b2);
      if (a.lv3_bits) a.lv3_bits[gi] = static_cast<uint16_t>(b3);
      if (a.scale_byte) {
        const uint32_t b = __float_as_uint(s);
        const int e = static_cast<int>(b >> 23) - 127;
        a.scale_byte[gi] = static_cast<uint8_t>(((e + 48) << 2) | ((b >> 21) & 3u));
      }
    }
  }
}


// ------------------------------------------------------------------ packed decode

struct UnpackArgs {
  const uint8_t* codes;        // [rows, cols / 2]: value 2i in the low nibble of byte i
  const uint8_t* scale_byte;   // [rows, groups]: ((e + 48) << 2) | m, scale 2^e (1 + m/4)
  const uint8_t* lv2_bits;     // [rows, groups]: bit j = level-2 exponent of 8-group j
  const uint16_t* lv3_bits;    // [rows, groups]: bit j = level-3 exponent of 4-group j
  void* y;                     // [rows, cols]
  int64_t rows;
  int64_t cols;                // multiple of 64
};

// Values of the packed HiF4 storage view (hif4.py:67-79 content): a code c (bit 3 sign,
// bits 0-2 magnitude) in 4-group j of 8-group i is +-(c & 7)/4 * s * 2^(lv2_i + lv3_j), exact
// in fp32 as (c & 7)(4 + m) 2^(e + k - 4).  One lane per 8 values (one 8-group).
template <typename T>
__global__ __launch_bounds__(256) void unpack_rows_kernel(UnpackArgs a) {
  const int64_t groups = a.cols / 64;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= a.rows * groups * 8) return;
  const int64_t gi = tid >> 3;  // (row, group)
  const int part = static_cast<int>(tid & 7);
  const int64_t row = gi / groups;
  const int64_t c0 = (gi % groups) * 64 + part * 8;
  const uint32_t word = *reinterpret_cast<const uint32_t*>(a.codes + row * (a.cols / 2) + c0 / 2);
  const uint32_t sb = a.scale_byte[gi];
  const int e = static_cast<int>(sb >> 2) - 48;
  const int m = static_cast<int>(sb & 3u);
  const int lv2 = (a.lv2_bits[gi] >> part) & 1;
  const int lv3a = (a.lv3_bits[gi] >> (2 * part)) & 1;
  const int lv3b = (a.lv3_bits[gi] >> (2 * part + 1)) & 1;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t c = (word >> (4 * i)) & 0xFu;
    const int k = lv2 + (i < 4 ? lv3a : lv3b);
    const float mag = ldexpf(static_cast<float>((c & 7u) * static_cast<uint32_t>(4 + m)), e + k - 4);
    v[i] = (c & 8u) ? -mag : mag;
  }
  Io<T>::store8(static_cast<T*>(a.y) + row * a.cols + c0, v);
}

// ------------------------------------------------------------------ Hadamard

// In-register stages of stride 1, 2, 4 (8 consecutive values per lane), then
// cross-lane stages of stride 8 m for m = 1, 2, ... < n / 8, pairing lane l with l ^ m.
// Each stage writes (left + right, left - right) with the left half at the lower
// index, the order of rotation.py:21-28.

// Cross-lane stage of stride 8 M: (left + right, left - right) with the left half at the
// lower lane; the upper lane of a pair computes other - v as fma(-1, v, other), the lower
// one v + other as fma(1, v, other), both exactly the rounded sum or difference.
template <int M>
__device__ __forceinline__ void fwht_lane_stage(float* v) {
  const float sgn = (threadIdx.x & M) != 0 ? -1.0f : 1.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float other = lane_xor<M>(v[i]);
    v[i] = __builtin_fmaf(sgn, v[i], other);
  }
}

// All stages of a block of N values (N a power of two in [2, 512]).
template <int N>
__device__ __forceinline__ void fwht8_fixed(float* v) {
  if constexpr (N >= 2) fwht_inlane_stage<1>(v);
  if constexpr (N >= 4) fwht_inlane_stage<2>(v);
  if constexpr (N >= 8) fwht_inlane_stage<4>(v);
  if constexpr (N > 8) fwht_lane_stage<1>(v);
  if constexpr (N > 16) fwht_lane_stage<2>(v);
  if constexpr (N > 32) fwht_lane_stage<4>(v);
  if constexpr (N > 64) fwht_lane_stage<8>(v);
  if constexpr (N > 128) fwht_lane_stage<16>(v);
  if constexpr (N > 256) fwht_lane_stage<32>(v);
}

// The block sizes of the attention prologues (64, 128) run as straight-line code; other
// sizes take one uniform branch per stage (each branch joins with register copies).
__device__ __forceinline__ void fwht8_lanes(float* v, int n) {
  if (n == 64) {
    fwht8_fixed<64>(v);
    return;
  }
  if (n == 128) {
    fwht8_fixed<128>(v);
    return;
  }
  if (n >= 2) fwht_inlane_stage<1>(v);
  if (n >= 4) fwht_inlane_stage<2>(v);
  if (n >= 8) fwht_inlane_stage<4>(v);
  if (n > 8) fwht_lane_stage<1>(v);
  if (n > 16) fwht_lane_stage<2>(v);
  if (n > 32) fwht_lane_stage<4>(v);
  if (n > 64) fwht_lane_stage<8>(v);
  if (n > 128) fwht_lane_stage<16>(v);
  if (n > 256) fwht_lane_stage<32>(v);
}


struct HadamardRowsArgs {
  const void* x;
  void* y;
  int64_t rows;
  int64_t cols;   // multiple of n and of 8
  int n;          // block size, power of two in [2, 512]
  SqrtDiv div;    // division by fp32(sqrt(n))
};

// The stages of fwht8_lanes with every value rounded to T after each stage: the
// reference's butterflies on a bf16 / fp16 tensor, where each `left + right` and
// `left - right` is an fp32 add rounded to the tensor's dtype (rotation.py:21-27).
template <typename T>
__device__ __forceinline__ void fwht8_lanes_rounded(float* v, int n) {
  auto rnd = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Io<T>::round(v[i]);
  };
  if (n >= 2) { fwht_inlane_stage<1>(v); rnd(); }
  if (n >= 4) { fwht_inlane_stage<2>(v); rnd(); }
  if (n >= 8) { fwht_inlane_stage<4>(v); rnd(); }
  if (n > 8) { fwht_lane_stage<1>(v); rnd(); }
  if (n > 16) { fwht_lane_stage<2>(v); rnd(); }
  if (n > 32) { fwht_lane_stage<4>(v); rnd(); }
  if (n > 64) { fwht_lane_stage<8>(v); rnd(); }
  if (n > 128) { fwht_lane_stage<16>(v); rnd(); }
  if (n > 256) { fwht_lane_stage<32>(v); rnd(); }
}

// kStageRound: the transform in the tensor's own dtype (Tin == Tout, hadamard_transform
// on a bf16 / fp16 tensor); the division's fp32 quotient is rounded to Tout by the store,
// as torch rounds its fp32 opmath result.  Otherwise fp32 butterflies and one rounding.
template <typename Tin, typename Tout, bool kStageRound = false>
__global__ __launch_bounds__(256) void hadamard_rows_kernel(HadamardRowsArgs a) {
  const int64_t lanes_per_row = a.cols / 8;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool live = tid < a.rows * lanes_per_row;
  const int64_t row = live ? tid / lanes_per_row : 0;
  const int64_t c0 = live ? (tid % lanes_per_row) * 8 : 0;
  float v[8];
  if (live) {
    Io<Tin>::load8(static_cast<const Tin*>(a.x) + row * a.cols + c0, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  if (kStageRound) fwht8_lanes_rounded<Tout>(v, a.n);
  else fwht8_lanes(v, a.n);
  div_sqrt_n(v, a.div);
  if (live) Io<Tout>::store8(static_cast<Tout*>(a.y) + row * a.cols + c0, v);
}

// ------------------------------------------------------------------ activation prologue

struct ActQdqArgs {
  const void* x;          // [rows, cols] contiguous, dtype T
  void* y;                // [rows, cols] contiguous, dtype T
  int64_t rows;
  int64_t cols;           // multiple of 8; of 64 and of n when n > 0
  const float* col_scale; // optional per-column input scale, [cols]
  int n;                  // 0, or the block Hadamard size (power of two in [2, 512])
  SqrtDiv div;            // division by fp32(sqrt(n))
  int quant;              // 1: HiF4 QDQ
};

// The activation path of a quantized Linear (quantization.py:204-276 without the
// rotation, clamp and companding options): x * bf16(scale) in the input dtype, the
// per-block fp32 Hadamard with one cast back (rotation.py:117-135), then the HiF4 QDQ
// in the input dtype.  Lanes map like qdq_rows_kernel: 8 lanes per (row, 64-value
// group), so a Hadamard block of n <= 512 values is n / 8 consecutive lanes.
template <typename T, int LV>
__global__ __launch_bounds__(256) void act_qdq_rows_kernel(ActQdqArgs a) {
  const int64_t groups = (a.cols + 63) / 64;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t unit = tid >> 3;
  const int part = threadIdx.x & 7;
  const bool live = unit < a.rows * groups;
  const int64_t row = live ? unit / groups : 0;
  const int64_t g = live ? unit % groups : 0;
  const int64_t c0 = g * 64 + part * 8;
  const bool have = live && c0 < a.cols;
  const T* x = static_cast<const T*>(a.x) + row * a.cols;
  T* y = static_cast<T*>(a.y) + row * a.cols;
  float v[8];
  if (have) {
    Io<T>::load8(x + c0, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  if (a.col_scale && have) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Io<T>::round(v[i] * Io<T>::round(a.col_scale[c0 + i]));
  }
  if (a.n) {
    fwht8_lanes(v, a.n);
    div_sqrt_n(v, a.div);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Io<T>::round(v[i]);
  }
  if (a.quant) qdq8<LV>(v);
  if (have) Io<T>::store8(y + c0, v);
}

// ------------------------------------------------------------------ full activation path

// The whole activation path of FakeQuantLinear.forward (quantization.py:199-276) for a row
// that fits LDS: x * dtype(input_scale); the HiSQ input rotation (quantization.py:201-219:
// fp32 x times the signs, gathered by the permutation, the per-block fp32 Hadamard of
// rotation.py:117-135 when a block size is set, one cast back); the activation clamp (bounds
// in the input dtype, NaN kept); x * companding scale; the online block Hadamard with one
// cast back; the HiF4 QDQ; x / companding scale.  Every elementwise step rounds to the input
// dtype as torch does.  One workgroup per row (256 or 512 threads), the row in registers;
// LDS holds an fp32 copy for the permutation gather and the Hadamard strides above 4.
constexpr int kActMaxCols = 32768;

struct ActRowArgs {
  const void* x;            // [rows, cols] contiguous, dtype T
  void* y;                  // [rows, cols] contiguous, dtype T
  int64_t rows;
  int cols;                 // multiple of 64, at most kActMaxCols
  const float* col_scale;   // [cols] input scale, or null
  const int8_t* rot_signs;  // [cols] +1 / -1, or null: no rotation
  const int32_t* rot_perm;  // [cols] gather order (index_select), values in [0, cols)
  int rot_block;            // 0, or the rotation's block Hadamard size (power of two dividing cols)
  SqrtDiv rot_div;
  int has_min, has_max;
  float act_min, act_max;   // clamp bounds (rounded to T in the kernel)
  const float* compand;     // [cols] companding scale (values of T), or null
  const float* compand_rcp; // [cols] fp32(1 / compand) where the product form is exact, else 0; or null
  int stage_round;          // 1: the online transform in T (every butterfly stage and the 12-point
                            // mix rounded to T, as torch runs it on a T tensor)
  int n;                    // 0, or the online block Hadamard size (with gen12: cols / 12)
  int gen12;                // 1: the generalized transform of a row of 12 n values
  SqrtDiv div;              // division by fp32(sqrt(n)) (with gen12: of the row length)
  int quant;                // 1: HiF4 QDQ
};

// Layout of act_row_kernel (NT threads, R chunks per lane): lane tid holds chunk
// c = tid + NT r (r < R) of the row, the 8 values 8 c .. 8 c + 7, in registers (the
// coalesced load / store layout and the QDQ layout: 8 consecutive lanes hold one 64-value
// group).  LDS holds one fp32 copy of the row for the permutation gather and for the
// butterfly stages that cross lanes.
// Value j sits at lds_pad(j) = j + j / 8: one spare word after every 8 values, so lanes that
// write or read their 8-value chunks (8 words apart), and the first butterfly pass over LDS
// (stride 8), touch distinct banks.
__host__ __device__ constexpr size_t act_row_lds_bytes(int cols) {
  return static_cast<size_t>(cols + cols / 8) * sizeof(float);
}
__device__ __forceinline__ int lds_pad(int j) { return j + (j >> 3); }

// First value of chunk r of lane `tid`.
template <int R, int NT>
__device__ __forceinline__ int act_c0(int tid, int r) {
  return 8 * (tid + NT * r);
}

// Butterflies (left + right, left - right) of the stages of stride 1 .. S (S = 1, 2 or 4)
// on each lane's chunks (their pairs lie inside one chunk).
template <int R, int S, typename RT = float>
__device__ __forceinline__ void fwht_in_chunks(float (&v)[R][8]) {
#pragma unroll
  for (int s = 1; s <= S; s <<= 1)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (!(i & s)) {
          const float l = v[r][i], h = v[r][i + s];
          v[r][i] = Io<RT>::round(l + h);
          v[r][i + s] = Io<RT>::round(l - h);
        }
}

// Butterfly stages per pass over the LDS row (radix 16: a 1024-block's strides 8 .. 512 in
// two passes instead of three with radix 8; 12-18% less time at 4096 and 12288 features).
constexpr int kActRadix = 4;

// One pass over the LDS row of the LR stages of stride s, 2 s, .. (LR = 1 .. 4; s a
// multiple of 8, 2^LR s dividing the block): group g holds the 2^LR values j0 + m s.
template <int LR, int NT, typename RT = float>
__device__ __forceinline__ void fwht_lds_pass(float* lds, int cols, int ls, int tid) {
  constexpr int kRad = 1 << LR;
  const int s = 1 << ls;
  const int as = s + (s >> 3);  // j0 + m s sits at lds_pad(j0) + m (s + s / 8)
  for (int g = tid; g < (cols >> LR); g += NT) {
    const int a0 = lds_pad(((g >> ls) << (ls + LR)) | (g & (s - 1)));
    float w[kRad];
#pragma unroll
    for (int m = 0; m < kRad; ++m) w[m] = lds[a0 + m * as];
#pragma unroll
    for (int t = 1; t < kRad; t <<= 1)
#pragma unroll
      for (int m = 0; m < kRad; ++m)
        if (!(m & t)) {
          const float l = w[m], h = w[m + t];
          w[m] = Io<RT>::round(l + h);
          w[m + t] = Io<RT>::round(l - h);
        }
#pragma unroll
    for (int m = 0; m < kRad; ++m) lds[a0 + m * as] = w[m];
  }
}

template <int R, int NT>
__device__ __forceinline__ void row_to_lds(const float (&v)[R][8], float* lds, int cols, int tid) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c0 = act_c0<R, NT>(tid, r);
    if (c0 < cols)
#pragma unroll
      for (int i = 0; i < 8; ++i) lds[lds_pad(c0) + i] = v[r][i];
  }
}

template <int R, int NT>
__device__ __forceinline__ void row_from_lds(float (&v)[R][8], const float* lds, int cols, int tid) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c0 = act_c0<R, NT>(tid, r);
    if (c0 < cols)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[r][i] = lds[lds_pad(c0) + i];
  }
}

// Unnormalized Walsh-Hadamard transform of every b-block of the row (rotation.py:14-29
// without its division): the stages of stride 1, 2, ..., b / 2 in that order, each pair
// (i, i + s) becoming (left + right, left - right).  Strides 1, 2, 4 run in registers; larger
// strides in passes over LDS of up to kActRadix stages (s, 2 s, 4 s, ..) on the values
// j0 + m s read into registers: the same additions as one stage at a time.  Ends with the
// transformed row in v.
template <int R, int NT, typename RT = float>
__device__ __forceinline__ void fwht_row_raw(float (&v)[R][8], float* lds, int cols, int b, int tid) {
  if (b == 2) fwht_in_chunks<R, 1, RT>(v);
  else if (b == 4) fwht_in_chunks<R, 2, RT>(v);
  else fwht_in_chunks<R, 4, RT>(v);
  if (b > 8) {
    row_to_lds<R, NT>(v, lds, cols, tid);
    const int lb = __builtin_ctz(b);
    for (int ls = 3; ls < lb; ls += kActRadix) {
      __syncthreads();
      const int lr = min(kActRadix, lb - ls);
      if (lr == 4) fwht_lds_pass<4, NT, RT>(lds, cols, ls, tid);
      else if (lr == 3) fwht_lds_pass<3, NT, RT>(lds, cols, ls, tid);
      else if (lr == 2) fwht_lds_pass<2, NT, RT>(lds, cols, ls, tid);
      else fwht_lds_pass<1, NT, RT>(lds, cols, ls, tid);
    }
    __syncthreads();
    row_from_lds<R, NT>(v, lds, cols, tid);
    // the next user of the LDS row writes it again
    __syncthreads();
  }
}

// The normalized transform of every b-block: fwht_row_raw, then the division by
// fp32(sqrt(b)) (b a power of two: the fma form equals the IEEE division on its range).
template <int R, int NT, typename RT = float>
__device__ __forceinline__ void fwht_row(float (&v)[R][8], float* lds, int cols, int b, const SqrtDiv& dv, int tid) {
  fwht_row_raw<R, NT, RT>(v, lds, cols, b, tid);
#pragma unroll
  for (int r = 0; r < R; ++r) div_sqrt_n(v[r], dv);
}

// The 12-point Hadamard matrix of rotation.py:32-50, row r as a mask of its -1 entries
// (compile-time: each term of the mix is an add or a subtract).
constexpr uint16_t kH12NegMask[12] = {0xFFE, 0x474, 0x8E8, 0x1D2, 0x3A4, 0x748,
                                      0xE90, 0xD22, 0xA46, 0x48E, 0x91C, 0x23A};

// generalized_hadamard_transform (rotation.py:53-69) of a row of n = 12 b values (b a power
// of two): the reference pairs elements 2i, 2i + 1 and concatenates sums before differences,
// which is the unnormalized FWHT of every b-block; then out[r b + c] = sum_h H12[r][h]
// W[h b + c], accumulated in h order from 0 as the matmul does (each step one rounding), then
// the IEEE division by fp32(sqrt(n)) (the fma form is not exact for these divisors).  With
// RT = T (the transform on a T tensor) every stage and the mix's fp32 sum are rounded to T
// (torch's T matmul accumulates in fp32 and rounds once; the 12 terms of +-1 times T values
// sum exactly in fp32 unless their exponents span more than 16 binades).
template <int R, int NT, typename RT = float>
__device__ __forceinline__ void generalized_row(float (&v)[R][8], float* lds, int cols, int b, float d, int tid) {
  fwht_row_raw<R, NT, RT>(v, lds, cols, b, tid);
  row_to_lds<R, NT>(v, lds, cols, tid);
  __syncthreads();
  for (int c = tid; c < b; c += NT) {
    float w[12];
#pragma unroll
    for (int h = 0; h < 12; ++h) w[h] = lds[lds_pad(h * b + c)];
#pragma unroll
    for (int r = 0; r < 12; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int h = 0; h < 12; ++h) acc = __builtin_fmaf((kH12NegMask[r] >> h) & 1u ? -1.0f : 1.0f, w[h], acc);
      lds[lds_pad(r * b + c)] = Io<RT>::round(acc);
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c0 = act_c0<R, NT>(tid, r);
    if (c0 < cols)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[r][i] = lds[lds_pad(c0) + i] / d;
  }
  __syncthreads();
}

// v as a T value before the companding quotient.  v is the QDQ output (a HiF4 value: at most
// six significant bits, exact in bf16 and fp32, while fp16 can round it below its normal
// range) or an earlier step's value already rounded to T, so only fp16 rounds here.
template <typename T>
__device__ __forceinline__ float in_dtype(float v) {
  if constexpr (std::is_same<T, __half>::value) return Io<T>::round(v);
  else return v;
}

// Whether the companding quotient T(x / c) of every T value x equals T(x * fp32(1 / c)):
// bf16 scales that are normal numbers, fp16 scales below 8 in magnitude (the reference's
// scales exp(clamp(log_scale, -2.079, 2.079)) lie in (0.125, 8)).  Proved over every pair of
// 16-bit values on the CPU (tests/compand_div_check.c); fp32 always divides.
template <typename T>
__device__ __forceinline__ bool compand_product_exact(float c) {
  const uint32_t u = __float_as_uint(c) & 0x7FFFFFFFu;
  if constexpr (std::is_same<T, __hip_bfloat16>::value) return (u & 0x7F800000u) != 0;
  else if constexpr (std::is_same<T, __half>::value) return u < 0x41000000u;
  else return false;
}

// rcp[j] = fp32(1 / c[j]) where the product form of the companding quotient is exact for
// dtype T, 0 elsewhere (the activation kernel divides those columns).
template <typename T>
__global__ __launch_bounds__(256) void compand_rcp_kernel(const float* c, float* rcp, int64_t n) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j < n) rcp[j] = compand_product_exact<T>(c[j]) ? 1.0f / c[j] : 0.0f;
}

// One workgroup of NT threads per row of at most 8 NT R values.  R stays at most 4: with
// 8 chunks per lane the compiler keeps the row in scratch memory instead of registers.
// With R <= 2 the kernel asks for 8 waves per SIMD (at most 64 VGPRs): two 1024-thread or
// eight 256-thread workgroups per CU (at 67 VGPRs one fewer fits, and a 12288-feature row
// with a 1024-block rotation took 126 instead of 103 us).
// kStage: the online transform in T (ActRowArgs::stage_round), its own instance (the
// roundings cost registers) for the standalone transforms, which quantize nothing.
template <typename T, int LV, int R, int NT, bool kGen12, bool kStage = false>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(R <= 2 ? 8 : 1))) void act_row_kernel(
    ActRowArgs a) {
  extern __shared__ float act_row_lds[];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* x = static_cast<const T*>(a.x) + row * a.cols;
  T* y = static_cast<T*>(a.y) + row * a.cols;
  float v[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c0 = act_c0<R, NT>(tid, r);
    if (c0 < a.cols) {
      Io<T>::load8(x + c0, v[r]);
      if (a.col_scale) {
        float sc[8];
        Io<float>::load8(a.col_scale + c0, sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[r][i] = Io<T>::round(v[r][i] * Io<T>::round(sc[i]));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[r][i] = 0.0f;
    }
  }
  if (a.rot_signs) {
    // fp32 x times the signs in feature order (coalesced sign loads), then gathered by the
    // permutation (index_select): value j is x[perm[j]] sign[perm[j]]
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c0 = act_c0<R, NT>(tid, r);
      if (c0 < a.cols) {
        const uint2 sw = *reinterpret_cast<const uint2*>(a.rot_signs + c0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int8_t sg = static_cast<int8_t>(((i < 4 ? sw.x : sw.y) >> (8 * (i & 3))) & 0xFFu);
          act_row_lds[lds_pad(c0) + i] = v[r][i] * static_cast<float>(sg);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c0 = act_c0<R, NT>(tid, r);
      if (c0 < a.cols) {
        const int4 pa = *reinterpret_cast<const int4*>(a.rot_perm + c0);
        const int4 pb = *reinterpret_cast<const int4*>(a.rot_perm + c0 + 4);
        const int pp[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
        for (int i = 0; i < 8; ++i)  // (one unsigned min keeps any index in range; a valid permutation is)
          v[r][i] = act_row_lds[lds_pad(static_cast<int>(min(static_cast<uint32_t>(pp[i]), static_cast<uint32_t>(a.cols - 1))))];
      }
    }
    // every gather has read the row before the transform writes it
    __syncthreads();
    if (a.rot_block) fwht_row<R, NT>(v, act_row_lds, a.cols, a.rot_block, a.rot_div, tid);
  }
  // one cast back after the rotation, the clamp (bounds in T, NaN kept), the companding
  // product
  const float lo = Io<T>::round(a.act_min), hi = Io<T>::round(a.act_max);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c0 = act_c0<R, NT>(tid, r);
    float cs[8];
    if (a.compand && c0 < a.cols) Io<float>::load8(a.compand + c0, cs);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float t = v[r][i];
      if (a.rot_signs) t = Io<T>::round(t);
      if (!__builtin_isnan(t)) {
        if (a.has_min) t = fmaxf(t, lo);
        if (a.has_max) t = fminf(t, hi);
      }
      if (a.compand && c0 < a.cols) t = Io<T>::round(t * cs[i]);
      v[r][i] = t;
    }
  }
  if (a.n) {
    // the generalized form is its own instance: its 12-point mix costs registers
    using RT = typename std::conditional<kStage, T, float>::type;
    if constexpr (kGen12) generalized_row<R, NT, RT>(v, act_row_lds, a.cols, a.n, a.div.d, tid);
    else fwht_row<R, NT, RT>(v, act_row_lds, a.cols, a.n, a.div, tid);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[r][i] = Io<T>::round(v[r][i]);
  }
  // QDQ: every lane takes part (zeros past the row), as qdq8 exchanges values within its 8
  // lanes; then the companding quotient of the quantized values in T: a product with the
  // column's reciprocal (compand_rcp) where every column of the lane's chunk has one and the
  // wave agrees (a uniform branch), the IEEE division otherwise
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c0 = act_c0<R, NT>(tid, r);
    if (a.quant) qdq8<LV>(v[r]);
    if (a.compand) {
      float rc[8];
      bool ok = a.compand_rcp != nullptr;
      if (ok && c0 < a.cols) {
        Io<float>::load8(a.compand_rcp + c0, rc);
#pragma unroll
        for (int i = 0; i < 8; ++i) ok = ok && rc[i] != 0.0f;
      }
      if (__all(ok)) {
        if (c0 < a.cols)
#pragma unroll
          for (int i = 0; i < 8; ++i) v[r][i] = Io<T>::round(in_dtype<T>(v[r][i]) * rc[i]);
      } else if (c0 < a.cols) {
        float cs[8];
        Io<float>::load8(a.compand + c0, cs);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[r][i] = Io<T>::round(in_dtype<T>(v[r][i]) / cs[i]);
      }
    }
    if (c0 < a.cols) Io<T>::store8(y + c0, v[r]);
  }
}

// ------------------------------------------------------------------ operand prologue

struct OperandPrepArgs {
  const void* x;                 // [B, H, L, 128], last stride 1
  int64_t sb, sh, sl;            // element strides of x
  int B, H, L;
  const float* key_offset;       // subtracted first (keys), [H or 1, 128] or null
  int64_t off_sh;                // head stride of key_offset (0 to broadcast)
  const float* smooth;           // Smooth-QK scale, [H or 1, 128] or null
  int64_t smooth_sh;
  int smooth_divide;             // 1 for keys (k / s), 0 for queries (q * s)
  int hadamard;                  // 0, 64 or 128
  SqrtDiv div;                   // division by fp32(sqrt(hadamard))
  void* rotated;                 // optional: the rotated operand in the round dtype, [B, H, L, 128] contiguous
  void* y;                       // bf16 output [B, H, L, 128] with strides below
  int64_t yb, yh, yl;
  int quant;                     // 1: HiF4 QDQ after the cast
  // optional packed HiF4 rows (decode K/V caches; needs quant): per row 16 code words (dims
  // 8u .. 8u + 7 in word (u & 1) 8 + u / 2) and 2 meta words at row index
  // b pk_sb + h pk_sh + position; y may then be null
  uint32_t* pk_codes;
  uint32_t* pk_meta;
  int64_t pk_sb, pk_sh;
};

// Packed HiF4 form of the 8 values a lane quantized with qdq8 (a 64-value group spans the 8
// lanes part8 = 0..7, dims 8 part8 .. + 7 of the group): the code word (nibble i = 8 + the
// signed code of value i, so a value is (nibble - 8) 2^k s / 4) and the group's meta word
// (E6M2 byte ((e + 48) << 2) | m, level-2 bits << 8, level-3 bits << 16, the content of
// hif4.py:67-79), the same on all 8 lanes.  A group that became NaN gets E6M2 byte 0xFF
// (no real scale has it: the largest is 49152 = 2^15 1.5, byte 0xFE).
template <int LV>
__device__ __forceinline__ void pack_hif4_word(const float* y, uint32_t sm_codes, float s, int ka, int kb,
                                               int part8, uint32_t& word, uint32_t& meta) {
  word = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t nib = (sm_codes >> (4 * i)) & 0xFu;  // bit 3 sign, bits 0-2 code
    const uint32_t mag = nib & 7u;
    word |= ((nib & 8u) ? 8u - mag : 8u + mag) << (4 * i);
  }
  // k = lv2 + lv3 per 4-group (as in qdq_rows_kernel)
  const int e2 = LV == 123 ? (ka == 2 || kb == 2) : (LV == 12 ? ka : 0);
  uint32_t b2 = static_cast<uint32_t>(e2) << part8;
  uint32_t b3 = (static_cast<uint32_t>(ka - e2) | (static_cast<uint32_t>(kb - e2) << 1)) << (2 * part8);
  b2 |= static_cast<uint32_t>(lane_xor<1>(static_cast<int>(b2)));
  b2 |= static_cast<uint32_t>(lane_xor<2>(static_cast<int>(b2)));
  b2 |= static_cast<uint32_t>(lane_xor<4>(static_cast<int>(b2)));
  b3 |= static_cast<uint32_t>(lane_xor<1>(static_cast<int>(b3)));
  b3 |= static_cast<uint32_t>(lane_xor<2>(static_cast<int>(b3)));
  b3 |= static_cast<uint32_t>(lane_xor<4>(static_cast<int>(b3)));
  const uint32_t sbits = __float_as_uint(s);
  const int e = static_cast<int>(sbits >> 23) - 127;
  uint32_t sb = (static_cast<uint32_t>(e + 48) << 2) | ((sbits >> 21) & 3u);
  if (y[0] != y[0]) sb = 0xFFu;
  meta = sb | (b2 << 8) | (b3 << 16);
}

// One lane owns 8 of a row's 128 values; a row spans 16 lanes, and each lane takes
// kPrepRows rows 16 positions apart (a block covers 16 kPrepRows consecutive positions): the
// loads of all its rows are issued before any arithmetic, so each wave keeps kPrepRows KiB
// in flight (one row per lane is latency-bound at under half the HBM rate).  Grid: x =
// blocks of positions, y = head, z = batch (no integer division in the index math).
constexpr int kPrepRows = 2;

template <typename Tin, typename Tround, int LV>
__global__ __launch_bounds__(256) void operand_prep_kernel(OperandPrepArgs a) {
  const int h = static_cast<int>(blockIdx.y);
  const int b = static_cast<int>(blockIdx.z);
  const int lp0 = static_cast<int>(blockIdx.x) * (16 * kPrepRows) + static_cast<int>(threadIdx.x >> 4);
  const int part = threadIdx.x & 15;
  const int d0 = part * 8;
  float v[kPrepRows][8];
#pragma unroll
  for (int j = 0; j < kPrepRows; ++j) {
    const int lp = lp0 + 16 * j;
    if (lp < a.L) {
      Io<Tin>::load8(static_cast<const Tin*>(a.x) + b * a.sb + h * a.sh + static_cast<int64_t>(lp) * a.sl + d0, v[j]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[j][i] = 0.0f;
    }
  }
  float off[8], sc[8];
  if (a.key_offset) {
#pragma unroll
    for (int i = 0; i < 8; ++i) off[i] = a.key_offset[h * a.off_sh + d0 + i];
  }
  if (a.smooth) {
#pragma unroll
    for (int i = 0; i < 8; ++i) sc[i] = a.smooth[h * a.smooth_sh + d0 + i];
  }
#pragma unroll
  for (int j = 0; j < kPrepRows; ++j) {
    const int lp = lp0 + 16 * j;
    const bool live = lp < a.L;
    const int l = live ? lp : 0;
    const int64_t r = (static_cast<int64_t>(b) * a.H + h) * a.L + l;
    float* w = v[j];
    if (a.key_offset) {
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = w[i] - off[i];
    }
    if (a.smooth) {
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = a.smooth_divide ? w[i] / sc[i] : w[i] * sc[i];
    }
    if (a.hadamard) {
      fwht8_lanes(w, a.hadamard);
      div_sqrt_n(w, a.div);
    }
    // the single cast back to the operand dtype (qwen3.py:129-130)
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = Io<Tround>::round(w[i]);
    if (a.rotated && live) Io<Tround>::store8(static_cast<Tround*>(a.rotated) + r * 128 + d0, w);
    if (a.pk_codes) {
      float s;
      int ka, kb;
      uint32_t sm = 0, word, meta;
      qdq8<LV>(w, &s, nullptr, &ka, &kb, &sm);
      pack_hif4_word<LV>(w, sm, s, ka, kb, part & 7, word, meta);
      if (live) {
        const int64_t pr = b * a.pk_sb + h * a.pk_sh + l;
        a.pk_codes[pr * 16 + (part & 1) * 8 + (part >> 1)] = word;  // dims 8 part .. + 7
        if ((part & 7) == 0) a.pk_meta[pr * 2 + (part >> 3)] = meta;
      }
    } else if (a.quant) {
      qdq8<LV>(w);
    }
    if (live && a.y) {
      Io<__hip_bfloat16>::store8(
          reinterpret_cast<__hip_bfloat16*>(static_cast<uint16_t*>(a.y) + b * a.yb + h * a.yh + static_cast<int64_t>(l) * a.yl + d0), w);
    }
  }
}

struct OperandPrepVtArgs {
  const void* x;            // V [B, H, L, 128], last stride 1
  int64_t sb, sh, sl;
  int B, H, L;
  int Lpad;                 // multiple of 128, >= L
  uint16_t* vt;             // bf16 [B, H, 128, Lpad]
  int quant;
};

// 64 keys x 128 dims per block: QDQ rows in registers, transpose through LDS, store
// 16-byte runs of keys for each dim.  Keys >= L are zeros.
template <typename Tin, int LV>
__global__ __launch_bounds__(256) void operand_prep_vt_kernel(OperandPrepVtArgs a) {
  constexpr int KB = 64;
  constexpr int PITCH = KB + 8;  // uint16 elements per LDS row (16-byte aligned rows)
  __shared__ uint16_t tile[128 * PITCH];
  const int bh = blockIdx.y;
  const int b = bh / a.H;
  const int h = bh % a.H;
  const int key0 = blockIdx.x * KB;
  const int part = threadIdx.x & 15;
  const int d0 = part * 8;
  const Tin* x = static_cast<const Tin*>(a.x) + b * a.sb + h * a.sh;
#pragma unroll
  for (int it = 0; it < KB / 16; ++it) {
    const int rr = it * 16 + (threadIdx.x >> 4);
    const int key = key0 + rr;
    float v[8];
    if (key < a.L) {
      Io<Tin>::load8(x + static_cast<int64_t>(key) * a.sl + d0, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Io<Tin>::round(v[i]);
    if (a.quant) qdq8<LV>(v);
#pragma unroll
    for (int i = 0; i < 8; ++i) tile[(d0 + i) * PITCH + rr] = f32_to_bf16_bits_rne(v[i]);
  }
  __syncthreads();
  uint16_t* out = a.vt + (static_cast<int64_t>(b) * a.H + h) * 128 * a.Lpad + key0;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = threadIdx.x + 256 * it;
    const int d = c >> 3;
    const int k8 = (c & 7) * 8;
    const uint4 w = *reinterpret_cast<const uint4*>(&tile[d * PITCH + k8]);
    *reinterpret_cast<uint4*>(out + static_cast<int64_t>(d) * a.Lpad + k8) = w;
  }
}

}  // namespace faq
