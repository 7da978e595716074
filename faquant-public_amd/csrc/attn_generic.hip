// General-shape HiF4 flash attention on gfx950: the simulator's recurrence
// (src/faquant/simulated_flash_attention.py:457-909) for the shapes and operand types the
// MFMA kernel (hif4_attention.hip: head_dim 128, key tiles of 128, bf16 operands) does not
// take: any head_dim up to 256, any key tile up to 1024 keys, and fp32, bf16 or fp16 Q/K/V
// multiplied in fp32 (the reference multiplies unquantized fp32 operands as they are,
// sfa:723-724, 848-850).  Quantized operands (sfa:592-619) come in already quantized.
//
// Per query row and key tile [k0, k0 + W), in the reference's order of operations:
//   s = fp32(dot(q, k) * scale)                          sfa:723-724 (fp32 fma over d)
//   s = tanh(s / softcap) * softcap                      sfa:725-727 (softcap > 0)
//   s = s + mask  |  s = -inf outside the row's keys     sfa:730-776
//   m' = max(m, max_k s);  prev = exp(m - m') (0 for m = -inf)          sfa:778-787
//   P = exp(s - m') (0 for s = -inf)                     sfa:788-792
//   P^ = HiF4 QDQ of P in 64-key groups from the tile start, zero-padded (sfa:793-806,
//        292-338), with the reference's E6M2 scale and micro exponents (hif4_device.h)
//   l = prev l + sum(P^ or P);  acc = prev acc + P^ V   sfa:826-850
// and O = acc / max(l, FLT_MIN) where l > 0, else 0 (sfa:871-876).  exp and tanh are the
// device library's (a few ulp from torch's CPU functions), and the fp32 sums run in this
// kernel's order, so outputs agree with the simulator within fp32 rounding; P^ is the
// reference quantizer applied to this kernel's P, bit for bit.
//
// Work decomposition: a 256-thread workgroup owns 16 consecutive query positions of one
// (batch, query head).  Q rows stay in LDS as fp32; K and V pass through LDS 32 keys at a
// time (converted to fp32); the tile's scores, then its P^, sit in LDS.  Score phase:
// thread (row tid % 16, key tid / 16 and + 16 of the chunk).  Row phase: the 16 lanes
// tid / 16 = row own 8 consecutive keys of a 128-key block each (lanes 8 g .. 8 g + 7 one
// 64-key HiF4 group) and 4 consecutive dims of every 64 in PV.  Key tiles no row of the
// workgroup sees are skipped (bitwise the same as a tile of -inf scores).
#include <cfloat>

#include "attn_generic.h"
#include "hif4_device.h"

namespace faq {
namespace {

// dt: 0 fp32, 1 bf16, 2 fp16 (the C ABI's dtype codes)
__device__ __forceinline__ float gen_load(const void* p, int dt, int64_t i) {
  if (dt == 0) return static_cast<const float*>(p)[i];
  if (dt == 1) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return __half2float(static_cast<const __half*>(p)[i]);
}

// Reductions over the 16 lanes of one row (lanes 16 r .. 16 r + 15 of a wave).
__device__ __forceinline__ float row_max16(float x) {
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 16));
  return x;
}

__device__ __forceinline__ float row_sum16(float x) {
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) x += __shfl_xor(x, m, 16);
  return x;
}

// HiF4 QDQ of 8 values per lane, lanes 8 j .. 8 j + 7 holding one 64-value group in order:
// the steps of hif4.py:143-271 (group maximum, E6M2 scale, micro exponents per 8- and
// 4-value group, element codes), a NaN anywhere making the group NaN.
template <int LV>
__device__ __forceinline__ void gen_qdq8(float* v) {
  const float m3a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  const float m3b = fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7])));
  int nan = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) nan |= v[i] != v[i];
  float m1 = fmaxf(m3a, m3b);
#pragma unroll
  for (int m = 1; m <= 4; m <<= 1) {
    nan |= __shfl_xor(nan, m, 8);
    m1 = fmaxf(m1, __shfl_xor(m1, m, 8));
  }
  float s, rec;
  hif4_scale<LV>(m1, s, rec);
  int ka, kb;
  hif4_micro<LV>(m3a, m3b, rec, ka, kb);
  float qa, da, qb, db;
  hif4_group_mults(s, rec, ka, qa, da);
  hif4_group_mults(s, rec, kb, qb, db);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = hif4_element(fabsf(v[i]), i < 4 ? qa : qb, i < 4 ? da : db);
    v[i] = nan ? __builtin_nanf("") : (v[i] < 0.0f ? -y : y);
  }
}

__device__ __forceinline__ int gen_dim_pad(int D) { return (D + 3) / 4 * 4 + 4; }
__device__ __forceinline__ int gen_tile_pad(int T) { return (T + 7) / 8 * 8 + 4; }

// Rows j < nk of a key chunk into LDS as fp32 (dst[j Dp + d], d < D; rows nk .. 31 as zeros):
// the row of key j starts at element base + j sl of src.  16-byte loads (8 bf16 / fp16 or
// 4 fp32 values) where the dims, the strides and the pointer allow them, so that one load
// and one index division serve 4-8 values; otherwise one value per load, every padding
// word included.
__device__ __forceinline__ void gen_stage_chunk(float* dst, const void* src, int dt, int64_t base, int64_t sl,
                                                int nk, int D, int Dp, int tid) {
  const int vw = dt == 0 ? 4 : 8;  // values per 16 bytes
  const bool vec = D % vw == 0 && base % vw == 0 && sl % vw == 0 &&
                   (reinterpret_cast<uintptr_t>(src) & 15u) == 0;
  if (vec) {
    const int upr = D / vw;  // 16-byte units per row
    for (int u = tid; u < kGenChunk * upr; u += 256) {
      const int j = u / upr, d0 = (u - j * upr) * vw;
      float* o = dst + j * Dp + d0;
      if (j < nk) {
        const int64_t at = base + static_cast<int64_t>(j) * sl + d0;
        if (dt == 0) {
          *reinterpret_cast<float4*>(o) = *reinterpret_cast<const float4*>(static_cast<const float*>(src) + at);
        } else {
          const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + at);
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
          float f[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (dt == 1) {
              f[2 * i] = __uint_as_float(ws[i] << 16);
              f[2 * i + 1] = __uint_as_float(ws[i] & 0xFFFF0000u);
            } else {
              f[2 * i] = __half2float(__ushort_as_half(static_cast<unsigned short>(ws[i] & 0xFFFFu)));
              f[2 * i + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(ws[i] >> 16)));
            }
          }
          *reinterpret_cast<float4*>(o) = make_float4(f[0], f[1], f[2], f[3]);
          *reinterpret_cast<float4*>(o + 4) = make_float4(f[4], f[5], f[6], f[7]);
        }
      } else {
        *reinterpret_cast<float4*>(o) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (dt != 0) *reinterpret_cast<float4*>(o + 4) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  } else {
    for (int idx = tid; idx < kGenChunk * Dp; idx += 256) {
      const int j = idx / Dp, d = idx - j * Dp;
      dst[idx] = (j < nk && d < D) ? gen_load(src, dt, base + static_cast<int64_t>(j) * sl + d) : 0.0f;
    }
  }
}

template <int LV>
__global__ __launch_bounds__(256) void gen_attention_kernel(GenAttnArgs a) {
  extern __shared__ float4 gen_lds4[];
  float* const lds = reinterpret_cast<float*>(gen_lds4);
  __shared__ int sh_lo, sh_hi;
  const int tid = threadIdx.x;
  const int D = a.D, T = a.T;
  const int Dp = gen_dim_pad(D), Tp = gen_tile_pad(T);
  float* const Qs = lds;                 // [16][Dp]
  float* const KV = Qs + kGenRows * Dp;  // [32][Dp]
  float* const S = KV + kGenChunk * Dp;  // [16][Tp]

  const int b = blockIdx.z, hq = blockIdx.y, p0 = blockIdx.x * kGenRows;
  const int kvh = hq / (a.Hq / a.Hkv);
  const int off = a.Lk - a.Lq;  // bottom-right causal: position p sees keys <= p + off
  const bool ranges = a.row_lo != nullptr;
  const bool dense = a.amask != nullptr;

  for (int idx = tid; idx < kGenRows * Dp; idx += 256) {
    const int r = idx / Dp, d = idx - r * Dp, pos = p0 + r;
    Qs[idx] = (pos < a.Lq && d < D) ? gen_load(a.q, a.q_dt, b * a.q_sb + hq * a.q_sh + pos * a.q_sl + d) : 0.0f;
  }

  // key range [lo, hi] of a position (rows past Lq see nothing)
  auto row_range = [&](int pos, int& lo, int& hi) {
    lo = 0;
    hi = a.Lk - 1;
    if (pos >= a.Lq) {
      lo = a.Lk;
      hi = -1;
    } else if (ranges) {
      lo = a.row_lo[static_cast<int64_t>(b) * a.Lq + pos];
      hi = a.row_hi[static_cast<int64_t>(b) * a.Lq + pos];
    } else if (a.causal && !dense) {
      hi = min(a.Lk - 1, pos + off);
    }
  };
  // score phase: row sr, keys sj and sj + 16 of each chunk
  const int sr = tid & 15, sj = tid >> 4;
  const int spos = p0 + sr;
  int slo, shi;
  row_range(spos, slo, shi);
  // row phase: row rr, lanes `sub`
  const int rr = tid >> 4, sub = tid & 15;
  const int rpos = p0 + rr;
  const bool rlive = rpos < a.Lq;

  // key tiles some row of the workgroup sees (all of them under a dense mask, as in the
  // reference, where no tile is skipped)
  if (tid == 0) {
    sh_lo = a.Lk;
    sh_hi = -1;
  }
  __syncthreads();
  if (sj == 0) {
    int lo = 0, hi = a.Lk - 1;
    if (!dense) row_range(spos, lo, hi);
    if (spos < a.Lq && lo <= hi) {
      atomicMin(&sh_lo, max(lo, 0));
      atomicMax(&sh_hi, min(hi, a.Lk - 1));
    }
  }
  __syncthreads();
  const int t_lo = sh_lo <= sh_hi ? sh_lo / T : 1;
  const int t_hi = sh_lo <= sh_hi ? sh_hi / T : 0;

  float m_run = -INFINITY, l_run = 0.0f;
  float dq_run = 0.0f, dp_run = 0.0f, dg_zero = 0.0f, dg_err = 0.0f, dg_ref = 0.0f;
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  const int nd4 = (D + 63) / 64;  // 64-dim blocks of PV

  for (int t = t_lo; t <= t_hi; ++t) {
    const int key0 = t * T;
    const int W = min(T, a.Lk - key0);
    // ---- scores
    for (int c0 = 0; c0 < W; c0 += kGenChunk) {
      const int nk = min(kGenChunk, W - c0);
      __syncthreads();
      gen_stage_chunk(KV, a.k, a.k_dt, b * a.k_sb + kvh * a.k_sh + static_cast<int64_t>(key0 + c0) * a.k_sl, a.k_sl,
                      nk, D, Dp, tid);
      __syncthreads();
      // both keys' dot products in one pass over d (each Q read serves two keys; every KV row
      // of the chunk is written, rows past nk as zeros), each summed in d order
      float dots[2] = {0.0f, 0.0f};
      {
        const float4* qp = reinterpret_cast<const float4*>(Qs + sr * Dp);
        const float4* kp0 = reinterpret_cast<const float4*>(KV + sj * Dp);
        const float4* kp1 = reinterpret_cast<const float4*>(KV + (sj + 16) * Dp);
        for (int d4 = 0; d4 < (D + 3) / 4; ++d4) {
          const float4 qv = qp[d4], k0 = kp0[d4], k1 = kp1[d4];
          dots[0] = __builtin_fmaf(qv.x, k0.x, dots[0]);
          dots[1] = __builtin_fmaf(qv.x, k1.x, dots[1]);
          dots[0] = __builtin_fmaf(qv.y, k0.y, dots[0]);
          dots[1] = __builtin_fmaf(qv.y, k1.y, dots[1]);
          dots[0] = __builtin_fmaf(qv.z, k0.z, dots[0]);
          dots[1] = __builtin_fmaf(qv.z, k1.z, dots[1]);
          dots[0] = __builtin_fmaf(qv.w, k0.w, dots[0]);
          dots[1] = __builtin_fmaf(qv.w, k1.w, dots[1]);
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = sj + 16 * h;
        if (j < nk) {
          const float dot = dots[h];
          const int key = key0 + c0 + j;
          float s = dot * a.scale;
          if (a.softcap > 0.0f) s = tanhf(s / a.softcap) * a.softcap;
          if (dense) {
            s = s + a.amask[b * a.am_sb + hq * a.am_sh + static_cast<int64_t>(spos < a.Lq ? spos : 0) * a.am_sq + key];
          } else {
            bool ok = key >= slo && key <= shi;
            if (ranges && ok) ok = (a.key_bits[b * a.key_words + (key >> 5)] >> (key & 31)) & 1u;
            if (!ok) s = -INFINITY;
          }
          S[sr * Tp + c0 + j] = s;
        }
      }
    }
    __syncthreads();
    // ---- row phase: maximum, P, P^, row sums (each row's 16 lanes are one wave's)
    float mx = -INFINITY;
    for (int j = sub; j < W; j += 16) mx = fmaxf(mx, S[rr * Tp + j]);
    mx = row_max16(mx);
    const float m_new = fmaxf(m_run, mx);
    const float prev = isfinite(m_run) ? expf(m_run - m_new) : 0.0f;
    float rs = 0.0f, sq = 0.0f, sp = 0.0f;
    for (int j0 = 0; j0 < W; j0 += 128) {
      const int jb = j0 + 8 * sub;
      float p[8], ph[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float s = jb + e < W ? S[rr * Tp + jb + e] : -INFINITY;
        p[e] = isfinite(s) ? expf(s - m_new) : 0.0f;
        ph[e] = p[e];
      }
      if (a.quant_p) gen_qdq8<LV>(ph);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (jb + e < W) {
          S[rr * Tp + jb + e] = ph[e];
          rs += (a.quant_p && a.norm_same) ? ph[e] : p[e];
          if (a.diag) {
            sq += ph[e];
            sp += p[e];
            const float d = ph[e] - p[e];
            dg_err = __builtin_fmaf(d, d, dg_err);
            dg_ref = __builtin_fmaf(p[e], p[e], dg_ref);
            dg_zero += (ph[e] == 0.0f && p[e] > 0.0f) ? 1.0f : 0.0f;
          }
        }
      }
    }
    l_run = prev * l_run + row_sum16(rs);
    if (a.diag) {
      dq_run = prev * dq_run + row_sum16(sq);
      dp_run = prev * dp_run + row_sum16(sp);
    }
    m_run = m_new;
    // ---- PV: pv = P^ V over the tile, then acc = prev acc + pv
    float pv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) pv[i] = 0.0f;
    for (int c0 = 0; c0 < W; c0 += kGenChunk) {
      const int nk = min(kGenChunk, W - c0);
      __syncthreads();
      gen_stage_chunk(KV, a.v, a.v_dt, b * a.v_sb + kvh * a.v_sh + static_cast<int64_t>(key0 + c0) * a.v_sl, a.v_sl,
                      nk, D, Dp, tid);
      __syncthreads();
      for (int j = 0; j < nk; ++j) {
        const float pj = S[rr * Tp + c0 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i < nd4 && 64 * i + 4 * sub < D) {
            const float4 vv = *reinterpret_cast<const float4*>(KV + j * Dp + 64 * i + 4 * sub);
            pv[4 * i] = __builtin_fmaf(pj, vv.x, pv[4 * i]);
            pv[4 * i + 1] = __builtin_fmaf(pj, vv.y, pv[4 * i + 1]);
            pv[4 * i + 2] = __builtin_fmaf(pj, vv.z, pv[4 * i + 2]);
            pv[4 * i + 3] = __builtin_fmaf(pj, vv.w, pv[4 * i + 3]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = prev * acc[i] + pv[i];
  }

  // (all 16 lanes of a row reduce together, before any of them leaves)
  dg_zero = row_sum16(dg_zero);
  dg_err = row_sum16(dg_err);
  dg_ref = row_sum16(dg_ref);
  if (!rlive) return;
  const int64_t row = (static_cast<int64_t>(b) * a.Hq + hq) * a.Lq + rpos;
  const bool pos_l = l_run > 0.0f;
  const float den = fmaxf(l_run, FLT_MIN);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 64 * i + 4 * sub + e;
      if (i < nd4 && d < D) {
        const float o = pos_l ? acc[4 * i + e] / den : 0.0f;
        const int64_t at = b * a.o_sb + hq * a.o_sh + static_cast<int64_t>(rpos) * a.o_sl + d;
        if (a.o_dt == 0) {
          static_cast<float*>(a.o)[at] = o;
        } else if (a.o_dt == 1) {
          const __bf16 h = static_cast<__bf16>(o);
          __builtin_memcpy(static_cast<uint16_t*>(a.o) + at, &h, 2);
        } else {
          static_cast<__half*>(a.o)[at] = __float2half_rn(o);
        }
      }
    }
  }
  if (sub == 0) {
    if (a.row_den) a.row_den[row] = l_run;
    if (a.diag) {
      float* dg = a.diag + row * 5;
      dg[0] = dq_run;
      dg[1] = dp_run;
      dg[2] = dg_zero;
      dg[3] = dg_err;
      dg[4] = dg_ref;
    }
  }
}

template <int LV>
hipError_t launch_lv(const GenAttnArgs& a, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024) {
    // more than the default dynamic LDS limit (at most 116 KB here, of the 160 KB a gfx950
    // workgroup may hold)
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gen_attention_kernel<LV>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  const dim3 grid((a.Lq + kGenRows - 1) / kGenRows, a.Hq, a.B);
  hipLaunchKernelGGL((gen_attention_kernel<LV>), grid, dim3(256), lds, st, a);
  return hipSuccess;
}

}  // namespace

size_t gen_attention_lds_bytes(int D, int T) {
  const int Dp = (D + 3) / 4 * 4 + 4, Tp = (T + 7) / 8 * 8 + 4;
  return static_cast<size_t>(kGenRows * Dp + kGenChunk * Dp + kGenRows * Tp) * sizeof(float);
}

hipError_t launch_gen_attention(const GenAttnArgs& a, hipStream_t st) {
  const size_t lds = gen_attention_lds_bytes(a.D, a.T);
  if (a.p_levels == 12) return launch_lv<12>(a, lds, st);
  if (a.p_levels == 13) return launch_lv<13>(a, lds, st);
  return launch_lv<123>(a, lds, st);
}

}  // namespace faq
