// Split-key passes (tile maxima scan, combine) and the key ranges of 2-D masks: the small
// kernels around the attention kernel (hif4_attention.hip), compiled with the C ABI.
#pragma once
#include "hif4_attention.hip"

namespace faq {

// ---------------------------------------------------------------------------------------
// Split-key attention (decode and other short grids): after the maxima pass, the running
// maximum before split j of row r is the maximum of the c1-scaled tile maxima of its first
// t_lo(j) tiles (-inf if none), restricted to the tiles the row sees.
constexpr int kScanThreads = 256;
constexpr int kScanMaxTiles = 16384;  // the row's tile maxima in LDS (64 KiB)

struct SplitScanArgs {
  const float* mx;     // [rows_total, mx_stride]
  int mx_stride;
  int ntiles;          // key tiles of Lk (<= kScanMaxTiles)
  float* m_start;      // [nsplit, rows_total]
  int rows_total;
  int nsplit;
  int tiles_per_split;
  int Hq, Lq, Lk, causal;
  const int* row_lo;  // key-range mode: the row's key range (the attention kernel's bounds)
  const int* row_hi;
};

// One workgroup per row: the row's tile maxima (-inf outside the tiles it sees) go to LDS in
// one coalesced pass, thread j takes the maximum of split j's tiles, and a Hillis-Steele scan
// over the splits (in chunks of 256 with a carry) gives each split the exclusive prefix
// maximum.  The maxima are exact, so the result equals a serial scan.
__global__ __launch_bounds__(kScanThreads) void split_scan_kernel(SplitScanArgs a) {
  extern __shared__ float tm[];  // [ntiles]
  __shared__ float sm[kScanThreads];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int pos = row % a.Lq;
  // key tiles [t0, t1) of this row; the maxima pass wrote every one of them
  int t0 = 0, t1;
  if (a.row_lo) {
    const int64_t br = static_cast<int64_t>(row / (a.Hq * a.Lq)) * a.Lq + pos;
    const int lo = a.row_lo[br], hi = a.row_hi[br];
    t0 = lo <= hi ? lo / kKeyTile : 0;
    t1 = lo <= hi ? hi / kKeyTile + 1 : 0;
  } else {
    const int kend = a.causal ? min(a.Lk, max(0, pos + a.Lk - a.Lq + 1)) : a.Lk;
    t1 = (kend + kKeyTile - 1) / kKeyTile;
  }
  const float* mr = a.mx + static_cast<int64_t>(row) * a.mx_stride;
  for (int t = tid; t < a.ntiles; t += kScanThreads) tm[t] = (t >= t0 && t < t1) ? mr[t] : -INFINITY;
  __syncthreads();
  float carry = -INFINITY;
  for (int j0 = 0; j0 < a.nsplit; j0 += kScanThreads) {
    const int j = j0 + tid;
    float m = -INFINITY;
    if (j < a.nsplit) {
      const int e = min(a.ntiles, (j + 1) * a.tiles_per_split);
      for (int t = j * a.tiles_per_split; t < e; ++t) m = fmaxf(m, tm[t]);
    }
    sm[tid] = m;
    __syncthreads();
    for (int d = 1; d < kScanThreads; d <<= 1) {
      const float o = tid >= d ? sm[tid - d] : -INFINITY;
      __syncthreads();
      sm[tid] = fmaxf(sm[tid], o);
      __syncthreads();
    }
    if (j < a.nsplit) a.m_start[static_cast<int64_t>(j) * a.rows_total + row] = fmaxf(carry, tid > 0 ? sm[tid - 1] : -INFINITY);
    carry = fmaxf(carry, sm[kScanThreads - 1]);
    __syncthreads();
  }
}

// O = sum_j 2^(m_j - M) O_j / sum_j 2^(m_j - M) l_j with M the row's final running maximum;
// the per-split recurrences already used the reference's maxima, so only the fp32 order of
// the O and l sums differs from one pass.
constexpr int kCombineThreads = 128;
constexpr int kCombineMaxSplits = 4096;
constexpr int kCombineGroups = 16;  // split groups
constexpr int kCombineSlots = 512;  // l partial sums
constexpr int kCombineQuarters = 4; // workgroups per row, 32 dims each

struct SplitCombineArgs {
  const float* part_o;   // [nsplit, rows_total, 128]
  const float* part_lm;  // [nsplit, rows_total, 2]
  int rows_total, nsplit;
  int Hq, Lq;
  void* o;               // [B, Hq, Lq, 128] via strides
  int64_t o_sb, o_sh, o_sl;
  int o_f32;
  float* row_den;        // optional [rows_total]
};

// Workgroup (row, quarter k) of 128 threads writes dims 32 k .. 32 k + 31 of the row.  The
// split weights w_j = 2^(m_j - M) (0 for an empty split) go to LDS.  Thread (g, qq),
// g = tid / 8, sums w_j O_j[4 q .. 4 q + 3], q = 8 k + qq, over the splits j = g mod 16 in
// order, and the 16 group sums are added in the fixed tree g += g + d, d = 8, 4, 2, 1.  l is
// the fixed tree over 512 slots (slot s sums w_j l_j over j = s mod 512 in order, then
// slot s += slot s + d, d = 256, ..., 1), which every quarter computes the same way.  The
// results do not depend on the launch shape: the same pairs are added in the same order.
// The first eight O loads of each thread and its first (l, m) pairs are issued before the
// reductions that need M.
__global__ __launch_bounds__(kCombineThreads) void split_combine_kernel(SplitCombineArgs a) {
  __shared__ float wsh[kCombineMaxSplits];
  __shared__ float red[kCombineSlots];
  __shared__ float wmax[kCombineThreads / 64];
  __shared__ float4 gsum[kCombineGroups][8];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int g = tid / 8, qq = tid % 8, q = 8 * static_cast<int>(blockIdx.y) + qq;
  const float4* po = reinterpret_cast<const float4*>(a.part_o + static_cast<int64_t>(row) * kDim) + q;
  const int64_t js = static_cast<int64_t>(a.rows_total) * (kDim / 4);  // float4 stride of one split
  const float2* plm = reinterpret_cast<const float2*>(a.part_lm) + row;  // split j at plm[j * rows_total]
  float4 v0[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int jj = g + kCombineGroups * u;
    v0[u] = jj < a.nsplit ? po[static_cast<int64_t>(jj) * js] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float2 lm0[4];  // splits tid + 128 r
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int j = tid + kCombineThreads * r;
    lm0[r] = j < a.nsplit ? plm[static_cast<int64_t>(j) * a.rows_total] : make_float2(0.0f, -INFINITY);
  }
  // M: the maximum over the splits (a maximum is exact: any reduction order gives the same value)
  float mloc = fmaxf(fmaxf(lm0[0].y, lm0[1].y), fmaxf(lm0[2].y, lm0[3].y));
  for (int j = tid + kCombineSlots; j < a.nsplit; j += kCombineThreads)
    mloc = fmaxf(mloc, plm[static_cast<int64_t>(j) * a.rows_total].y);
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, d, 64));
  if ((tid & 63) == 0) wmax[tid >> 6] = mloc;
  __syncthreads();
  const float mmax = fmaxf(wmax[0], wmax[1]);
  // weights, and slot s = tid + 128 r of the l tree: sum of w_j l_j over j = s mod 512
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int s = tid + kCombineThreads * r;
    float lloc = 0.0f;
    for (int j = s; j < a.nsplit; j += kCombineSlots) {
      const float2 lm = j == s ? lm0[r] : plm[static_cast<int64_t>(j) * a.rows_total];
      const float w = (mmax == -INFINITY || lm.x == 0.0f) ? 0.0f : __builtin_amdgcn_exp2f(lm.y - mmax);
      wsh[j] = w;
      lloc = __builtin_fmaf(w, lm.x, lloc);
    }
    red[s] = lloc;
  }
  __syncthreads();
  // O: splits j = g, g + 16, ... of group g (the first eight from the loads issued at the start)
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  auto add = [&](float w, float4 v) {
    acc.x = __builtin_fmaf(w, v.x, acc.x);
    acc.y = __builtin_fmaf(w, v.y, acc.y);
    acc.z = __builtin_fmaf(w, v.z, acc.z);
    acc.w = __builtin_fmaf(w, v.w, acc.w);
  };
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (g + kCombineGroups * u < a.nsplit) add(wsh[g + kCombineGroups * u], v0[u]);
  int j = g + 8 * kCombineGroups;
  for (; j + 7 * kCombineGroups < a.nsplit; j += 8 * kCombineGroups) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = po[static_cast<int64_t>(j + kCombineGroups * u) * js];
#pragma unroll
    for (int u = 0; u < 8; ++u) add(wsh[j + kCombineGroups * u], v[u]);
  }
  for (; j < a.nsplit; j += kCombineGroups) add(wsh[j], po[static_cast<int64_t>(j) * js]);
  gsum[g][qq] = acc;
  // the first step of each tree (l: d = 256, two slots per thread; O: d = 8)
  red[tid] += red[tid + 256];
  red[tid + 128] += red[tid + 384];
  __syncthreads();
  red[tid] += red[tid + 128];  // d = 128
  if (g < 8) {
    const float4 o = gsum[g + 8][qq];
    float4 m = gsum[g][qq];
    m.x += o.x;
    m.y += o.y;
    m.z += o.z;
    m.w += o.w;
    gsum[g][qq] = m;
  }
  __syncthreads();
#pragma unroll
  for (int d = 4; d >= 2; d >>= 1) {
    if (g < d) {
      const float4 o = gsum[g + d][qq];
      float4 m = gsum[g][qq];
      m.x += o.x;
      m.y += o.y;
      m.z += o.z;
      m.w += o.w;
      gsum[g][qq] = m;
    }
    __syncthreads();
  }
  if (tid < 64) {
    // l: d = 64 from LDS, then d = 32 .. 1 as shuffles (lane 0 ends with the sum)
    float x = red[tid] + red[tid + 64];
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) x += __shfl_down(x, d, 64);
    const float l = __shfl(x, 0, 64);
    // O: d = 1, groups 0 and 1 (lanes 0..7 and 8..15)
    float4 sum = gsum[g < 2 ? g : 0][qq];
    sum.x += __shfl_down(sum.x, 8, 64);
    sum.y += __shfl_down(sum.y, 8, 64);
    sum.z += __shfl_down(sum.z, 8, 64);
    sum.w += __shfl_down(sum.w, 8, 64);
    if (g == 0) {
      const int pos = row % a.Lq;
      const int hq = (row / a.Lq) % a.Hq;
      const int b = row / (a.Lq * a.Hq);
      if (a.row_den && q == 0) a.row_den[row] = l;
      const float vals[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = l > 0.0f ? vals[e] / fmaxf(l, 1.17549435e-38f) : 0.0f;
        const int64_t off = b * a.o_sb + hq * a.o_sh + static_cast<int64_t>(pos) * a.o_sl + 4 * q + e;
        if (a.o_f32) static_cast<float*>(a.o)[off] = v;
        else static_cast<uint16_t*>(a.o)[off] = f32_to_bf16_bits_rne(v);
      }
    }
  }
}

inline void launch_split_combine(const SplitCombineArgs& ca, hipStream_t st) {
  hipLaunchKernelGGL(split_combine_kernel, dim3(static_cast<unsigned>(ca.rows_total), kCombineQuarters),
                     dim3(kCombineThreads), 0, st, ca);
}

// ---------------------------------------------------------------------------------------
// Key ranges of a 2-D attention mask.  sfa:341-368 takes the last Lk mask columns as
// key_valid and their last Lq (zero-extended in front when Lq > Lk) as query_valid;
// sfa:406-427 then compares ranks among valid keys: key rank r(k) = #valid keys < k, query
// anchor = query rank + #valid keys - #valid queries, which is r(j) for the query's own key
// column j = p + Lk - Lq.  Row p (query_valid) sees the valid keys with rank in
//   [max(0, anchor - window + 1) if window else 0,
//    min(#valid - 1, anchor if causal, else anchor + window - 1 if window)]
// and, ranks growing with k, those keys are exactly the valid keys between two positions:
// row_lo = the key of rank lo, row_hi = the key of rank hi.  Without a mask (sfa:395-405)
// the same rule runs on positions.  One workgroup per batch row.
constexpr int kMaskThreads = 1024;
constexpr int kMaskMaxWords = 16384;  // Lk <= 524288

struct MaskBoundsArgs {
  const uint8_t* mask;  // [B, Lk] (row stride mask_sb), nonzero = valid; nullptr: all valid
  int64_t mask_sb;
  int Lq, Lk, causal, window;
  int* row_lo;          // [B, Lq]
  int* row_hi;
  int* row_blocks;      // [B, ceil(Lq / 32), 4] (see AttnArgs::row_blocks)
  uint32_t* key_bits;   // optional [B, key_words]
  int64_t key_words;
};

__global__ __launch_bounds__(kMaskThreads) void mask_bounds_kernel(MaskBoundsArgs a) {
  __shared__ uint32_t bits[kMaskMaxWords];
  __shared__ int base[kMaskMaxWords];
  __shared__ int part[kMaskThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int nw = (a.Lk + 31) / 32;
  for (int wd = tid; wd < nw; wd += kMaskThreads) {
    const int n = min(32, a.Lk - 32 * wd);
    uint32_t m = n == 32 ? ~0u : ((1u << n) - 1u);
    if (a.mask) {
      const uint8_t* src = a.mask + b * a.mask_sb + 32 * wd;
      m = 0;
      for (int i = 0; i < n; ++i) m |= (src[i] != 0 ? 1u : 0u) << i;
    }
    bits[wd] = m;
  }
  __syncthreads();
  if (a.key_bits)
    for (int64_t wd = tid; wd < a.key_words; wd += kMaskThreads)
      a.key_bits[b * a.key_words + wd] = wd < nw ? bits[wd] : 0u;
  // exclusive prefix counts of valid keys per word: contiguous word chunks per thread,
  // wave scans of the chunk sums, then the 16 wave totals
  const int chunk = (nw + kMaskThreads - 1) / kMaskThreads;
  const int w0 = min(nw, tid * chunk), w1 = min(nw, w0 + chunk);
  int own = 0;
  for (int wd = w0; wd < w1; ++wd) own += __popc(bits[wd]);
  const int lane = tid & 63, wv = tid >> 6;
  int inc = own;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(inc, d, 64);
    if (lane >= d) inc += y;
  }
  if (lane == 63) part[wv] = inc;
  __syncthreads();
  int before = inc - own;
  for (int i = 0; i < wv; ++i) before += part[i];
  int total = 0;
  for (int i = 0; i < kMaskThreads / 64; ++i) total += part[i];
  for (int wd = w0; wd < w1; ++wd) {
    base[wd] = before;
    before += __popc(bits[wd]);
  }
  __syncthreads();
  // position of the valid key of rank r (0 <= r < total)
  auto select = [&](int r) {
    int lo = 0, hi = nw - 1;  // last word with base <= r
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (base[mid] <= r) lo = mid;
      else hi = mid - 1;
    }
    uint32_t m = bits[lo];
    for (int k = r - base[lo]; k > 0; --k) m &= m - 1u;
    return 32 * lo + __ffs(static_cast<int>(m)) - 1;
  };
  const int nblk = (a.Lq + 31) / 32;
  for (int p0 = 0; p0 < a.Lq; p0 += kMaskThreads) {
    const int p = p0 + tid;  // every thread takes part in the 32-position summaries
    int lo = a.Lk, hi = -1;
    const int j = p + a.Lk - a.Lq;
    // without a mask every query is valid and ranks are positions (sfa:395-405), so the
    // anchor is j itself, negative for the first Lq - Lk queries when Lq > Lk
    const bool valid = p < a.Lq && (a.mask ? (j >= 0 && ((bits[j >> 5] >> (j & 31)) & 1u)) : true);
    if (valid) {
      // (signed: __popc is unsigned, and a negative j must stay negative)
      const int64_t anchor =
          a.mask ? static_cast<int64_t>(base[j >> 5]) + static_cast<int64_t>(__popc(bits[j >> 5] & ((1u << (j & 31)) - 1u)))
                 : static_cast<int64_t>(j);
      int64_t rlo = 0, rhi = total - 1;
      if (a.causal) rhi = min(rhi, anchor);
      if (a.window > 0) {
        rlo = max(rlo, anchor - a.window + 1);
        if (!a.causal) rhi = min(rhi, anchor + a.window - 1);
      }
      if (rlo <= rhi) {
        lo = select(static_cast<int>(rlo));
        hi = select(static_cast<int>(rhi));
      }
    }
    if (p < a.Lq) {
      a.row_lo[static_cast<int64_t>(b) * a.Lq + p] = lo;
      a.row_hi[static_cast<int64_t>(b) * a.Lq + p] = hi;
    }
    // summaries of the 32 positions [32 q, 32 q + 32) held by 32 consecutive lanes
    const bool any = lo <= hi;
    int kb = any ? lo : a.Lk, ke = any ? hi + 1 : 0;
    int lmax = p < a.Lq ? (any ? lo : a.Lk) : 0, hmin = p < a.Lq ? (any ? hi : -1) : a.Lk;
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) {
      kb = min(kb, __shfl_xor(kb, m, 64));
      ke = max(ke, __shfl_xor(ke, m, 64));
      lmax = max(lmax, __shfl_xor(lmax, m, 64));
      hmin = min(hmin, __shfl_xor(hmin, m, 64));
    }
    if ((p & 31) == 0 && p < a.Lq) {
      int* rb = a.row_blocks + (static_cast<int64_t>(b) * nblk + (p >> 5)) * 4;
      rb[0] = kb;
      rb[1] = ke;
      rb[2] = lmax;
      rb[3] = hmin;
    }
  }
}

}  // namespace faq
