// C ABI of the HiF4 attention path (declarations and contracts: include/faquant_amd.h).
// Validates arguments on the host, selects the kernel instantiation, launches it on the
// caller's stream and reports errors through a thread-local message.
#include <algorithm>
#include <cstdarg>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/faquant_amd.h"
#include "attn_aux.hip"
#include "attn_decode.h"
#include "attn_generic.h"
#include "hif4_linear.h"
#include "hif4_attention.hip"
#include "hif4_quant.hip"
#include "mfma_probe.hip"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FAQ_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_err.clear();
  return FAQ_OK;
}

bool valid_levels(int lv) { return lv == 123 || lv == 12 || lv == 13; }
bool valid_dtype(int dt) { return dt == FAQ_F32 || dt == FAQ_BF16 || dt == FAQ_F16; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

unsigned grid_for(int64_t threads) { return static_cast<unsigned>((threads + 255) / 256); }

template <typename T>
void launch_qdq(const faq::QdqRowsArgs& a, int levels, int64_t threads, hipStream_t st) {
  const dim3 grid(grid_for(threads));
  if (levels == 123) hipLaunchKernelGGL((faq::qdq_rows_kernel<T, 123>), grid, dim3(256), 0, st, a);
  else if (levels == 12) hipLaunchKernelGGL((faq::qdq_rows_kernel<T, 12>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((faq::qdq_rows_kernel<T, 13>), grid, dim3(256), 0, st, a);
}

template <typename Tin, typename Tout>
void launch_hadamard(const faq::HadamardRowsArgs& a, int64_t threads, hipStream_t st) {
  hipLaunchKernelGGL((faq::hadamard_rows_kernel<Tin, Tout>), dim3(grid_for(threads)), dim3(256), 0, st, a);
}

template <typename Tin>
void launch_hadamard_in(const faq::HadamardRowsArgs& a, int out_dtype, int64_t threads, hipStream_t st) {
  if (out_dtype == FAQ_F32) launch_hadamard<Tin, float>(a, threads, st);
  else if (out_dtype == FAQ_BF16) launch_hadamard<Tin, __hip_bfloat16>(a, threads, st);
  else launch_hadamard<Tin, __half>(a, threads, st);
}

template <typename T>
void launch_act(const faq::ActQdqArgs& a, int levels, int64_t threads, hipStream_t st) {
  const dim3 grid(grid_for(threads));
  if (levels == 12) hipLaunchKernelGGL((faq::act_qdq_rows_kernel<T, 12>), grid, dim3(256), 0, st, a);
  else if (levels == 13) hipLaunchKernelGGL((faq::act_qdq_rows_kernel<T, 13>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((faq::act_qdq_rows_kernel<T, 123>), grid, dim3(256), 0, st, a);
}

template <typename T, int R, int NT, bool G>
void launch_act_row_g(const faq::ActRowArgs& a, int levels, size_t lds, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.rows));
  if (a.stage_round) hipLaunchKernelGGL((faq::act_row_kernel<T, 123, R, NT, G, true>), grid, dim3(NT), lds, st, a);
  else if (levels == 12) hipLaunchKernelGGL((faq::act_row_kernel<T, 12, R, NT, G>), grid, dim3(NT), lds, st, a);
  else if (levels == 13) hipLaunchKernelGGL((faq::act_row_kernel<T, 13, R, NT, G>), grid, dim3(NT), lds, st, a);
  else hipLaunchKernelGGL((faq::act_row_kernel<T, 123, R, NT, G>), grid, dim3(NT), lds, st, a);
}

template <typename T, int R, int NT>
void launch_act_row_r(const faq::ActRowArgs& a, int levels, size_t lds, hipStream_t st) {
  if (a.gen12) launch_act_row_g<T, R, NT, true>(a, levels, lds, st);
  else launch_act_row_g<T, R, NT, false>(a, levels, lds, st);
}

// 8-value chunks per lane and threads per workgroup: 256 threads with 1 or 2 chunks each up
// to 4096 features, then 512 and 1024 threads with 2, and 1024 threads with 4 up to 32768.
template <typename T>
void launch_act_row(const faq::ActRowArgs& a, int levels, size_t lds, hipStream_t st) {
  if (a.cols <= 2048) launch_act_row_r<T, 1, 256>(a, levels, lds, st);
  else if (a.cols <= 4096) launch_act_row_r<T, 2, 256>(a, levels, lds, st);
  else if (a.cols <= 8192) launch_act_row_r<T, 2, 512>(a, levels, lds, st);
  // three chunks per lane for Qwen3-8B's 12288-feature rows: every lane busy (two chunks of
  // 1024 threads leave a quarter idle), same-box A/B 110.8 -> 108.1 us for the full path
  else if (a.cols <= 12288) launch_act_row_r<T, 3, 512>(a, levels, lds, st);
  else if (a.cols <= 16384) launch_act_row_r<T, 2, 1024>(a, levels, lds, st);
  else launch_act_row_r<T, 4, 1024>(a, levels, lds, st);
}

// LDS bytes one workgroup of the current device may hold (cached per device; 64 KiB when
// the query fails).
size_t device_lds_per_block() {
  static size_t cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
  if (cached[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) v = 65536;
    cached[dev] = static_cast<size_t>(v);
  }
  return cached[dev];
}

template <typename Tin, typename Tround>
void launch_prep(const faq::OperandPrepArgs& a, int levels, int64_t, hipStream_t st) {
  const int per_block = 16 * faq::kPrepRows;
  const dim3 grid(static_cast<unsigned>((a.L + per_block - 1) / per_block), static_cast<unsigned>(a.H),
                  static_cast<unsigned>(a.B));
  if (levels == 12) hipLaunchKernelGGL((faq::operand_prep_kernel<Tin, Tround, 12>), grid, dim3(256), 0, st, a);
  else if (levels == 13) hipLaunchKernelGGL((faq::operand_prep_kernel<Tin, Tround, 13>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((faq::operand_prep_kernel<Tin, Tround, 123>), grid, dim3(256), 0, st, a);
}

template <typename Tin>
void launch_prep_in(const faq::OperandPrepArgs& a, int round_dtype, int levels, int64_t threads, hipStream_t st) {
  if (round_dtype == FAQ_F32) launch_prep<Tin, float>(a, levels, threads, st);
  else if (round_dtype == FAQ_BF16) launch_prep<Tin, __hip_bfloat16>(a, levels, threads, st);
  else launch_prep<Tin, __half>(a, levels, threads, st);
}

template <typename Tin>
void launch_prep_vt(const faq::OperandPrepVtArgs& a, int levels, dim3 grid, hipStream_t st) {
  if (levels == 12) hipLaunchKernelGGL((faq::operand_prep_vt_kernel<Tin, 12>), grid, dim3(256), 0, st, a);
  else if (levels == 13) hipLaunchKernelGGL((faq::operand_prep_vt_kernel<Tin, 13>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((faq::operand_prep_vt_kernel<Tin, 123>), grid, dim3(256), 0, st, a);
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Workgroups of the attention kernel for n_items work items per split: one per CU in total
// (a multiple of 8 when that many), never more than the items.
int workers_for(int n_items, int nsplit) {
  int p = std::max(1, device_cus() / std::max(1, nsplit));
  if (p >= 8) p -= p % 8;
  return std::max(1, std::min(n_items, p));
}

int n_items_of(const faq::AttnArgs& a) {
  return a.B * a.Hkv * (a.Hq / a.Hkv / a.hpw) * a.n_pblocks;
}

// fp32(sqrt(n)), its fp32 reciprocal and whether it is a power of two (n = 4^k)
faq::SqrtDiv sqrt_div(int n) {
  faq::SqrtDiv d{};
  d.d = static_cast<float>(std::sqrt(static_cast<double>(n > 0 ? n : 1)));
  d.r = 1.0f / d.d;
  int k = 0;
  while ((1 << k) < n) ++k;
  d.pow2 = (n > 0 && (1 << k) == n && k % 2 == 0) ? 1 : 0;
  return d;
}


// Validation and kernel arguments shared by the one-pass and split-key entry points.
// Returns FAQ_OK with `a`/`grid` filled, 1 when there is nothing to launch, or a status.
int attention_setup(const char* who, const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                    int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* vt, int64_t v_sb, int64_t v_sh,
                    int64_t v_sd, int Lpad, void* o, int o_dtype, int64_t o_sb, int64_t o_sh, int64_t o_sl, int B,
                    int Hq, int Hkv, int Lq, int Lk, int causal, float scale, int quant_p, int p_levels,
                    float* row_den, int out_levels, const faq_attn_opts* opts, faq::AttnArgs& a, dim3& grid) {
  if (!q || !k || !vt || !o) return fail(FAQ_EINVAL, "%s: null operand", who);
  if (opts) {
    const bool any = opts->row_lo || opts->row_hi || opts->row_blocks || opts->key_bits;
    if (any && !(opts->row_lo && opts->row_hi && opts->row_blocks && opts->key_bits))
      return fail(FAQ_EINVAL, "%s: row_lo, row_hi, row_blocks and key_bits go together", who);
    if (opts->row_blocks && (reinterpret_cast<uintptr_t>(opts->row_blocks) & 15u))
      return fail(FAQ_EINVAL, "%s: row_blocks must be 16-byte aligned", who);
    if (any && opts->key_words < 4 * ((static_cast<int64_t>(Lk) + 127) / 128))
      return fail(FAQ_EINVAL, "%s: key_words must be >= 4 * ceil(Lk / 128)", who);
    if (!(opts->softcap >= 0.0f) || opts->softcap == INFINITY)
      return fail(FAQ_EINVAL, "softcap must be non-negative");
    if (opts->softcap > 0.0f && !any && !opts->dense_mask)
      return fail(FAQ_EINVAL, "%s: the softcap needs key ranges (faq_attention_mask_bounds)", who);
    if (opts->pv_probe && !quant_p) return fail(FAQ_EINVAL, "%s: the PV-normalizer probe needs quant_p", who);
    if (opts->dense_mask && any)
      return fail(FAQ_EINVAL, "%s: a dense mask and key ranges are exclusive", who);
    if (opts->dense_mask && (!aligned16(opts->dense_mask) || (opts->dm_sb | opts->dm_sh | opts->dm_sq) & 3))
      return fail(FAQ_EINVAL, "%s: the dense mask needs 16-byte aligned rows", who);
    if (opts->pv_probe && !aligned16(opts->pv_probe)) return fail(FAQ_EINVAL, "%s: misaligned pv_probe", who);
    if (opts->p_dump && !quant_p) return fail(FAQ_EINVAL, "%s: the P dump needs quant_p", who);
    if (opts->q_prep && opts->q_hadamard != 0 && opts->q_hadamard != 64 && opts->q_hadamard != 128)
      return fail(FAQ_EUNSUP, "%s: the Q prologue's Hadamard block must be 0, 64 or 128, got %d", who, opts->q_hadamard);
    if (opts->q_prep && opts->q_levels != 0 && !valid_levels(opts->q_levels))
      return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", opts->q_levels);
    if (opts->p_dump && (!aligned16(opts->p_dump) || opts->p_dump_stride % 4 ||
                         opts->p_dump_stride < 128 * ((static_cast<int64_t>(Lk) + 127) / 128)))
      return fail(FAQ_EINVAL, "%s: p_dump must be 16-byte aligned with a stride >= 128 * ceil(Lk / 128), a multiple of 4",
                  who);
  }
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Lq < 0 || Lk < 0) return fail(FAQ_EINVAL, "%s: bad sizes", who);
  if (Hq % Hkv) return fail(FAQ_EINVAL, "query heads must be divisible by key/value heads");
  if (Lpad % 128 || Lpad < Lk) return fail(FAQ_EINVAL, "%s: Lpad must be a multiple of 128 >= Lk", who);
  if (o_dtype != FAQ_F32 && o_dtype != FAQ_BF16) return fail(FAQ_EUNSUP, "%s: output must be fp32 or bf16", who);
  if (quant_p && !valid_levels(p_levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", p_levels);
  if (out_levels != 0 && !valid_levels(out_levels))
    return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", out_levels);
  if (!aligned16(q) || !aligned16(k) || !aligned16(vt) || !aligned16(o))
    return fail(FAQ_EINVAL, "%s: pointers must be 16-byte aligned", who);
  if ((q_sb | q_sh | q_sl | k_sb | k_sh | k_sl | v_sb | v_sh | v_sd) & 7)
    return fail(FAQ_EINVAL, "%s: operand strides must be multiples of 8 elements", who);
  if ((o_sb | o_sh | o_sl) & 3) return fail(FAQ_EINVAL, "%s: output strides must be multiples of 4 elements", who);
  if (v_sd < Lpad) return fail(FAQ_EINVAL, "%s: v_sd must be >= Lpad", who);
  // the kernel addresses one head's K and V^T with 32-bit byte offsets
  if (k_sl > (int64_t(1) << 22) || v_sd > (int64_t(1) << 22) ||
      (static_cast<int64_t>(Lk) * k_sl + 128) * 2 >= (int64_t(1) << 32) || 128 * v_sd * 2 >= (int64_t(1) << 32))
    return fail(FAQ_EUNSUP, "%s: one head's K or V^T spans more than 4 GiB of addresses", who);
  if (B == 0 || Lq == 0) return 1;
  const int G = Hq / Hkv;
  // eight waves of 32 query rows per workgroup; hpw query heads of one KV head share it
  const int hpw = (G % 8 == 0) ? 8 : (G % 4 == 0) ? 4 : (G % 2 == 0) ? 2 : 1;
  const int pos_per_wg = 32 * (8 / hpw);
  a = faq::AttnArgs{};
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_sl = q_sl;
  a.k = k;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_sl = k_sl;
  a.vt = vt;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.v_sd = v_sd;
  a.o = o;
  a.o_sb = o_sb;
  a.o_sh = o_sh;
  a.o_sl = o_sl;
  a.o_f32 = o_dtype == FAQ_F32;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Lq = Lq;
  a.Lk = Lk;
  a.causal = causal != 0;
  a.scale = scale;
  if (opts) {
    a.row_lo = opts->row_lo;
    a.row_hi = opts->row_hi;
    a.row_blocks = opts->row_blocks;
    a.key_bits = opts->key_bits;
    a.key_words = opts->key_words;
    a.softcap = opts->softcap;
    a.softcap_rec = opts->softcap > 0.0f ? static_cast<float>(1.0 / static_cast<double>(opts->softcap)) : 0.0f;
    a.diag = opts->pv_probe;
    a.p_dump = opts->p_dump;
    a.p_dump_stride = opts->p_dump_stride;
    a.amask = opts->dense_mask;
    a.am_sb = opts->dm_sb;
    a.am_sh = opts->dm_sh;
    a.am_sq = opts->dm_sq;
    if (a.amask) a.causal = 0;  // the dense mask replaces the causal rule (sfa:731-757)
    if (opts->q_prep) {
      a.q_prep = 1;
      a.q_had = opts->q_hadamard;
      a.q_levels = opts->q_levels;
      a.q_div = sqrt_div(opts->q_hadamard);
    }
  }
  // the softcap and dense-mask paths scale the scores themselves, which then enter the
  // exponent unscaled
  a.c1 = static_cast<float>(static_cast<double>(a.softcap > 0.0f || a.amask ? 1.0f : scale) * 1.4426950408889634);
  a.hpw = hpw;
  a.n_pblocks = (Lq + pos_per_wg - 1) / pos_per_wg;
  a.row_den = row_den;
  a.out_levels = out_levels;
  a.rows_total = B * Hq * Lq;
  // one workgroup per CU (the K/V stages fill most of its LDS) running work items back to
  // back; P a multiple of 8 keeps item i on XCD i % 8, as a one-item-per-workgroup grid does
  const int64_t n_items = static_cast<int64_t>(B) * Hkv * (G / hpw) * a.n_pblocks;
  if (n_items > INT32_MAX) return fail(FAQ_EUNSUP, "%s: too many work items", who);
  grid = dim3(static_cast<unsigned>(workers_for(static_cast<int>(n_items), 1)), 1, 1);
  return FAQ_OK;
}

void launch_attention(const faq::AttnArgs& a, int quant_p, int p_levels, int norm_same, dim3 grid, hipStream_t st) {
  if (a.amask && a.softcap > 0.0f) faq::launch_attention_mask<4>(a, quant_p, p_levels, norm_same, grid, st);
  else if (a.amask) faq::launch_attention_mask<3>(a, quant_p, p_levels, norm_same, grid, st);
  else if (a.softcap > 0.0f) faq::launch_attention_mask<2>(a, quant_p, p_levels, norm_same, grid, st);
  else if (a.row_lo) faq::launch_attention_mask<1>(a, quant_p, p_levels, norm_same, grid, st);
  else faq::launch_attention_mask<0>(a, quant_p, p_levels, norm_same, grid, st);
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

struct SplitLayout {
  int64_t mx, m_start, part_o, part_lm, total;  // byte offsets and size
  int ntiles, tiles_per_split;
};

SplitLayout split_layout(int B, int Hq, int Lq, int Lk, int nsplit) {
  SplitLayout s{};
  const int64_t rows = static_cast<int64_t>(B) * Hq * Lq;
  s.ntiles = (Lk + 127) / 128;
  s.tiles_per_split = nsplit > 0 ? (s.ntiles + nsplit - 1) / nsplit : 0;
  s.mx = 0;
  s.m_start = align256(rows * std::max(s.ntiles, 1) * 4);
  s.part_o = s.m_start + align256(rows * nsplit * 4);
  s.part_lm = s.part_o + align256(rows * nsplit * 128 * 4);
  s.total = s.part_lm + align256(rows * nsplit * 2 * 4);
  return s;
}

struct DecodeLayout {
  int64_t s, gmx, smx, part_o, part_lm, total;  // byte offsets and size
  int ntiles, tps;
};

DecodeLayout decode_layout(int B, int Hq, int Lq, int Lk, int nsplit) {
  DecodeLayout d{};
  const int64_t rows = static_cast<int64_t>(B) * Hq * Lq;
  d.ntiles = (Lk + 127) / 128;
  d.tps = nsplit > 0 ? (d.ntiles + nsplit - 1) / nsplit : 0;
  d.s = 0;
  d.gmx = align256(rows * d.ntiles * 128 * 4);
  d.smx = d.gmx + align256(rows * d.ntiles * 2 * 4);
  d.part_o = d.smx + align256(rows * nsplit * 4);
  d.part_lm = d.part_o + align256(rows * nsplit * 128 * 4);
  d.total = d.part_lm + align256(rows * nsplit * 2 * 4);
  return d;
}

}  // namespace

// Scratch of faq_attention_fwd_split_noalloc: the split path's workspace (tile maxima, the
// running maximum before each key range, partial O and (l, m) per range) for callers that
// cannot allocate.  Each GPU the library runs on holds its own copy for the life of the
// process.  Host code must not use this name as a device address: the per-device address
// comes from hipGetSymbolAddress (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[FAQ_NOALLOC_SCRATCH_BYTES];

namespace {

// Device address of `scratch` on the current device, looked up once per device with that
// device current; nullptr (and the error message set) on failure.
void* noalloc_scratch() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(FAQ_ELAUNCH, "faq_attention_fwd_split_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(FAQ_ELAUNCH, "faq_attention_fwd_split_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace

extern "C" {

const char* faq_last_error(void) { return g_err.c_str(); }

const char* faq_version(void) { return "faquant_amd 0.1 gfx950"; }

int faq_hif4_qdq_rows(const void* x, void* y, int64_t rows, int64_t cols, int dtype, int levels, float* scale,
                      float* rec, int8_t* lv2, int8_t* lv3, uint8_t* codes, uint8_t* scale_byte, uint8_t* lv2_bits,
                      uint16_t* lv3_bits, faq_stream_t stream) {
  if ((!x || !y) && rows > 0) return fail(FAQ_EINVAL, "faq_hif4_qdq_rows: null input or output");
  if (rows < 0 || cols <= 0) return fail(FAQ_EINVAL, "HiF4 fake quantization does not support an empty axis");
  if (!valid_dtype(dtype)) return fail(FAQ_EINVAL, "faq_hif4_qdq_rows: unsupported dtype %d", dtype);
  if (!valid_levels(levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", levels);
  if (codes && cols % 64) return fail(FAQ_EINVAL, "faq_hif4_qdq_rows: packed codes need cols %% 64 == 0");
  if (rows == 0) return FAQ_OK;
  faq::QdqRowsArgs a{};
  a.x = x;
  a.y = y;
  a.rows = rows;
  a.cols = cols;
  a.vec = (cols % 8 == 0) && aligned16(x) && aligned16(y);
  a.scale = scale;
  a.rec = rec;
  a.lv2 = lv2;
  a.lv3 = lv3;
  a.codes = codes;
  a.scale_byte = scale_byte;
  a.lv2_bits = lv2_bits;
  a.lv3_bits = lv3_bits;
  const int64_t threads = rows * ((cols + 63) / 64) * 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FAQ_F32) launch_qdq<float>(a, levels, threads, st);
  else if (dtype == FAQ_BF16) launch_qdq<__hip_bfloat16>(a, levels, threads, st);
  else launch_qdq<__half>(a, levels, threads, st);
  return check_launch("faq_hif4_qdq_rows");
}

int faq_hadamard_rows(const void* x, void* y, int64_t rows, int64_t cols, int block, int in_dtype, int out_dtype,
                      faq_stream_t stream) {
  if (rows < 0) return fail(FAQ_EINVAL, "faq_hadamard_rows: negative size");
  if ((!x || !y) && rows > 0) return fail(FAQ_EINVAL, "faq_hadamard_rows: null input or output");
  if (block < 2 || block > 512 || (block & (block - 1)))
    return fail(FAQ_EINVAL, "Hadamard dimension must be a power of two, got %d", block);
  if (cols <= 0 || cols % block)
    return fail(FAQ_EINVAL, "dimension %lld must be divisible by power-of-two block_size=%d",
                static_cast<long long>(cols), block);
  if (cols % 8) return fail(FAQ_EUNSUP, "faq_hadamard_rows: row width must be a multiple of 8");
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype)) return fail(FAQ_EINVAL, "faq_hadamard_rows: bad dtype");
  if (!aligned16(x) || !aligned16(y)) return fail(FAQ_EINVAL, "faq_hadamard_rows: pointers must be 16-byte aligned");
  if (rows == 0) return FAQ_OK;
  faq::HadamardRowsArgs a{x, y, rows, cols, block, sqrt_div(block)};
  const int64_t threads = rows * (cols / 8);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == FAQ_F32) launch_hadamard_in<float>(a, out_dtype, threads, st);
  else if (in_dtype == FAQ_BF16) launch_hadamard_in<__hip_bfloat16>(a, out_dtype, threads, st);
  else launch_hadamard_in<__half>(a, out_dtype, threads, st);
  return check_launch("faq_hadamard_rows");
}

int faq_hadamard_rows_native(const void* x, void* y, int64_t rows, int64_t cols, int dtype, faq_stream_t stream) {
  if (rows < 0) return fail(FAQ_EINVAL, "faq_hadamard_rows_native: negative size");
  if ((!x || !y) && rows > 0) return fail(FAQ_EINVAL, "faq_hadamard_rows_native: null input or output");
  if (cols < 2 || cols > 512 || (cols & (cols - 1)))
    return fail(cols > 512 && !(cols & (cols - 1)) ? FAQ_EUNSUP : FAQ_EINVAL,
                cols > 512 && !(cols & (cols - 1)) ? "faq_hadamard_rows_native: dimension %lld above 512"
                                                   : "Hadamard dimension must be a power of two, got %lld",
                static_cast<long long>(cols));
  if (cols % 8) return fail(FAQ_EUNSUP, "faq_hadamard_rows_native: row width must be a multiple of 8");
  if (dtype != FAQ_BF16 && dtype != FAQ_F16) return fail(FAQ_EINVAL, "faq_hadamard_rows_native: dtype must be bf16 or fp16");
  if (rows < 0) return fail(FAQ_EINVAL, "faq_hadamard_rows_native: negative size");
  if (!aligned16(x) || !aligned16(y)) return fail(FAQ_EINVAL, "faq_hadamard_rows_native: pointers must be 16-byte aligned");
  if (rows == 0) return FAQ_OK;
  const int n = static_cast<int>(cols);
  faq::HadamardRowsArgs a{x, y, rows, cols, n, sqrt_div(n)};
  const dim3 grid(grid_for(rows * (cols / 8)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FAQ_BF16)
    hipLaunchKernelGGL((faq::hadamard_rows_kernel<__hip_bfloat16, __hip_bfloat16, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((faq::hadamard_rows_kernel<__half, __half, true>), grid, dim3(256), 0, st, a);
  return check_launch("faq_hadamard_rows_native");
}

int faq_hif4_unpack_rows(const uint8_t* codes, const uint8_t* scale_byte, const uint8_t* lv2_bits,
                         const uint16_t* lv3_bits, int64_t rows, int64_t cols, int out_dtype, void* y,
                         faq_stream_t stream) {
  if (!codes || !scale_byte || !lv2_bits || !lv3_bits || !y) return fail(FAQ_EINVAL, "faq_hif4_unpack_rows: null pointer");
  if (rows < 0) return fail(FAQ_EINVAL, "faq_hif4_unpack_rows: negative size");
  if (cols <= 0 || cols % 64) return fail(FAQ_EINVAL, "HiF4 packing needs a last axis that is a multiple of 64");
  if (!valid_dtype(out_dtype)) return fail(FAQ_EINVAL, "faq_hif4_unpack_rows: bad dtype");
  if (!aligned16(y) || reinterpret_cast<uintptr_t>(codes) % 4)
    return fail(FAQ_EINVAL, "faq_hif4_unpack_rows: misaligned codes or output");
  if (rows == 0) return FAQ_OK;
  faq::UnpackArgs a{codes, scale_byte, lv2_bits, lv3_bits, y, rows, cols};
  const dim3 grid(grid_for(rows * (cols / 8)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (out_dtype == FAQ_F32) hipLaunchKernelGGL((faq::unpack_rows_kernel<float>), grid, dim3(256), 0, st, a);
  else if (out_dtype == FAQ_BF16) hipLaunchKernelGGL((faq::unpack_rows_kernel<__hip_bfloat16>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((faq::unpack_rows_kernel<__half>), grid, dim3(256), 0, st, a);
  return check_launch("faq_hif4_unpack_rows");
}

int faq_act_qdq_rows(const void* x, void* y, int64_t rows, int64_t cols, int dtype, const float* col_scale,
                     int hadamard, int levels, faq_stream_t stream) {
  if (rows < 0) return fail(FAQ_EINVAL, "faq_act_qdq_rows: negative size");
  if ((!x || !y) && rows > 0) return fail(FAQ_EINVAL, "faq_act_qdq_rows: null input or output");
  if (!valid_dtype(dtype)) return fail(FAQ_EINVAL, "faq_act_qdq_rows: bad dtype");
  if (levels != 0 && !valid_levels(levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", levels);
  if (hadamard != 0) {
    if (hadamard < 2 || hadamard > 512 || (hadamard & (hadamard - 1)))
      return fail(FAQ_EINVAL, "Hadamard dimension must be a power of two, got %d", hadamard);
    if (cols <= 0 || cols % hadamard)
      return fail(FAQ_EINVAL, "dimension %lld must be divisible by power-of-two block_size=%d",
                  static_cast<long long>(cols), hadamard);
    if (cols % 64) return fail(FAQ_EUNSUP, "faq_act_qdq_rows: a rotated row must be a multiple of 64 wide");
  }
  if (cols <= 0) return fail(FAQ_EINVAL, "HiF4 fake quantization does not support an empty axis");
  if (cols % 8) return fail(FAQ_EUNSUP, "faq_act_qdq_rows: row width must be a multiple of 8");
  if (!aligned16(x) || !aligned16(y)) return fail(FAQ_EINVAL, "faq_act_qdq_rows: pointers must be 16-byte aligned");
  if (rows == 0) return FAQ_OK;
  faq::ActQdqArgs a{x, y, rows, cols, col_scale, hadamard, sqrt_div(hadamard), levels != 0};
  const int64_t threads = rows * ((cols + 63) / 64) * 8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FAQ_F32) launch_act<float>(a, levels, threads, st);
  else if (dtype == FAQ_BF16) launch_act<__hip_bfloat16>(a, levels, threads, st);
  else launch_act<__half>(a, levels, threads, st);
  return check_launch("faq_act_qdq_rows");
}

int faq_act_prep_rows(const void* x, void* y, int64_t rows, int64_t cols, int dtype, const faq_act_opts* opts,
                      int levels, faq_stream_t stream) {
  const char* who = "faq_act_prep_rows";
  if (rows < 0) return fail(FAQ_EINVAL, "%s: negative size", who);
  if ((!x || !y) && rows > 0) return fail(FAQ_EINVAL, "%s: null input or output", who);
  if (!valid_dtype(dtype)) return fail(FAQ_EINVAL, "%s: bad dtype", who);
  if (levels != 0 && !valid_levels(levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", levels);
  if (cols <= 0) return fail(FAQ_EINVAL, "HiF4 fake quantization does not support an empty axis");
  if (cols % 64) return fail(FAQ_EUNSUP, "%s: row width must be a multiple of 64", who);
  if (cols > faq::kActMaxCols) return fail(FAQ_EUNSUP, "%s: at most %d features per row", who, faq::kActMaxCols);
  if (rows > 0x7FFFFFFF) return fail(FAQ_EUNSUP, "%s: too many rows", who);
  if (!aligned16(x) || !aligned16(y)) return fail(FAQ_EINVAL, "%s: pointers must be 16-byte aligned", who);
  faq_act_opts o{};
  if (opts) o = *opts;
  auto check_block = [&](int b) -> int {
    if (b == 0) return FAQ_OK;
    if (b < 2 || (b & (b - 1))) return fail(FAQ_EINVAL, "Hadamard dimension must be a power of two, got %d", b);
    if (cols % b)
      return fail(FAQ_EINVAL, "dimension %lld must be divisible by power-of-two block_size=%d", static_cast<long long>(cols), b);
    return FAQ_OK;
  };
  if (!aligned16(o.col_scale) || !aligned16(o.rot_perm) || !aligned16(o.compand) || !aligned16(o.rot_signs) ||
      !aligned16(o.compand_rcp))
    return fail(FAQ_EINVAL, "%s: the input scale, sign, permutation and companding vectors must be 16-byte aligned", who);
  if (o.compand_rcp && !o.compand) return fail(FAQ_EINVAL, "%s: a companding reciprocal needs the companding scale", who);
  if (o.rot_signs && !o.rot_perm) return fail(FAQ_EINVAL, "%s: a rotation needs both signs and permutation", who);
  if (!o.rot_signs && (o.rot_perm || o.rot_block)) return fail(FAQ_EINVAL, "%s: a rotation needs both signs and permutation", who);
  if (int st = check_block(o.rot_block)) return st;
  if (int st = check_block(o.hadamard)) return st;
  int online = o.hadamard, gen12 = 0;
  if (o.hadamard_generalized) {
    if (o.hadamard) return fail(FAQ_EINVAL, "%s: a block Hadamard and the generalized one are exclusive", who);
    const int64_t b = cols % 12 ? 0 : cols / 12;
    if (!(cols & (cols - 1))) {
      online = static_cast<int>(cols);
    } else if (b > 0 && !(b & (b - 1))) {
      online = static_cast<int>(b);
      gen12 = 1;
    } else {
      return fail(FAQ_EINVAL, "unsupported generalized Hadamard dimension: %lld", static_cast<long long>(cols));
    }
  }
  if (rows == 0) return FAQ_OK;
  faq::ActRowArgs a{};
  a.x = x;
  a.y = y;
  a.rows = rows;
  a.cols = static_cast<int>(cols);
  a.col_scale = o.col_scale;
  a.rot_signs = o.rot_signs;
  a.rot_perm = o.rot_perm;
  a.rot_block = o.rot_block;
  a.rot_div = sqrt_div(o.rot_block);
  a.has_min = o.has_min != 0;
  a.has_max = o.has_max != 0;
  a.act_min = o.act_min;
  a.act_max = o.act_max;
  a.compand = o.compand;
  a.compand_rcp = o.compand_rcp;
  a.stage_round = o.stage_round != 0;
  if (a.stage_round && (levels != 0 || o.col_scale || o.rot_signs || o.has_min || o.has_max || o.compand))
    return fail(FAQ_EUNSUP, "%s: the in-dtype transform (stage_round) takes no other step", who);
  a.n = online;
  a.gen12 = gen12;
  a.div = sqrt_div(gen12 ? static_cast<int>(cols) : online);
  a.quant = levels != 0;
  const bool uses_lds = o.rot_signs || o.rot_block > 8 || online > 8;
  const size_t lds = uses_lds ? faq::act_row_lds_bytes(a.cols) : 0;
  if (lds > device_lds_per_block())
    return fail(FAQ_EUNSUP, "%s: a row of %lld features needs %zu bytes of LDS, the device has %zu", who,
                static_cast<long long>(cols), lds, device_lds_per_block());
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FAQ_F32) launch_act_row<float>(a, levels, lds, st);
  else if (dtype == FAQ_BF16) launch_act_row<__hip_bfloat16>(a, levels, lds, st);
  else launch_act_row<__half>(a, levels, lds, st);
  return check_launch(who);
}

int faq_act_compand_rcp(const float* compand, float* rcp, int64_t n, int dtype, faq_stream_t stream) {
  const char* who = "faq_act_compand_rcp";
  if (n < 0) return fail(FAQ_EINVAL, "%s: negative size", who);
  if ((!compand || !rcp) && n > 0) return fail(FAQ_EINVAL, "%s: null input or output", who);
  if (!valid_dtype(dtype)) return fail(FAQ_EINVAL, "%s: bad dtype", who);
  if (n == 0) return FAQ_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  if (dtype == FAQ_F32) hipLaunchKernelGGL(faq::compand_rcp_kernel<float>, grid, dim3(256), 0, st, compand, rcp, n);
  else if (dtype == FAQ_BF16)
    hipLaunchKernelGGL(faq::compand_rcp_kernel<__hip_bfloat16>, grid, dim3(256), 0, st, compand, rcp, n);
  else hipLaunchKernelGGL(faq::compand_rcp_kernel<__half>, grid, dim3(256), 0, st, compand, rcp, n);
  return check_launch(who);
}

int faq_operand_prep(const void* x, int in_dtype, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                     const float* key_offset, int64_t off_sh, const float* smooth, int64_t smooth_sh,
                     int smooth_divide, int hadamard, int round_dtype, void* rotated, void* y, int64_t yb,
                     int64_t yh, int64_t yl, int levels, faq_stream_t stream) {
  if (!x || !y) return fail(FAQ_EINVAL, "faq_operand_prep: null input or output");
  if (B < 0 || H < 0 || L < 0) return fail(FAQ_EINVAL, "faq_operand_prep: negative size");
  if (!valid_dtype(in_dtype) || !valid_dtype(round_dtype)) return fail(FAQ_EINVAL, "faq_operand_prep: bad dtype");
  if (hadamard != 0 && hadamard != 64 && hadamard != 128)
    return fail(FAQ_EUNSUP, "faq_operand_prep: Hadamard block must be 64 or 128, got %d", hadamard);
  if (levels != 0 && !valid_levels(levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", levels);
  if (!aligned16(x) || !aligned16(y)) return fail(FAQ_EINVAL, "faq_operand_prep: pointers must be 16-byte aligned");
  const int esz = in_dtype == FAQ_F32 ? 4 : 2;
  if ((sb * esz) % 16 || (sh * esz) % 16 || (sl * esz) % 16 || (yb * 2) % 16 || (yh * 2) % 16 || (yl * 2) % 16)
    return fail(FAQ_EINVAL, "faq_operand_prep: strides must keep 16-byte alignment");
  const int64_t rows = static_cast<int64_t>(B) * H * L;
  if (rows == 0) return FAQ_OK;
  if (B > 65535 || H > 65535) return fail(FAQ_EUNSUP, "faq_operand_prep: at most 65535 batches and heads");
  faq::OperandPrepArgs a{};
  a.x = x;
  a.sb = sb;
  a.sh = sh;
  a.sl = sl;
  a.B = B;
  a.H = H;
  a.L = L;
  a.key_offset = key_offset;
  a.off_sh = off_sh;
  a.smooth = smooth;
  a.smooth_sh = smooth_sh;
  a.smooth_divide = smooth_divide;
  a.hadamard = hadamard;
  a.div = sqrt_div(hadamard);
  a.rotated = rotated;
  a.y = y;
  a.yb = yb;
  a.yh = yh;
  a.yl = yl;
  a.quant = levels != 0;
  const int64_t threads = rows * 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == FAQ_F32) launch_prep_in<float>(a, round_dtype, levels, threads, st);
  else if (in_dtype == FAQ_BF16) launch_prep_in<__hip_bfloat16>(a, round_dtype, levels, threads, st);
  else launch_prep_in<__half>(a, round_dtype, levels, threads, st);
  return check_launch("faq_operand_prep");
}

int faq_operand_prep_vt(const void* x, int in_dtype, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                        int Lpad, uint16_t* vt, int levels, faq_stream_t stream) {
  if (!x || !vt) return fail(FAQ_EINVAL, "faq_operand_prep_vt: null input or output");
  if (B < 0 || H < 0 || L < 0) return fail(FAQ_EINVAL, "faq_operand_prep_vt: negative size");
  if (Lpad % 128 || Lpad < L) return fail(FAQ_EINVAL, "faq_operand_prep_vt: Lpad must be a multiple of 128 >= L");
  if (!valid_dtype(in_dtype)) return fail(FAQ_EINVAL, "faq_operand_prep_vt: bad dtype");
  if (levels != 0 && !valid_levels(levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", levels);
  if (!aligned16(x) || !aligned16(vt)) return fail(FAQ_EINVAL, "faq_operand_prep_vt: pointers must be 16-byte aligned");
  const int esz = in_dtype == FAQ_F32 ? 4 : 2;
  if ((sb * esz) % 16 || (sh * esz) % 16 || (sl * esz) % 16)
    return fail(FAQ_EINVAL, "faq_operand_prep_vt: strides must keep 16-byte alignment");
  if (static_cast<int64_t>(B) * H * Lpad == 0) return FAQ_OK;
  faq::OperandPrepVtArgs a{x, sb, sh, sl, B, H, L, Lpad, vt, levels != 0};
  const dim3 grid(Lpad / 64, B * H);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == FAQ_F32) launch_prep_vt<float>(a, levels, grid, st);
  else if (in_dtype == FAQ_BF16) launch_prep_vt<__hip_bfloat16>(a, levels, grid, st);
  else launch_prep_vt<__half>(a, levels, grid, st);
  return check_launch("faq_operand_prep_vt");
}

int faq_attention_fwd(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k, int64_t k_sb,
                      int64_t k_sh, int64_t k_sl, const uint16_t* vt, int64_t v_sb, int64_t v_sh, int64_t v_sd,
                      int Lpad, void* o, int o_dtype, int64_t o_sb, int64_t o_sh, int64_t o_sl, int B, int Hq,
                      int Hkv, int Lq, int Lk, int causal, float scale, int quant_p, int p_levels, int norm_same,
                      float* row_den, int out_levels, const faq_attn_opts* opts, faq_stream_t stream) {
  faq::AttnArgs a;
  dim3 grid;
  const int rc = attention_setup("faq_attention_fwd", q, q_sb, q_sh, q_sl, k, k_sb, k_sh, k_sl, vt, v_sb, v_sh, v_sd,
                                 Lpad, o, o_dtype, o_sb, o_sh, o_sl, B, Hq, Hkv, Lq, Lk, causal, scale, quant_p,
                                 p_levels, row_den, out_levels, opts, a, grid);
  if (rc != FAQ_OK) return rc == 1 ? FAQ_OK : rc;
  // XCD pacing epoch: nonzero and new per launch; off on a stream being captured (a recorded
  // launch would reuse its epoch's counters on every replay)
  {
    static std::atomic<uint32_t> pace_epochs{0};
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &capture) != hipSuccess ||
                           capture != hipStreamCaptureStatusNone;
    uint32_t e = 0;
    const char* pace_env = std::getenv("FAQ_ATTN_PACE");  // test hook: 0 turns pacing off
    if (!capturing && !(pace_env && pace_env[0] == '0')) {
      do e = ++pace_epochs; while (e == 0);
    }
    a.pace_epoch = e;
    const char* lead_env = std::getenv("FAQ_ATTN_PACE_LEAD");  // test hook: the lead in tiles
    a.pace_lead = lead_env ? std::max(1, std::atoi(lead_env)) : faq::kPaceLead;
  }
  launch_attention(a, quant_p, p_levels, norm_same, grid, static_cast<hipStream_t>(stream));
  return check_launch("faq_attention_fwd");
}

int faq_attention_mask_bounds(const uint8_t* mask, int64_t mask_sb, int B, int Lq, int Lk, int causal, int window,
                              int32_t* row_lo, int32_t* row_hi, int32_t* row_blocks, uint32_t* key_bits,
                              int64_t key_words, faq_stream_t stream) {
  if (!row_lo || !row_hi || !row_blocks) return fail(FAQ_EINVAL, "faq_attention_mask_bounds: null output");
  if (B < 0 || Lq < 0 || Lk < 0) return fail(FAQ_EINVAL, "faq_attention_mask_bounds: bad sizes");
  if (window < 0) return fail(FAQ_EINVAL, "sliding_window must be positive");
  if (Lk > 32 * faq::kMaskMaxWords)
    return fail(FAQ_EUNSUP, "faq_attention_mask_bounds: at most %d keys", 32 * faq::kMaskMaxWords);
  if (key_bits && key_words < 4 * ((static_cast<int64_t>(Lk) + 127) / 128))
    return fail(FAQ_EINVAL, "faq_attention_mask_bounds: key_words must be >= 4 * ceil(Lk / 128)");
  if (mask && mask_sb < Lk) return fail(FAQ_EINVAL, "faq_attention_mask_bounds: mask row stride < Lk");
  if (B == 0 || (Lq == 0 && !key_bits)) return FAQ_OK;
  faq::MaskBoundsArgs a{mask, mask_sb, Lq, Lk, causal != 0, window, row_lo, row_hi, row_blocks, key_bits, key_words};
  hipLaunchKernelGGL(faq::mask_bounds_kernel, dim3(static_cast<unsigned>(B)), dim3(faq::kMaskThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("faq_attention_mask_bounds");
}

int64_t faq_attention_split_workspace(int B, int Hq, int Lq, int Lk, int nsplit) {
  if (B < 0 || Hq < 0 || Lq < 0 || Lk < 0 || nsplit < 1) return -1;
  return split_layout(B, Hq, Lq, Lk, nsplit).total;
}

int faq_attention_fwd_split(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                            int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* vt, int64_t v_sb, int64_t v_sh,
                            int64_t v_sd, int Lpad, void* o, int o_dtype, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                            int B, int Hq, int Hkv, int Lq, int Lk, int causal, float scale, int quant_p,
                            int p_levels, int norm_same, float* row_den, int nsplit, void* workspace,
                            int64_t workspace_bytes, const faq_attn_opts* opts, faq_stream_t stream) {
  if (nsplit < 1 || nsplit > faq::kCombineMaxSplits)
    return fail(FAQ_EINVAL, "faq_attention_fwd_split: nsplit must be in [1, %d]", faq::kCombineMaxSplits);
  faq::AttnArgs a;
  dim3 grid;
  const int rc = attention_setup("faq_attention_fwd_split", q, q_sb, q_sh, q_sl, k, k_sb, k_sh, k_sl, vt, v_sb, v_sh,
                                 v_sd, Lpad, o, o_dtype, o_sb, o_sh, o_sl, B, Hq, Hkv, Lq, Lk, causal, scale, quant_p,
                                 p_levels, row_den, 0, opts, a, grid);
  if (rc != FAQ_OK) return rc == 1 ? FAQ_OK : rc;
  if (a.diag || a.p_dump)
    return fail(FAQ_EINVAL, "faq_attention_fwd_split: the PV-normalizer probe and the P dump run in faq_attention_fwd");
  const SplitLayout L = split_layout(B, Hq, Lq, Lk, nsplit);
  if (L.ntiles > faq::kScanMaxTiles)
    return fail(FAQ_EUNSUP, "faq_attention_fwd_split: %d key tiles, the split path handles at most %d", L.ntiles,
                faq::kScanMaxTiles);
  if (!workspace || !aligned16(workspace)) return fail(FAQ_EINVAL, "faq_attention_fwd_split: null or misaligned workspace");
  if (workspace_bytes < L.total)
    return fail(FAQ_EINVAL, "faq_attention_fwd_split: workspace of %lld bytes, need %lld",
                static_cast<long long>(workspace_bytes), static_cast<long long>(L.total));
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  grid.x = static_cast<unsigned>(workers_for(n_items_of(a), nsplit));
  grid.z = static_cast<unsigned>(nsplit);
  a.tiles_per_split = L.tiles_per_split;
  // 1. c1-scaled tile maxima of every row
  faq::AttnArgs am = a;
  am.mx_out = reinterpret_cast<float*>(ws + L.mx);
  am.mx_stride = std::max(L.ntiles, 1);
  launch_attention(am, quant_p, p_levels, norm_same, grid, st);
  // 2. running maximum before each split
  faq::SplitScanArgs sa{am.mx_out, am.mx_stride, L.ntiles, reinterpret_cast<float*>(ws + L.m_start), a.rows_total,
                        nsplit, L.tiles_per_split, Hq, Lq, Lk, a.causal, a.row_lo, a.row_hi};
  hipLaunchKernelGGL(faq::split_scan_kernel, dim3(static_cast<unsigned>(a.rows_total)), dim3(faq::kScanThreads),
                     static_cast<size_t>(std::max(L.ntiles, 1)) * sizeof(float), st, sa);
  // 3. per-split recurrences from those maxima
  faq::AttnArgs ap = a;
  ap.m_start = sa.m_start;
  ap.part_o = reinterpret_cast<float*>(ws + L.part_o);
  ap.part_lm = reinterpret_cast<float*>(ws + L.part_lm);
  launch_attention(ap, quant_p, p_levels, norm_same, grid, st);
  // 4. combine
  faq::SplitCombineArgs ca{ap.part_o, ap.part_lm, a.rows_total, nsplit, Hq, Lq, o, o_sb, o_sh, o_sl, a.o_f32, row_den};
  faq::launch_split_combine(ca, st);
  return check_launch("faq_attention_fwd_split");
}

int faq_attention_fwd_split_noalloc(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                                    int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* vt, int64_t v_sb,
                                    int64_t v_sh, int64_t v_sd, int Lpad, void* o, int o_dtype, int64_t o_sb,
                                    int64_t o_sh, int64_t o_sl, int B, int Hq, int Hkv, int Lq, int Lk, int causal,
                                    float scale, int quant_p, int p_levels, int norm_same, float* row_den,
                                    int nsplit, const faq_attn_opts* opts, faq_stream_t stream) {
  if (nsplit < 1 || nsplit > faq::kCombineMaxSplits)
    return fail(FAQ_EINVAL, "faq_attention_fwd_split_noalloc: nsplit must be in [1, %d]", faq::kCombineMaxSplits);
  if (B < 0 || Hq <= 0 || Lq < 0 || Lk < 0) return fail(FAQ_EINVAL, "faq_attention_fwd_split_noalloc: bad sizes");
  const int64_t need = split_layout(B, Hq, Lq, Lk, nsplit).total;
  if (need > FAQ_NOALLOC_SCRATCH_BYTES)
    return fail(FAQ_EINVAL,
                "faq_attention_fwd_split_noalloc: this call needs %lld bytes of scratch, the static buffer holds %lld "
                "(use faq_attention_fwd_split with a workspace)",
                static_cast<long long>(need), static_cast<long long>(FAQ_NOALLOC_SCRATCH_BYTES));
  if (stream) {
    // the scratch address belongs to the current device: the stream must run there
    hipDevice_t sdev = -1;
    int cur = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess || hipGetDevice(&cur) != hipSuccess ||
        sdev != cur)
      return fail(FAQ_EINVAL, "faq_attention_fwd_split_noalloc: the stream's device must be the current device");
  }
  void* ws = noalloc_scratch();
  if (!ws) return FAQ_ELAUNCH;
  return faq_attention_fwd_split(q, q_sb, q_sh, q_sl, k, k_sb, k_sh, k_sl, vt, v_sb, v_sh, v_sd, Lpad, o, o_dtype,
                                 o_sb, o_sh, o_sl, B, Hq, Hkv, Lq, Lk, causal, scale, quant_p, p_levels, norm_same,
                                 row_den, nsplit, ws, FAQ_NOALLOC_SCRATCH_BYTES, opts, stream);
}

int faq_operand_prep_hif4_kv(const void* x, int in_dtype, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                             const float* key_offset, int64_t off_sh, const float* smooth, int64_t smooth_sh,
                             int smooth_divide, int hadamard, int round_dtype, int levels, uint32_t* codes,
                             uint32_t* meta, int64_t p_sb, int64_t p_sh, faq_stream_t stream) {
  if (!x || !codes || !meta) return fail(FAQ_EINVAL, "faq_operand_prep_hif4_kv: null input or output");
  if (B < 0 || H < 0 || L < 0) return fail(FAQ_EINVAL, "faq_operand_prep_hif4_kv: negative size");
  if (!valid_dtype(in_dtype) || !valid_dtype(round_dtype)) return fail(FAQ_EINVAL, "faq_operand_prep_hif4_kv: bad dtype");
  if (hadamard != 0 && hadamard != 64 && hadamard != 128)
    return fail(FAQ_EUNSUP, "faq_operand_prep_hif4_kv: Hadamard block must be 64 or 128, got %d", hadamard);
  if (!valid_levels(levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", levels);
  if (!aligned16(x)) return fail(FAQ_EINVAL, "faq_operand_prep_hif4_kv: x must be 16-byte aligned");
  if (!aligned16(codes) || (reinterpret_cast<uintptr_t>(meta) & 7u))
    return fail(FAQ_EINVAL, "faq_operand_prep_hif4_kv: codes must be 16-byte and meta 8-byte aligned");
  const int esz = in_dtype == FAQ_F32 ? 4 : 2;
  if ((sb * esz) % 16 || (sh * esz) % 16 || (sl * esz) % 16)
    return fail(FAQ_EINVAL, "faq_operand_prep_hif4_kv: strides must keep 16-byte alignment");
  if (p_sb < 0 || p_sh < 0) return fail(FAQ_EINVAL, "faq_operand_prep_hif4_kv: negative row strides");
  const int64_t rows = static_cast<int64_t>(B) * H * L;
  if (rows == 0) return FAQ_OK;
  if (B > 65535 || H > 65535) return fail(FAQ_EUNSUP, "faq_operand_prep_hif4_kv: at most 65535 batches and heads");
  faq::OperandPrepArgs a{};
  a.x = x;
  a.sb = sb;
  a.sh = sh;
  a.sl = sl;
  a.B = B;
  a.H = H;
  a.L = L;
  a.key_offset = key_offset;
  a.off_sh = off_sh;
  a.smooth = smooth;
  a.smooth_sh = smooth_sh;
  a.smooth_divide = smooth_divide;
  a.hadamard = hadamard;
  a.div = sqrt_div(hadamard);
  a.quant = 1;
  a.pk_codes = codes;
  a.pk_meta = meta;
  a.pk_sb = p_sb;
  a.pk_sh = p_sh;
  const int64_t threads = rows * 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == FAQ_F32) launch_prep_in<float>(a, round_dtype, levels, threads, st);
  else if (in_dtype == FAQ_BF16) launch_prep_in<__hip_bfloat16>(a, round_dtype, levels, threads, st);
  else launch_prep_in<__half>(a, round_dtype, levels, threads, st);
  return check_launch("faq_operand_prep_hif4_kv");
}

int64_t faq_attention_decode_workspace(int B, int Hq, int Lq, int Lk, int nsplit) {
  if (B < 0 || Hq < 0 || Lq < 0 || Lk < 0 || nsplit < 1) return -1;
  return decode_layout(B, Hq, Lq, Lk, nsplit).total;
}

int faq_attention_decode(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                         int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* v, int64_t v_sb, int64_t v_sh,
                         int64_t v_sl, const faq_hif4_kv* kp, const faq_hif4_kv* vp, void* o, int o_dtype,
                         int64_t o_sb, int64_t o_sh, int64_t o_sl, int B, int Hq, int Hkv, int Lq, int Lk, int causal,
                         float scale, int quant_p, int p_levels, int norm_same, float* row_den, int nsplit,
                         void* workspace, int64_t workspace_bytes, faq_stream_t stream) {
  const char* who = "faq_attention_decode";
  const bool packed = kp != nullptr;
  if ((kp == nullptr) != (vp == nullptr)) return fail(FAQ_EINVAL, "%s: K and V are both packed or both bf16", who);
  if (!q || !o) return fail(FAQ_EINVAL, "%s: null operand", who);
  if (packed ? !(kp->codes && kp->meta && vp->codes && vp->meta) : !(k && v))
    return fail(FAQ_EINVAL, "%s: null operand", who);
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Lq < 0 || Lk < 0) return fail(FAQ_EINVAL, "%s: bad sizes", who);
  if (Hq % Hkv) return fail(FAQ_EINVAL, "query heads must be divisible by key/value heads");
  if (Hq / Hkv > 32) return fail(FAQ_EUNSUP, "%s: at most 32 query heads per key/value head", who);
  if (nsplit < 1 || nsplit > faq::kCombineMaxSplits)
    return fail(FAQ_EINVAL, "%s: nsplit must be in [1, %d]", who, faq::kCombineMaxSplits);
  if (o_dtype != FAQ_F32 && o_dtype != FAQ_BF16) return fail(FAQ_EUNSUP, "%s: output must be fp32 or bf16", who);
  if (quant_p && !valid_levels(p_levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", p_levels);
  if (!aligned16(q) || !aligned16(o)) return fail(FAQ_EINVAL, "%s: pointers must be 16-byte aligned", who);
  if ((q_sb | q_sh | q_sl) & 7) return fail(FAQ_EINVAL, "%s: operand strides must be multiples of 8 elements", who);
  if ((o_sb | o_sh | o_sl) & 3) return fail(FAQ_EINVAL, "%s: output strides must be multiples of 4 elements", who);
  const DecodeLayout L = decode_layout(B, Hq, Lq, Lk, nsplit);
  if (packed) {
    if (!aligned16(kp->codes) || !aligned16(vp->codes) || (reinterpret_cast<uintptr_t>(kp->meta) & 7u) ||
        (reinterpret_cast<uintptr_t>(vp->meta) & 7u))
      return fail(FAQ_EINVAL, "%s: packed codes must be 16-byte and meta 8-byte aligned", who);
    if (kp->sb < 0 || kp->sh < 0 || vp->sb < 0 || vp->sh < 0) return fail(FAQ_EINVAL, "%s: negative row strides", who);
  } else {
    if (!aligned16(k) || !aligned16(v)) return fail(FAQ_EINVAL, "%s: pointers must be 16-byte aligned", who);
    if ((k_sb | k_sh | k_sl | v_sb | v_sh | v_sl) & 7)
      return fail(FAQ_EINVAL, "%s: operand strides must be multiples of 8 elements", who);
  }
  if (B == 0 || Lq == 0) return FAQ_OK;
  if (!workspace || !aligned16(workspace)) return fail(FAQ_EINVAL, "%s: null or misaligned workspace", who);
  if (workspace_bytes < L.total)
    return fail(FAQ_EINVAL, "%s: workspace of %lld bytes, need %lld", who, static_cast<long long>(workspace_bytes),
                static_cast<long long>(L.total));
  const int G = Hq / Hkv;
  faq::DecodeArgs a{};
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_sl = q_sl;
  if (packed) {
    a.kc = kp->codes;
    a.km = kp->meta;
    a.kp_sb = kp->sb;
    a.kp_sh = kp->sh;
    a.vc = vp->codes;
    a.vm = vp->meta;
    a.vp_sb = vp->sb;
    a.vp_sh = vp->sh;
  } else {
    a.k = k;
    a.k_sb = k_sb;
    a.k_sh = k_sh;
    a.k_sl = k_sl;
    a.v = v;
    a.v_sb = v_sb;
    a.v_sh = v_sh;
    a.v_sl = v_sl;
  }
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Lq = Lq;
  a.Lk = Lk;
  a.causal = causal != 0;
  a.c1 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  a.G = G;
  a.pb = 32 / G;
  a.n_rb = (Lq + a.pb - 1) / a.pb;
  a.ntiles = L.ntiles;
  a.tps = L.tps;
  a.nsplit = nsplit;
  a.rows_total = B * Hq * Lq;
  char* ws = static_cast<char*>(workspace);
  a.s = reinterpret_cast<float*>(ws + L.s);
  a.s_stride = static_cast<int64_t>(L.ntiles) * 128;
  a.gmx = reinterpret_cast<float*>(ws + L.gmx);
  a.smx = reinterpret_cast<float*>(ws + L.smx);
  a.part_o = reinterpret_cast<float*>(ws + L.part_o);
  a.part_lm = reinterpret_cast<float*>(ws + L.part_lm);
  const int64_t waves = static_cast<int64_t>(B) * Hkv * a.n_rb * nsplit;
  if (waves > static_cast<int64_t>(INT32_MAX) - faq::kDecWaves) return fail(FAQ_EUNSUP, "%s: too many work items", who);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the one-pass form where it applies.  Test hooks: FAQ_DECODE_FUSED=0 keeps the two
  // passes, =force requires the one pass (FAQ_EUNSUP where it does not apply);
  // FAQ_DECODE_SPIN sets the look-back's wait bound (negative: every earlier split's
  // maxima computed in the wave)
  const char* fused_env = std::getenv("FAQ_DECODE_FUSED");
  // The one pass tells its published maxima from an earlier call's by an epoch passed at
  // launch.  A launch recorded into a HIP graph keeps its epoch on every replay, so a replay
  // could accept the maxima a previous replay left; calls on a capturing stream (or where
  // the capture state cannot be read) take the two passes, which carry no state between
  // calls.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  const bool capturing = hipStreamIsCapturing(st, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone;
  const bool fits = faq::decode_fused_fits(a, quant_p, norm_same) && !capturing;
  if (fused_env && std::strcmp(fused_env, "force") == 0 && !fits)
    return fail(FAQ_EUNSUP, "%s: the one-pass decode does not apply to this call", who);
  if (!(fused_env && fused_env[0] == '0') && fits) {
    const char* spin_env = std::getenv("FAQ_DECODE_SPIN");
    const int spin = spin_env ? std::atoi(spin_env) : 4096;
    static std::atomic<uint32_t> epochs{0};
    uint32_t epoch = ++epochs;
    if (epoch == 0) epoch = ++epochs;
    faq::launch_decode_fused(a, packed ? 1 : 0, p_levels, epoch, spin, st);
  } else {
    faq::launch_decode(a, packed ? 1 : 0, quant_p, p_levels, norm_same, st);
  }
  faq::SplitCombineArgs ca{a.part_o, a.part_lm, a.rows_total, nsplit, Hq, Lq, o, o_sb, o_sh, o_sl,
                           o_dtype == FAQ_F32, row_den};
  faq::launch_split_combine(ca, st);
  return check_launch(who);
}

int faq_attention_fwd_general(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_sl, const void* k,
                              int k_dtype, int64_t k_sb, int64_t k_sh, int64_t k_sl, const void* v, int v_dtype,
                              int64_t v_sb, int64_t v_sh, int64_t v_sl, void* o, int o_dtype, int64_t o_sb,
                              int64_t o_sh, int64_t o_sl, int B, int Hq, int Hkv, int Lq, int Lk, int D, int key_tile,
                              int causal, float scale, int quant_p, int p_levels, int norm_same, float* row_den,
                              const faq_attn_opts* opts, faq_stream_t stream) {
  const char* who = "faq_attention_fwd_general";
  if (B < 0 || Hq < 1 || Hkv < 1 || Lq < 0 || Lk < 1) return fail(FAQ_EINVAL, "%s: bad sizes", who);
  if (Hq % Hkv) return fail(FAQ_EINVAL, "%s: query heads must be divisible by key/value heads", who);
  if (D < 1 || D > faq::kGenMaxDim) return fail(FAQ_EUNSUP, "%s: head_dim must lie in [1, %d], got %d", who, faq::kGenMaxDim, D);
  if (key_tile < 1 || key_tile > faq::kGenMaxTile)
    return fail(FAQ_EUNSUP, "%s: key tiles must hold 1 to %d keys, got %d", who, faq::kGenMaxTile, key_tile);
  if (B > 65535 || Hq > 65535) return fail(FAQ_EUNSUP, "%s: at most 65535 batches and query heads", who);
  for (int dt : {q_dtype, k_dtype, v_dtype, o_dtype})
    if (!valid_dtype(dt)) return fail(FAQ_EUNSUP, "%s: operands and output must be fp32, bf16 or fp16", who);
  if (quant_p && !valid_levels(p_levels)) return fail(FAQ_EINVAL, "%s: bad P levels %d", who, p_levels);
  if (!(scale == scale)) return fail(FAQ_EINVAL, "%s: scale is NaN", who);
  if (B == 0 || Lq == 0) return FAQ_OK;
  if (!q || !k || !v || !o) return fail(FAQ_EINVAL, "%s: null operand", who);
  faq::GenAttnArgs a{};
  a.q = q;
  a.q_dt = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_sl = q_sl;
  a.k = k;
  a.k_dt = k_dtype;
  a.k_sb = k_sb;
  a.k_sh = k_sh;
  a.k_sl = k_sl;
  a.v = v;
  a.v_dt = v_dtype;
  a.v_sb = v_sb;
  a.v_sh = v_sh;
  a.v_sl = v_sl;
  a.o = o;
  a.o_dt = o_dtype;
  a.o_sb = o_sb;
  a.o_sh = o_sh;
  a.o_sl = o_sl;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.Lq = Lq;
  a.Lk = Lk;
  a.D = D;
  a.T = key_tile;
  a.causal = causal != 0;
  a.scale = scale;
  a.quant_p = quant_p != 0;
  a.p_levels = quant_p ? p_levels : 123;
  a.norm_same = norm_same != 0;
  a.row_den = row_den;
  if (opts) {
    if (opts->p_dump || opts->q_prep) return fail(FAQ_EUNSUP, "%s: p_dump and q_prep are options of faq_attention_fwd", who);
    if (opts->softcap < 0.0f || !(opts->softcap == opts->softcap)) return fail(FAQ_EINVAL, "%s: bad softcap", who);
    a.softcap = opts->softcap;
    const bool any_range = opts->row_lo || opts->row_hi || opts->key_bits;
    if (any_range && !(opts->row_lo && opts->row_hi && opts->key_bits))
      return fail(FAQ_EINVAL, "%s: row_lo, row_hi and key_bits go together", who);
    if (any_range && opts->key_words < (static_cast<int64_t>(Lk) + 31) / 32)
      return fail(FAQ_EINVAL, "%s: key_words must cover every key", who);
    if (any_range && opts->dense_mask) return fail(FAQ_EINVAL, "%s: a dense mask and key ranges are exclusive", who);
    a.row_lo = opts->row_lo;
    a.row_hi = opts->row_hi;
    a.key_bits = opts->key_bits;
    a.key_words = opts->key_words;
    a.amask = opts->dense_mask;
    a.am_sb = opts->dm_sb;
    a.am_sh = opts->dm_sh;
    a.am_sq = opts->dm_sq;
    if (opts->pv_probe && !quant_p) return fail(FAQ_EINVAL, "%s: pv_probe needs quant_p", who);
    a.diag = opts->pv_probe;
  }
  const hipError_t e = faq::launch_gen_attention(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(FAQ_ELAUNCH, "%s: LDS limit of %zu bytes refused: %s", who, faq::gen_attention_lds_bytes(D, key_tile),
                hipGetErrorString(e));
  }
  return check_launch(who);
}

int faq_pquant_groups(const float* p, float* p_hat, int64_t groups, int levels, faq_stream_t stream) {
  if (groups < 0) return fail(FAQ_EINVAL, "faq_pquant_groups: negative group count");
  if (!valid_levels(levels)) return fail(FAQ_EINVAL, "HiF4 levels must be 123, 12 or 13, got %d", levels);
  if (groups == 0) return FAQ_OK;
  if (!p || !p_hat || !aligned16(p) || !aligned16(p_hat))
    return fail(FAQ_EINVAL, "faq_pquant_groups: null or misaligned pointer");
  const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (levels == 123) hipLaunchKernelGGL(faq::pquant_groups_kernel<123>, grid, dim3(256), 0, st, p, p_hat, groups);
  else if (levels == 12) hipLaunchKernelGGL(faq::pquant_groups_kernel<12>, grid, dim3(256), 0, st, p, p_hat, groups);
  else hipLaunchKernelGGL(faq::pquant_groups_kernel<13>, grid, dim3(256), 0, st, p, p_hat, groups);
  return check_launch("faq_pquant_groups");
}

int faq_hif4_linear_packed(const uint16_t* x, int64_t x_sm, const uint32_t* w_codes, const uint32_t* w_meta,
                           const void* bias, int bias_dtype, void* y, int y_dtype, int64_t y_sm, int M, int N, int K,
                           faq_stream_t stream) {
  const char* who = "faq_hif4_linear_packed";
  if (M < 0 || N < 1 || K < 1) return fail(FAQ_EINVAL, "%s: bad sizes", who);
  if (K % 128) return fail(FAQ_EUNSUP, "%s: in_features must be a multiple of 128, got %d", who, K);
  if (M > faq::kLinMaxRows) return fail(FAQ_EUNSUP, "%s: at most %d rows of x, got %d", who, faq::kLinMaxRows, M);
  if (M == 0) return FAQ_OK;
  if (!x || !w_codes || !w_meta || !y) return fail(FAQ_EINVAL, "%s: null operand", who);
  if (y_dtype != FAQ_F32 && y_dtype != FAQ_BF16) return fail(FAQ_EUNSUP, "%s: output must be fp32 or bf16", who);
  if (bias && bias_dtype != FAQ_F32 && bias_dtype != FAQ_BF16)
    return fail(FAQ_EUNSUP, "%s: bias must be fp32 or bf16", who);
  if (!aligned16(x) || x_sm < K || x_sm % 8)
    return fail(FAQ_EINVAL, "%s: x must be 16-byte aligned with a row stride >= K, a multiple of 8", who);
  if (!aligned16(w_codes) || (reinterpret_cast<uintptr_t>(w_meta) & 7u))
    return fail(FAQ_EINVAL, "%s: packed codes must be 16-byte and meta 8-byte aligned", who);
  if (y_sm < N || (reinterpret_cast<uintptr_t>(y) & (y_dtype == FAQ_F32 ? 3u : 1u)))
    return fail(FAQ_EINVAL, "%s: y must be aligned to its dtype with a row stride >= N", who);
  if (static_cast<int64_t>(N) * (K / 128) > (int64_t(1) << 40)) return fail(FAQ_EUNSUP, "%s: weight too large", who);
  faq::LinArgs a{};
  a.x = x;
  a.x_sm = x_sm;
  a.wc = w_codes;
  a.wm = w_meta;
  a.bias = bias;
  a.bias_f32 = bias_dtype == FAQ_F32;
  a.y = y;
  a.y_f32 = y_dtype == FAQ_F32;
  a.y_sm = y_sm;
  a.M = M;
  a.N = N;
  a.K = K;
  a.nkb = K / 128;
  // output features per wave: two waves per SIMD or more; per-call A/B at the Qwen3-8B shapes
  // (kernel traces): with one or two rows of x, two features per wave from N = 4096 up (gate /
  // up_proj 9.9 against 11.5 us with four); with more rows, four from N = 8192 up (16.7 against
  // 18.8 us) and two below
  int rows_per_wave = M <= 2 ? (N >= 4096 ? 2 : 1) : (N >= 8192 ? 4 : 2);
  if (const char* e = std::getenv("FAQ_LIN_RPW")) {  // test hook: 1, 2 or 4 output features per wave
    const int r = std::atoi(e);
    if (r == 1 || r == 2 || r == 4) rows_per_wave = r;
  }
  faq::launch_linear_packed(a, rows_per_wave, static_cast<hipStream_t>(stream));
  return check_launch(who);
}

int faq_mfma_probe(float* out, int blocks, int iters, faq_stream_t stream) {
  if (!out) return fail(FAQ_EINVAL, "faq_mfma_probe: null output");
  if (blocks < 1 || iters < 1) return fail(FAQ_EINVAL, "faq_mfma_probe: blocks and iters must be positive");
  hipLaunchKernelGGL(faq::mfma_probe_kernel, dim3(static_cast<unsigned>(blocks)), dim3(512), 0,
                     static_cast<hipStream_t>(stream), out, iters);
  return check_launch("faq_mfma_probe");
}

int faq_stream_probe(const void* x, int64_t bytes, float* out, int blocks, faq_stream_t stream) {
  if (!x || !out) return fail(FAQ_EINVAL, "faq_stream_probe: null input or output");
  if (!aligned16(x) || bytes < 16 || bytes % 16) return fail(FAQ_EINVAL, "faq_stream_probe: bytes must be a positive multiple of 16 at a 16-byte aligned address");
  if (blocks < 1) return fail(FAQ_EINVAL, "faq_stream_probe: blocks must be positive");
  hipLaunchKernelGGL(faq::stream_probe_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(x), bytes / 16, out);
  return check_launch("faq_stream_probe");
}

}  // extern "C"
