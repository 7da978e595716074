/*
 * faquant_amd.h -- C ABI of the MI355X (gfx950) HiF4 attention path.
 *
 * Every entry point takes raw device pointers, sizes and element strides, writes into
 * caller-allocated outputs, enqueues its kernels on the given HIP stream and returns 0
 * or a negative status (FAQ_E*).  faq_last_error() returns a thread-local message for
 * the last failure on the calling thread.  No entry point allocates device memory and
 * none synchronizes the stream; the library's only device memory of its own is two
 * file-scope arrays per GPU, loaded with the library (the scratch of
 * faq_attention_fwd_split_noalloc, 8 MiB, and the split maxima that faq_attention_decode's
 * one-pass form exchanges between waves, 4 MiB).  Pointers to float data must be 16-byte
 * aligned and rows must have a unit last-dimension stride.
 *
 * dtype codes: FAQ_F32 = 0, FAQ_BF16 = 1, FAQ_F16 = 2.
 * HiF4 levels: 123 (E6M2 per 64 + 1-bit exponents per 8 and per 4), 12, 13.
 *
 * Reference interfaces replaced (paths in MingZwhy/FAQUANT-Public):
 *   faq_hif4_qdq_rows     src/faquant/hif4.py:143-219 fit_hif4_compact_parameters,
 *                         hif4.py:377-390 fake_quantize_hif4,
 *                         src/faquant/quantization.py:30-57 fake_quantize(quant_format="hif4"),
 *                         src/faquant/wan22_attention.py:97-102 qdq_rows_128
 *   faq_hadamard_rows_native  src/faquant/rotation.py:14-29 hadamard_transform on a bf16 /
 *                         fp16 tensor (butterflies rounded to that dtype)
 *   faq_hadamard_rows     src/faquant/rotation.py:14-29 hadamard_transform,
 *                         rotation.py:117-135 chunked_block_hadamard_transform,
 *                         src/faquant/wan22_attention.py:186-192 rotate_heads
 *   faq_hif4_unpack_rows  src/faquant/hif4.py:222-271 expand_hif4_parameters +
 *                         quantize_hif4_with_parameters, from the packed 4.5-bit view
 *   faq_act_qdq_rows      src/faquant/quantization.py:204-276 FakeQuantLinear.forward (input
 *                         scale, online block Hadamard, HiF4 input QDQ) and
 *                         src/faquant/wan22_hif4.py:81-92 HiF4Linear.forward (input QDQ)
 *   faq_operand_prep      src/faquant/qwen3.py:97-136 (post-RoPE fp32 excursion: key offset,
 *                         Smooth-QK, Hadamard, one cast) and the Q/K QDQ of
 *                         src/faquant/simulated_flash_attention.py:592-619
 *   faq_operand_prep_vt   the V QDQ of simulated_flash_attention.py:600-611
 *                         (written transposed for the PV operand)
 *   faq_attention_fwd     src/faquant/simulated_flash_attention.py:457-909
 *                         simulated_flash_attention_forward (key tiles of 128; masks: none,
 *                         bottom-right causal, or key ranges + valid keys; logit softcap)
 *                         and src/faquant/wan22_attention.py:165-183 hif4_attention
 *   faq_attention_fwd_general  simulated_flash_attention.py:457-909 for any key chunk
 *                         (1..1024), head_dim 1..256 and fp32, bf16 or fp16 operands multiplied
 *                         in fp32 (sfa:723-724, 848-850: unquantized fp32 Q/K/V)
 *   faq_attention_mask_bounds  simulated_flash_attention.py:341-368 _two_dimensional_mask and
 *                         the rank form of 371-427 _streaming_mask (padding, sliding window)
 *   faq_attention_fwd_split  the same recurrence divided over key ranges (decode, where
 *                         the reference appends one position to its QDQ cache,
 *                         simulated_flash_attention.py:243-289, and runs the tile loop)
 *   faq_attention_split_workspace  workspace size of faq_attention_fwd_split
 *   faq_attention_fwd_split_noalloc  no counterpart in the reference: faq_attention_fwd_split
 *                         on a static per-GPU scratch array, for callers that cannot allocate
 *   faq_operand_prep_hif4_kv  faq_operand_prep writing the packed 4.5-bit HiF4 form (the
 *                         content of CompactHiF4Parameters, src/faquant/hif4.py:67-79) for
 *                         decode K/V caches, in place of the reference's QDQ cache tensors
 *                         (simulated_flash_attention.py:243-289)
 *   faq_attention_decode  the decode step of simulated_flash_attention.py:457-909 over that
 *                         cache (sfa:243-289): the recurrence of faq_attention_fwd_split
 *                         with the query heads of a KV head packed together, from bf16 or
 *                         packed HiF4 K/V
 *   faq_attention_decode_workspace  workspace size of faq_attention_decode
 *   faq_pquant_groups     the in-register P quantizer of faq_attention_fwd on given values
 *                         (simulated_flash_attention.py:801-806 via hif4.py:143-271)
 *   faq_act_prep_rows     quantization.py:199-276 (the full FakeQuantLinear activation path:
 *                         input scale, HiSQ rotation, clamp, companding, online Hadamard,
 *                         HiF4 QDQ), hisq_rotation.py:50-71
 *   faq_hif4_linear_packed  the contraction of quantization.py:199-277 FakeQuantLinear.forward
 *                         (F.linear on the HiF4-exact operands) for few input rows, with the
 *                         HiF4 weight kept packed (4.5 bits per weight)
 *   faq_mfma_probe        no reference counterpart: a measurement helper (the device's
 *                         sustained bf16 MFMA rate, the reference point of the benchmark)
 *   faq_stream_probe      no reference counterpart: a measurement helper (the device's
 *                         read rate for a plain stream, the reference point of the decode
 *                         benchmark)
 */
#ifndef FAQUANT_AMD_H
#define FAQUANT_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FAQ_OK 0
#define FAQ_EINVAL (-1)  /* invalid argument */
#define FAQ_EUNSUP (-2)  /* valid in the reference but not implemented by this library */
#define FAQ_ELAUNCH (-3) /* HIP launch error */

#define FAQ_F32 0
#define FAQ_BF16 1
#define FAQ_F16 2

typedef void* faq_stream_t; /* hipStream_t */

/* Message of the last failed call on this thread ("" if none). */
const char* faq_last_error(void);

/* Library version string. */
const char* faq_version(void);

/*
 * HiF4 fake quantization of `rows` rows of `cols` values (row stride = cols), along
 * the row in groups of 64 with zero padding of a short last group; y has x's dtype
 * (FAQ_F32 / FAQ_BF16 / FAQ_F16) and may alias x.  Optional outputs (NULL to skip),
 * with groups = ceil(cols / 64):
 *   scale, rec      fp32 [rows, groups]   E6M2 scale and bf16 reciprocal
 *   lv2             int8 [rows, groups, 8]   level-2 exponents (per 8 values)
 *   lv3             int8 [rows, groups, 16]  level-3 exponents (per 4 values)
 *   codes           uint8 [rows, cols / 2]   4-bit codes, value 2i in the low nibble
 *                   (bit 3 sign, bits 0-2 magnitude); requires cols % 64 == 0
 *   scale_byte      uint8 [rows, groups]  ((e + 48) << 2) | m with scale = 2^e (1 + m/4)
 *   lv2_bits        uint8 [rows, groups]  bit i = lv2 of 8-group i
 *   lv3_bits        uint16 [rows, groups] bit i = lv3 of 4-group i
 */
int faq_hif4_qdq_rows(const void* x, void* y, int64_t rows, int64_t cols, int dtype, int levels,
                      float* scale, float* rec, int8_t* lv2, int8_t* lv3, uint8_t* codes,
                      uint8_t* scale_byte, uint8_t* lv2_bits, uint16_t* lv3_bits, faq_stream_t stream);

/*
 * Normalized Walsh-Hadamard transform (Sylvester order, fp32 butterflies, true division
 * by fp32(sqrt(block))) applied independently to each `block`-wide slice of each row;
 * rows of `cols` values, cols % block == 0 and cols % 8 == 0, block a power of two in
 * [2, 512].  Input dtype in_dtype is converted to fp32, the result is rounded once to
 * out_dtype (the reference's chunked transform and rotate_heads).
 */
int faq_hadamard_rows(const void* x, void* y, int64_t rows, int64_t cols, int block, int in_dtype,
                      int out_dtype, faq_stream_t stream);

/*
 * Attention operand prologue for Q or K, head_dim 128: x [B, H, L, 128] with element
 * strides (sb, sh, sl).  In fp32: subtract key_offset[h * off_sh + d] (if non-NULL),
 * multiply (smooth_divide = 0) or divide (= 1) by smooth[h * smooth_sh + d] (if
 * non-NULL), apply the block Hadamard of size `hadamard` (0 = none, 64 or 128), round
 * once to round_dtype; optionally store that rotated tensor to `rotated` (round_dtype,
 * contiguous [B, H, L, 128]); then HiF4 QDQ with `levels` (0 = no quantization) and
 * store bf16 to y with element strides (yb, yh, yl).
 */
int faq_operand_prep(const void* x, int in_dtype, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                     const float* key_offset, int64_t off_sh, const float* smooth, int64_t smooth_sh,
                     int smooth_divide, int hadamard, int round_dtype, void* rotated, void* y, int64_t yb,
                     int64_t yh, int64_t yl, int levels, faq_stream_t stream);

/*
 * Normalized Walsh-Hadamard transform over rows of `cols` values (cols a power of two in
 * [8, 512]) computed in the tensor's own dtype (FAQ_BF16 or FAQ_F16), as
 * src/faquant/rotation.py:14-29 hadamard_transform runs on such a tensor: after every
 * butterfly stage each fp32 sum or difference is rounded to the dtype, and the division by
 * fp32(sqrt(cols)) is rounded once more.  y may alias x.
 */
int faq_hadamard_rows_native(const void* x, void* y, int64_t rows, int64_t cols, int dtype, faq_stream_t stream);

/*
 * Values of the packed HiF4 storage view written by faq_hif4_qdq_rows (4-bit codes, low
 * nibble = even element, bit 3 sign; one E6M2 byte ((e + 48) << 2) | m, 8 level-2 bits and
 * 16 level-3 bits per 64 values: the content of CompactHiF4Parameters, hif4.py:67-79, and
 * the per-value multipliers of expand_hif4_parameters, hif4.py:222-243).  Exact: decodes
 * to the fake-quantized values.  cols must be a multiple of 64; y is [rows, cols] in
 * out_dtype.
 */
int faq_hif4_unpack_rows(const uint8_t* codes, const uint8_t* scale_byte, const uint8_t* lv2_bits,
                         const uint16_t* lv3_bits, int64_t rows, int64_t cols, int out_dtype, void* y,
                         faq_stream_t stream);

/*
 * Activation prologue of a W4A4 Linear over x [rows, cols] (contiguous, dtype for input and
 * output): x * dtype(col_scale) in dtype (col_scale optional, fp32 [cols]), then an optional
 * per-block fp32 Hadamard of size `hadamard` (power of two <= 512, 0 = none) cast back to
 * dtype, then the HiF4 QDQ with `levels` (0 = none) in groups of 64.  Replaces the
 * input_scale / online_hadamard / fake_quantize steps of FakeQuantLinear.forward
 * (src/faquant/quantization.py:204-276) and the input QDQ of HiF4Linear
 * (src/faquant/wan22_hif4.py:81-92).
 */
int faq_act_qdq_rows(const void* x, void* y, int64_t rows, int64_t cols, int dtype, const float* col_scale,
                     int hadamard, int levels, faq_stream_t stream);

/*
 * Options of faq_act_prep_rows, each absent when NULL / 0.  Vectors hold one value per
 * feature (cols).
 */
typedef struct faq_act_opts {
  const float* col_scale;   /* input scale (multiplied in the input dtype) */
  const int8_t* rot_signs;  /* HiSQ input rotation: signs (+1 / -1) ... */
  const int32_t* rot_perm;  /* ... and the permutation (index_select order, a permutation of 0..cols-1) */
  int rot_block;            /* the rotation's block Hadamard size, or 0 for none */
  int has_min, has_max;     /* activation clamp bounds present */
  float act_min, act_max;   /* the bounds (applied in the input dtype, NaN kept) */
  const float* compand;     /* activation companding scale, already in the input dtype */
  int hadamard;             /* online block Hadamard size, or 0 */
  int hadamard_generalized; /* 1: the online transform is generalized_hadamard_transform over
                               the whole row (cols a power of two, or 12 times one;
                               rotation.py:53-69); hadamard must then be 0 */
  const float* compand_rcp; /* optional, with compand: faq_act_compand_rcp of the companding
                               scale; the final x / compand is then a product where exact */
  int stage_round;          /* 1: the online transform in the input dtype, as the reference's
                               hadamard_transform / generalized_hadamard_transform run on a
                               bf16 / fp16 tensor (rotation.py:14-69): every butterfly stage and
                               the 12-point mix rounded to the dtype */
} faq_act_opts;

/*
 * The whole activation path of a quantized Linear, as FakeQuantLinear.forward runs it
 * (src/faquant/quantization.py:199-276): x * input_scale, the HiSQ input rotation (fp32 x
 * times the signs, gathered by the permutation, the per-block fp32 Hadamard of
 * rotation.py:117-135 when rot_block is set, one cast back; quantization.py:201-219 and
 * hisq_rotation.py:50-71), the activation clamp, x * companding scale, the online block
 * Hadamard with one cast back, the HiF4 QDQ with `levels` (0: none), and x / companding
 * scale; each elementwise step rounds to the input dtype.  Rows of at most 32768 features
 * (a multiple of 64), contiguous, fp32 / bf16 / fp16; one workgroup per row.  With the
 * rotation or a Hadamard block above 8 the row passes through LDS as fp32 (4.5 bytes a
 * feature; FAQ_EUNSUP beyond the device's LDS per workgroup).  x, y and the col_scale, rot_signs,
 * rot_perm and compand vectors must be 16-byte aligned.  opts may be NULL (then this is faq_act_qdq_rows
 * without input scale or Hadamard).
 */
int faq_act_prep_rows(const void* x, void* y, int64_t rows, int64_t cols, int dtype, const faq_act_opts* opts,
                      int levels, faq_stream_t stream);

/*
 * The reciprocals faq_act_prep_rows uses for its companding quotient (quantization.py:268,
 * x / compand_scale in the activation dtype): rcp[j] = fp32(1 / compand[j]) where
 * dtype(x * rcp) equals dtype(x / compand) for every x of `dtype` (bf16: normal scales;
 * fp16: |scale| < 8, which holds the reference's scales exp(clamp(log, -2.079, 2.079));
 * proved over all pairs of 16-bit values), 0 elsewhere and for fp32 (those divide).  No
 * reference counterpart: a per-layer constant FakeQuantLinear computes once beside its
 * companding scale.  compand and rcp are n fp32 values on the device.
 */
int faq_act_compand_rcp(const float* compand, float* rcp, int64_t n, int dtype, faq_stream_t stream);

/*
 * V operand: x [B, H, L, 128] (strides sb, sh, sl), HiF4 QDQ with `levels` (0 = none),
 * written transposed as bf16 vt [B, H, 128, Lpad] (contiguous), Lpad = multiple of 128
 * >= L, keys >= L zero-filled.
 */
int faq_operand_prep_vt(const void* x, int in_dtype, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                        int Lpad, uint16_t* vt, int levels, faq_stream_t stream);

/*
 * Score options of faq_attention_fwd / faq_attention_fwd_split (a NULL pointer: none).
 *   row_lo, row_hi  int32 [B, Lq]: query position p of batch b sees only the keys in
 *   key_bits        [row_lo, row_hi] (inclusive, within [0, Lk - 1]; row_lo > row_hi: no
 *                   key, output row 0) whose bit k % 32 of key_bits word k / 32 is set;
 *                   key_bits is uint32 [B, key_words], key_words >= 4 * ceil(Lk / 128), zero
 *                   past Lk.
 *   row_blocks      int32 [B, ceil(Lq / 32), 4], 16-byte aligned: per 32 positions, the
 *                   minimum row_lo and maximum row_hi + 1 of the non-empty rows (Lk and 0
 *                   if none), the maximum row_lo and minimum row_hi of all rows (an empty
 *                   row counting as Lk and -1).  row_lo, row_hi, row_blocks and key_bits:
 *                   all or none; none: the `causal` argument decides.
 *   softcap         > 0: scores become softcap * tanh(scale * s / softcap) before masking
 *                   (simulated_flash_attention.py:725-727; needs the key ranges); 0: off.
 *   dense_mask      fp32 additive mask (3-D/4-D masks, simulated_flash_attention.py:430-454):
 *   dm_sb, dm_sh,   element [b, h, p, k] at dense_mask + b dm_sb + h dm_sh + p dm_sq + k
 *   dm_sq           (0 broadcasts; multiples of 4), k < Lpad; -inf masks, columns >= Lk
 *                   must be -inf.  Scores become scale * s (softcapped if softcap > 0)
 *                   + mask and the `causal` argument is not applied.  Exclusive with
 *                   the key ranges.
 *   pv_probe        fp32 [B, Hq, Lq, 5] (faq_attention_fwd with quant_p only), or NULL:
 *                   the PV-normalizer probe of simulated_flash_attention.py:36-185, 835-869.
 *                   Per row: sum of P-hat and sum of P (each rescaled like the running
 *                   denominator), #(P-hat = 0 < P), sum (P-hat - P)^2 and sum P^2 over
 *                   every processed key.
 *   p_dump          fp32 [B, Hq, Lq, 2, p_dump_stride] (faq_attention_fwd with quant_p only),
 *   p_dump_stride   or NULL: for every key k of every key tile a row processes, the kernel's
 *                   P at [..., 0, k] and its HiF4 QDQ P-hat at [..., 1, k] (keys of skipped
 *                   tiles are not written; masked and padding keys hold P = 0).  p_dump_stride
 *                   is a multiple of 4 and >= 128 * ceil(Lk / 128).  For verification: P-hat of
 *                   each 128-key tile equals fake_quantize_hif4 (hif4.py:377-390) of that
 *                   tile's P, bit for bit.
 * faq_attention_mask_bounds computes row_lo / row_hi / key_bits from a 2-D mask (or, with
 * mask = NULL, the plain causal / full ranges).
 */
typedef struct faq_attn_opts {
  const int32_t* row_lo;
  const int32_t* row_hi;
  const int32_t* row_blocks;
  const uint32_t* key_bits;
  int64_t key_words;
  float softcap;
  float* pv_probe;
  const float* dense_mask;
  int64_t dm_sb, dm_sh, dm_sq;
  float* p_dump;
  int64_t p_dump_stride;
  /* q_prep = 1: q holds the raw bf16 query rows, and the kernel applies the operand
     prologue of faq_operand_prep to them as it loads them (the per-block fp32 Hadamard of
     q_hadamard = 0, 64 or 128 dims, one bf16 cast, the HiF4 QDQ with q_levels = 0 (none),
     123, 12 or 13; no key offset or Smooth-QK): bit for bit the attention of the prepared
     operand, without its separate pass over Q (qwen3.py:97-130) */
  int q_prep, q_hadamard, q_levels;
} faq_attn_opts;

/*
 * Key ranges of a 2-D attention mask for faq_attn_opts.  `mask` is uint8/bool [B, Lk]
 * with row stride mask_sb (the last Lk columns of the caller's mask; nonzero = valid), or
 * NULL for all keys valid.  As the reference does (unpadded FlashAttention alignment):
 * query position p is valid when mask column p + Lk - Lq is (invalid when that column is
 * < 0), and it sees the valid keys whose rank among valid keys is <= its own column's rank
 * (causal), > rank - window (window > 0) and < rank + window (window > 0, not causal).
 * Writes row_lo / row_hi [B, Lq], row_blocks [B, ceil(Lq / 32), 4] and, if key_bits is
 * non-NULL, key_bits [B, key_words] (key_words >= 4 * ceil(Lk / 128)).  Lk <= 524288.
 */
int faq_attention_mask_bounds(const uint8_t* mask, int64_t mask_sb, int B, int Lq, int Lk, int causal, int window,
                              int32_t* row_lo, int32_t* row_hi, int32_t* row_blocks, uint32_t* key_bits,
                              int64_t key_words, faq_stream_t stream);

/*
 * HiF4 QK/PV flash attention forward, head_dim 128, key tiles of 128 in ascending
 * order from key 0.
 *   q   bf16 [B, Hq, Lq, 128]  strides (q_sb, q_sh, q_sl)   (quantized or not by caller)
 *   k   bf16 [B, Hkv, Lk, 128] strides (k_sb, k_sh, k_sl)
 *   vt  bf16 [B, Hkv, 128, Lpad] strides (v_sb, v_sh, v_sd) from faq_operand_prep_vt
 *   o   [B, Hq, Lq, 128] via strides (o_sb, o_sh, o_sl), o_dtype FAQ_F32 or FAQ_BF16
 *   Hq % Hkv == 0 (query head h reads KV head h / (Hq / Hkv)).
 *   causal      1: bottom-right causal mask (row p sees keys <= p + Lk - Lq)
 *   scale       softmax scale (e.g. 128^-0.5)
 *   quant_p     1: HiF4-quantize P along keys in 64-groups with p_levels
 *   norm_same   1: denominator sums the quantized P (P-Reordering, "quantized_same")
 *   row_den     optional fp32 [B, Hq, Lq]: the final softmax denominator of each row
 *   out_levels  0, or HiF4 levels (123 / 12 / 13) of a QDQ of every 64-value half of each
 *               output row after its rounding to o_dtype: the o_proj-input activation
 *               quantizer of src/faquant/qwen3.py:167-171, fused into the epilogue
 *   opts        NULL, or key-range masks and the logit softcap (faq_attn_opts)
 */
int faq_attention_fwd(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                      int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* vt, int64_t v_sb, int64_t v_sh,
                      int64_t v_sd, int Lpad, void* o, int o_dtype, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                      int B, int Hq, int Hkv, int Lq, int Lk, int causal, float scale, int quant_p, int p_levels,
                      int norm_same, float* row_den, int out_levels, const faq_attn_opts* opts,
                      faq_stream_t stream);

/*
 * The same recurrence for the shapes and operand types faq_attention_fwd does not take
 * (src/faquant/simulated_flash_attention.py:457-909 with any key chunk, head_dim, and fp32
 * operands that the reference multiplies as they are, sfa:723-724, 848-850): fp32 arithmetic
 * throughout, P-hat bit for bit the reference quantizer of this kernel's P.
 *   q, k, v   [B, Hq|Hkv, Lq|Lk, D] at element strides (last stride 1), each FAQ_F32,
 *             FAQ_BF16 or FAQ_F16, natural layout (V not transposed); quantized operands come
 *             in already quantized (faq_hif4_qdq_rows along D)
 *   o         [B, Hq, Lq, D] via strides, FAQ_F32, FAQ_BF16 or FAQ_F16
 *   D         head_dim, 1..256;  key_tile  keys per tile, 1..1024 (the simulator's
 *             faquant_attention_key_chunk_size; P groups of 64 start at each tile)
 *   causal, scale, quant_p, p_levels, norm_same, row_den  as faq_attention_fwd
 *   opts      NULL, or key ranges (row_lo, row_hi, key_bits, key_words; row_blocks unused),
 *             softcap, dense_mask and pv_probe with the meanings of faq_attn_opts; p_dump and
 *             q_prep are refused
 */
int faq_attention_fwd_general(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_sl, const void* k,
                              int k_dtype, int64_t k_sb, int64_t k_sh, int64_t k_sl, const void* v, int v_dtype,
                              int64_t v_sb, int64_t v_sh, int64_t v_sl, void* o, int o_dtype, int64_t o_sb,
                              int64_t o_sh, int64_t o_sl, int B, int Hq, int Hkv, int Lq, int Lk, int D, int key_tile,
                              int causal, float scale, int quant_p, int p_levels, int norm_same, float* row_den,
                              const faq_attn_opts* opts, faq_stream_t stream);

/*
 * Split-key form of faq_attention_fwd for grids that cannot fill the GPU (decode steps,
 * short prompts).  Same arguments and results (up to the fp32 order of the final O and l
 * sums; every P-hat code is the same); out_levels is not available.  Key tiles are divided
 * into nsplit ranges: a first pass records each row's c1-scaled maximum of every key
 * tile, a scan gives each range the running maximum of the tiles before it (the maximum
 * the reference's sequential recurrence holds there, sfa:788-806), each range then runs
 * the recurrence from it, and a combine rescales and sums the ranges.  `workspace` is
 * device memory of at least faq_attention_split_workspace(B, Hq, Lq, Lk, nsplit) bytes,
 * 16-byte aligned.  nsplit is 1..4096 and Lk at most 16384 key tiles (2097152 keys);
 * beyond that the call returns FAQ_EUNSUP (use faq_attention_fwd).
 */
int64_t faq_attention_split_workspace(int B, int Hq, int Lq, int Lk, int nsplit);
int faq_attention_fwd_split(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                            int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* vt, int64_t v_sb, int64_t v_sh,
                            int64_t v_sd, int Lpad, void* o, int o_dtype, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                            int B, int Hq, int Hkv, int Lq, int Lk, int causal, float scale, int quant_p,
                            int p_levels, int norm_same, float* row_den, int nsplit, void* workspace,
                            int64_t workspace_bytes, const faq_attn_opts* opts, faq_stream_t stream);

/*
 * faq_attention_fwd_split without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The workspace is a static device array of
 * FAQ_NOALLOC_SCRATCH_BYTES per GPU, held for the life of the process; the call allocates
 * and frees nothing.  Calls whose split layout (faq_attention_split_workspace) exceeds it
 * return FAQ_EINVAL.  The stream must belong to the current device.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (different streams, or threads)
 * race; calls on one stream are ordered.  Each call writes every scratch byte it reads, so
 * nothing carries over from the previous call.
 */
#define FAQ_NOALLOC_SCRATCH_BYTES (8ll << 20)
int faq_attention_fwd_split_noalloc(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                                    int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* vt, int64_t v_sb,
                                    int64_t v_sh, int64_t v_sd, int Lpad, void* o, int o_dtype, int64_t o_sb,
                                    int64_t o_sh, int64_t o_sl, int B, int Hq, int Hkv, int Lq, int Lk, int causal,
                                    float scale, int quant_p, int p_levels, int norm_same, float* row_den,
                                    int nsplit, const faq_attn_opts* opts, faq_stream_t stream);

/*
 * Packed HiF4 K or V (decode caches): one row of 128 values per key, 4.5 bits per value.
 * codes: 16 uint32 words per row; dims 8u .. 8u + 7 (u = 0..15) are word (u & 1) * 8 + u / 2,
 * dim 8u + i in bits 4i .. 4i + 3 as 8 + the signed code (-7 .. 7).  meta: 2 uint32 words per row, one per
 * 64-dim group: bits 0-7 the E6M2 byte ((e + 48) << 2) | m of the scale 2^e (1 + m/4), bits
 * 8-15 the level-2 exponents (bit j: 8-dim group j), bits 16-31 the level-3 exponents (bit
 * j: 4-dim group j).  A value is (nibble - 8) * 2^(lv2 + lv3) * scale / 4, the HiF4 QDQ
 * value.  A group that held a NaN has E6M2 byte 0xFF and decodes to NaN.  Row r of
 * (batch b, head h) is codes[(b * sb + h * sh + r) * 16], meta[(b * sb + h * sh + r) * 2].
 */
typedef struct faq_hif4_kv {
  const uint32_t* codes; /* 16-byte aligned */
  const uint32_t* meta;  /* 8-byte aligned */
  int64_t sb, sh;        /* batch and head strides in rows */
} faq_hif4_kv;

/*
 * faq_operand_prep with the HiF4 QDQ (levels, required) written in the packed form above
 * instead of bf16: positions 0..L-1 of x [B, H, L, 128] go to rows 0..L-1 of (b, h), rows
 * b * p_sb + h * p_sh + l.  The same prologue (key offset, Smooth-QK, Hadamard, one cast to
 * round_dtype) and the same quantizer, so decoding gives bitwise faq_operand_prep's bf16
 * output.  Rows are token-local: appending a decode position packs one row.  Replaces the
 * K/V QDQ of src/faquant/simulated_flash_attention.py:592-611 (with the qwen3.py:97-136
 * prologue) where its result is kept as a decode cache (sfa:243-289), stored in the
 * compact form of hif4.py:67-79.
 */
int faq_operand_prep_hif4_kv(const void* x, int in_dtype, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L,
                             const float* key_offset, int64_t off_sh, const float* smooth, int64_t smooth_sh,
                             int smooth_divide, int hadamard, int round_dtype, int levels, uint32_t* codes,
                             uint32_t* meta, int64_t p_sb, int64_t p_sh, faq_stream_t stream);

/*
 * Decode-shaped attention (few query rows per KV head, long key ranges): the results of
 * faq_attention_fwd_split with the same nsplit, bitwise, for masks none or bottom-right
 * causal (no opts, no out_levels), at most 32 query heads per KV head.  K and V come either
 * as bf16 K and V [B, Hkv, Lk, 128] at element strides (natural [key][dim] rows, as a decode
 * cache grows; not the V^T of faq_attention_fwd) or, with kp and vp non-NULL (both), as
 * packed HiF4 rows (k and v unused); the packed form decodes to the bf16 operands, so both
 * give the same bits.  The query
 * heads sharing a KV head are computed together (one pass over each K/V tile for all of
 * them): a scores pass writes S and tile maxima to the workspace, a values pass runs the
 * recurrence per key range, and a combine sums the ranges.  Calls with P quantized, the
 * quantized-same normalizer, at most 8 query rows per KV head (heads x positions), one key
 * tile per range and at most 8192 keys run the scores and values of each range in one
 * kernel instead (the same bits): each range publishes its maxima, stamped with a per-call
 * epoch, to a file-scope array of the library and reads the earlier ranges' maxima from
 * it, waiting a bounded time and otherwise computing them from K itself, so calls that
 * overlap on one GPU stay correct; they share the array, though, and a range whose
 * predecessors' maxima another call overwrote waits out the whole bound (4096 rounds)
 * before computing them, so overlapping decode calls can run much slower.  A call on a
 * stream that is capturing a HIP graph runs the two passes: a recorded launch would keep
 * its epoch on every replay.  `workspace` is device memory of at least
 * faq_attention_decode_workspace(B, Hq, Lq, Lk, nsplit) bytes, 16-byte aligned; nsplit is
 * 1..4096.  Replaces, for the decode steps of a KV cache
 * (src/faquant/simulated_flash_attention.py:243-289), the attention of
 * simulated_flash_attention.py:457-909.
 */
int64_t faq_attention_decode_workspace(int B, int Hq, int Lq, int Lk, int nsplit);
int faq_attention_decode(const uint16_t* q, int64_t q_sb, int64_t q_sh, int64_t q_sl, const uint16_t* k,
                         int64_t k_sb, int64_t k_sh, int64_t k_sl, const uint16_t* v, int64_t v_sb, int64_t v_sh,
                         int64_t v_sl, const faq_hif4_kv* kp, const faq_hif4_kv* vp, void* o, int o_dtype,
                         int64_t o_sb, int64_t o_sh, int64_t o_sl, int B, int Hq, int Hkv, int Lq, int Lk, int causal,
                         float scale, int quant_p, int p_levels, int norm_same, float* row_den, int nsplit,
                         void* workspace, int64_t workspace_bytes, faq_stream_t stream);

/*
 * y [M, N] = x [M, K] W^T (+ bias) with W kept as packed HiF4 rows, for M <= 8 rows of x:
 * the contraction of FakeQuantLinear.forward (src/faquant/quantization.py:199-277, F.linear
 * on the activation QDQ x and the weight QDQ W) where reading W dominates (decode steps, small
 * batches).  W's row for output feature n and columns 128 j .. 128 j + 127 is packed row
 * n * (K / 128) + j of `w_codes` (16 words per row) and `w_meta` (2 words per row) in the
 * faq_hif4_kv row format: faq_operand_prep_hif4_kv of W viewed as [1, 1, N K / 128, 128] with
 * the weight's levels writes it, and it decodes to the bf16 weight QDQ bitwise.  x: bf16
 * [M, K], 16-byte aligned, row stride x_sm elements (>= K, a multiple of 8); y: fp32 or bf16
 * [M, N], row stride y_sm (>= N); bias: NULL or fp32 / bf16 [N].  K must be a multiple of 128
 * and M at most 8 (FAQ_EUNSUP otherwise).  The products of a feature are summed in fp32 in a
 * fixed order (each lane over its blocks, then the lanes), so every call gives the same bits;
 * the bias is added to the fp32 sum and y rounded once (bf16: round to nearest even).  Not
 * bitwise the library GEMM of F.linear, whose fp32 sums run in another order.  No workspace.
 */
int faq_hif4_linear_packed(const uint16_t* x, int64_t x_sm, const uint32_t* w_codes, const uint32_t* w_meta,
                           const void* bias, int bias_dtype, void* y, int y_dtype, int64_t y_sm, int M, int N, int K,
                           faq_stream_t stream);

/*
 * The attention kernel's in-register P quantizer (the HiF4 QDQ of P along keys,
 * simulated_flash_attention.py:801-806 through hif4.py:143-271) applied to `groups`
 * contiguous 64-value groups of non-negative fp32 values p (group maximum from the
 * values), writing fp32 p_hat.  The same device code as faq_attention_fwd, exposed so
 * that its codes can be checked against fake_quantize_hif4 on chosen values (ties of
 * RN(p qm) 4 + 0.5 included).  levels 123 / 12 / 13.
 */
int faq_pquant_groups(const float* p, float* p_hat, int64_t groups, int levels, faq_stream_t stream);

/*
 * Measurement helper with no counterpart in the reference: `blocks` workgroups of the
 * attention kernel's launch shape (512 threads, two waves per SIMD) each run `iters`
 * iterations of four independent bf16 32x32x16 MFMA chains per wave, nothing else.
 * FLOP = blocks * 8 * iters * 4 * 32768.  Timed by the caller; the result is this
 * device's sustained dense bf16 MFMA rate.  out receives blocks * 512 fp32 values.
 */
int faq_mfma_probe(float* out, int blocks, int iters, faq_stream_t stream);

/*
 * Measurement helper with no counterpart in the reference: `blocks` 256-thread workgroups
 * read the `bytes` bytes at x (a positive multiple of 16, 16-byte aligned) with coalesced
 * 16-byte loads in a grid-stride loop, four loads per thread in flight, and write one fp32
 * word per workgroup to out.  Timed by the caller; the result is this device's read rate
 * for a plain stream (from HBM, or from the last-level cache when x fits there and was
 * read just before).
 */
int faq_stream_probe(const void* x, int64_t bytes, float* out, int blocks, faq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FAQUANT_AMD_H */
