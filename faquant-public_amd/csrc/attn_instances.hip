// Instantiations of the attention kernel for one masking form, FAQ_ATTN_MASK (0..4, the
// kMask of attn_fwd_kernel): the build compiles this file once per form, in parallel, and
// links the objects with the C ABI (capi.hip).
#include "hif4_attention.hip"

#ifndef FAQ_ATTN_MASK
#error "compile with -DFAQ_ATTN_MASK=<0..4>"
#endif

namespace faq {
namespace {

template <int LV, int kMask>
void launch_lv(const AttnArgs& a, int quant_p, int same, dim3 grid, hipStream_t st) {
  if (a.diag || a.p_dump) {  // the probe form exists only with P quantization (validated by the caller)
    if (same) hipLaunchKernelGGL((attn_fwd_kernel<LV, true, true, kMask | 8>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((attn_fwd_kernel<LV, true, false, kMask | 8>), grid, dim3(512), 0, st, a);
    return;
  }
  if (quant_p && same) hipLaunchKernelGGL((attn_fwd_kernel<LV, true, true, kMask>), grid, dim3(512), 0, st, a);
  else if (quant_p) hipLaunchKernelGGL((attn_fwd_kernel<LV, true, false, kMask>), grid, dim3(512), 0, st, a);
  else hipLaunchKernelGGL((attn_fwd_kernel<LV, false, false, kMask>), grid, dim3(512), 0, st, a);
}

}  // namespace

template <int kMask>
void launch_attention_mask(const AttnArgs& a, int quant_p, int p_levels, int norm_same, dim3 grid, hipStream_t st) {
  const int lv = quant_p ? p_levels : 123;
  if (lv == 12) launch_lv<12, kMask>(a, quant_p, norm_same, grid, st);
  else if (lv == 13) launch_lv<13, kMask>(a, quant_p, norm_same, grid, st);
  else launch_lv<123, kMask>(a, quant_p, norm_same, grid, st);
}

template void launch_attention_mask<FAQ_ATTN_MASK>(const AttnArgs&, int, int, int, dim3, hipStream_t);

}  // namespace faq
