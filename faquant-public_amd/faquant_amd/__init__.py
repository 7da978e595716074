"""faquant_amd: the HiF4 quantized attention path of FAQUANT on the AMD MI355X (gfx950).

Drop-in modules with the reference's names (MingZwhy/FAQUANT-Public, src/faquant/):
  hif4                       HiF4 codec (fake quantization, compact metadata, packing)
  quantization               fake_quantize (HiF4 branch)
  rotation                   hadamard_transform, chunked_block_hadamard_transform
  simulated_flash_attention  simulated_flash_attention_forward and its stats
  wan22_attention            hif4_attention, qdq_rows_128, rotate_heads, make_flash_attention
  qwen3                      post-RoPE Q/K excursion and the fused attention core
All compute runs in hand-written HIP kernels in libfaquant_amd.so (C ABI:
include/faquant_amd.h); there is no CPU path.
"""

from . import _lib

__version__ = "0.1.0"


def library_version() -> str:
    return _lib.load().faq_version().decode()
