"""``fake_quantize`` dispatcher: drop-in for faquant.quantization.fake_quantize (hif4 branch).

Reference: src/faquant/quantization.py:30-57.  The HiF4 branch validates its
arguments with the reference's messages and runs the HIP quantizer.  The int
and MXFP8 formats are not part of the HiF4 attention path and raise
NotImplementedError rather than silently computing something else.
"""

from __future__ import annotations

import torch

from .hif4 import HIF4_BLOCK_SIZE, fake_quantize_hif4


def check_hif4_arguments(*, bits: int = 4, group_size: int = -1, symmetric: bool = True, clip_ratio: float = 1.0) -> None:
    """The HiF4 branch's argument checks and messages (quantization.py:48-56)."""
    if bits != 4:
        raise ValueError("HiF4 requires bits=4")
    if group_size not in (-1, HIF4_BLOCK_SIZE):
        raise ValueError("HiF4 requires group_size=64 (or -1 for direct use)")
    if not symmetric:
        raise ValueError("HiF4 does not support asymmetric quantization")
    if clip_ratio != 1.0:
        raise ValueError("HiF4 direct-cast does not support clipping")


def fake_quantize(
    x: torch.Tensor,
    *,
    quant_format: str = "int",
    bits: int = 4,
    group_size: int = -1,
    symmetric: bool = True,
    clip_ratio: float = 1.0,
    hif4_levels: str | None = None,
) -> torch.Tensor:
    if quant_format == "hif4":
        check_hif4_arguments(bits=bits, group_size=group_size, symmetric=symmetric, clip_ratio=clip_ratio)
        return fake_quantize_hif4(x, levels=hif4_levels)
    if quant_format in ("int", "mxfp8e4m3"):
        if quant_format == "int" and bits >= 16:
            return x
        raise NotImplementedError(
            f"quant_format={quant_format!r} is outside the HiF4 attention path of this library"
        )
    raise ValueError(f"unsupported quant_format={quant_format!r}")
