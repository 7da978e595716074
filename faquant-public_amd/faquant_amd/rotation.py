"""Normalized Walsh-Hadamard transforms on the MI355X: drop-in for faquant.rotation (hot-path subset).

Reference: src/faquant/rotation.py:14-29 (``hadamard_transform``), 53-84
(``generalized_hadamard_transform`` and its chunked form), 87-114 (``OnlineHadamardLinear``)
and 117-135 (``chunked_block_hadamard_transform``).  The HIP kernels run the same fp32
butterfly stages in the same order (strides 1, 2, ..., n/2) and divide by
fp32(sqrt(n)) exactly as CPU torch does, so fp32 results are bit-identical.  Blocks
above 512 and the generalized transform run in the row kernel of the Linear activation
path (rows of at most 32768 features, a multiple of 64).
"""

from __future__ import annotations

import torch
from torch import nn

from . import _ops


def _is_power_of_two(value: int) -> bool:
    return value > 0 and value & (value - 1) == 0


def hadamard_transform(x: torch.Tensor) -> torch.Tensor:
    """Normalized Walsh-Hadamard transform over the final axis, computed in ``x.dtype`` as
    the reference's butterflies are (rotation.py:14-29): fp32 exactly, bf16 / fp16 with
    every stage rounded to that dtype.  Sizes up to 512 on the Hadamard kernels, larger ones
    (a multiple of 64, up to 32768) on the activation row kernel."""
    size = x.shape[-1]
    if not _is_power_of_two(size):
        raise ValueError(f"Hadamard dimension must be a power of two, got {size}")
    if x.dtype == torch.float32:
        if size > 512:
            return _row_path(x, hadamard=size)
        return _ops.hadamard_rows(x, size, torch.float32)
    if x.dtype in (torch.bfloat16, torch.float16):
        if size > 512:
            return _row_path(x, hadamard=size, stage_round=True)
        return _ops.hadamard_rows_native(x)
    raise NotImplementedError(f"hadamard_transform on the MI355X takes fp32, bf16 or fp16 input, got {x.dtype}")


def chunked_block_hadamard_transform(x: torch.Tensor, *, block_size: int, chunk_rows: int = 256) -> torch.Tensor:
    """Independent normalized Hadamard per ``block_size`` slice, fp32 math, cast back to x.dtype.

    ``chunk_rows`` only bounded the reference's fp32 temporaries; the kernel needs none.
    """
    del chunk_rows
    if not _is_power_of_two(block_size) or x.shape[-1] % block_size:
        raise ValueError(
            f"dimension {x.shape[-1]} must be divisible by power-of-two block_size={block_size}"
        )
    if block_size > 512:
        return _row_path(x, hadamard=block_size)
    return _ops.hadamard_rows(x, block_size, x.dtype)


def _row_path(x: torch.Tensor, **kw) -> torch.Tensor:
    """fp32 transform of each row with one cast back to x's dtype (the activation row
    kernel without its quantizer)."""
    cols = x.shape[-1]
    if cols % 64 or cols > 32768:
        raise NotImplementedError(
            f"transforms of {cols} values run on rows of a multiple of 64 features, at most 32768"
        )
    return _ops.act_prep_rows(x, levels=None, **kw)


def generalized_hadamard_transform(x: torch.Tensor) -> torch.Tensor:
    """Normalized Hadamard transform for power-of-two or 12 * power-of-two axes
    (rotation.py:53-69), computed in x's dtype as the reference does: fp32 exactly; bf16 /
    fp16 with every butterfly stage and the 12-point mix (a matmul accumulating in fp32)
    rounded to that dtype, then the division rounded to it."""
    size = x.shape[-1]
    if _is_power_of_two(size):
        return hadamard_transform(x)
    if size % 12 or not _is_power_of_two(size // 12):
        raise ValueError(f"unsupported generalized Hadamard dimension: {size}")
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise NotImplementedError(f"generalized_hadamard_transform takes fp32, bf16 or fp16 input, got {x.dtype}")
    return _row_path(x, hadamard_generalized=True, stage_round=x.dtype != torch.float32)


def chunked_generalized_hadamard_transform(x: torch.Tensor, *, chunk_rows: int = 256) -> torch.Tensor:
    """The generalized transform in fp32 with one cast back to x's dtype (rotation.py:72-84).
    ``chunk_rows`` only bounded the reference's fp32 temporaries."""
    del chunk_rows
    size = x.shape[-1]
    if not _is_power_of_two(size) and (size % 12 or not _is_power_of_two(size // 12)):
        raise ValueError(f"unsupported generalized Hadamard dimension: {size}")
    return _row_path(x, hadamard_generalized=True)


class OnlineHadamardLinear(nn.Module):
    """The online rotation right before a linear layer (rotation.py:87-114): the chunked
    generalized transform of the whole input row (``block_size`` None) or the per-block
    transform, then the wrapped module.  The rotation runs in the HIP row kernels above; the
    wrapped module is called as it is."""

    faquant_online_hadamard = True

    def __init__(self, module: nn.Linear, *, block_size: int | None = None) -> None:
        super().__init__()
        self.module = module
        self.in_features = module.in_features
        self.out_features = module.out_features
        self.faquant_online_hadamard_block_size = block_size

    @property
    def weight(self) -> nn.Parameter:
        return self.module.weight

    @property
    def bias(self) -> nn.Parameter | None:
        return self.module.bias

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.faquant_online_hadamard_block_size is None:
            rotated = chunked_generalized_hadamard_transform(x)
        else:
            rotated = chunked_block_hadamard_transform(x, block_size=self.faquant_online_hadamard_block_size)
        return self.module(rotated)
