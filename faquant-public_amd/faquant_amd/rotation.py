"""Normalized Walsh-Hadamard transforms on the MI355X: drop-in for faquant.rotation (hot-path subset).

Reference: src/faquant/rotation.py:14-29 (``hadamard_transform``) and 117-135
(``chunked_block_hadamard_transform``).  The HIP kernel runs the same fp32
butterfly stages in the same order (strides 1, 2, ..., n/2) and divides by
fp32(sqrt(n)) exactly as CPU torch does, so fp32 results are bit-identical.
"""

from __future__ import annotations

import torch

from . import _ops


def _is_power_of_two(value: int) -> bool:
    return value > 0 and value & (value - 1) == 0


def hadamard_transform(x: torch.Tensor) -> torch.Tensor:
    """Normalized Walsh-Hadamard transform over the final axis, computed in ``x.dtype`` as
    the reference's butterflies are (rotation.py:14-29): fp32 exactly, bf16 / fp16 with
    every stage rounded to that dtype.  Sizes up to 512 (the head_dim and Linear-block
    range of the hot path)."""
    size = x.shape[-1]
    if not _is_power_of_two(size):
        raise ValueError(f"Hadamard dimension must be a power of two, got {size}")
    if x.dtype == torch.float32:
        return _ops.hadamard_rows(x, size, torch.float32)
    if x.dtype in (torch.bfloat16, torch.float16):
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
    return _ops.hadamard_rows(x, block_size, x.dtype)
