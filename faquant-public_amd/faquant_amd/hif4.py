"""HiF4 codec on the MI355X: drop-in for ``faquant.hif4`` (the hot-path subset).

Mirrors src/faquant/hif4.py of the reference:
  * level selection from the environment, read at import      hif4.py:13-43
  * ``CompactHiF4Parameters``                                  hif4.py:67-79
  * ``fit_hif4_compact_parameters``                            hif4.py:143-219
  * ``fit_hif4_compact_parameters_for_axis``                   hif4.py:360-373
  * ``fake_quantize_hif4``                                     hif4.py:377-390
plus the packed storage view (4-bit codes, E6M2 byte, level bits) that the
reference's compact metadata describes.  All arithmetic runs in the HIP kernel
``qdq_rows_kernel``; results are bit-identical to the reference.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch

from . import _ops

HIF4_BLOCK_SIZE = 64

_LEVELS = ("123", "12", "13")

HIF4_SCALE_LEVELS = os.environ.get("FAQUANT_HIF4_SCALE_LEVELS", "123")
HIF4_ACT_SCALE_LEVELS = os.environ.get("FAQUANT_HIF4_ACT_SCALE_LEVELS", HIF4_SCALE_LEVELS)
HIF4_ATTN_SCALE_LEVELS = os.environ.get("FAQUANT_HIF4_ATTN_SCALE_LEVELS", HIF4_ACT_SCALE_LEVELS)
for _name, _value in (
    ("FAQUANT_HIF4_SCALE_LEVELS", HIF4_SCALE_LEVELS),
    ("FAQUANT_HIF4_ACT_SCALE_LEVELS", HIF4_ACT_SCALE_LEVELS),
    ("FAQUANT_HIF4_ATTN_SCALE_LEVELS", HIF4_ATTN_SCALE_LEVELS),
):
    if _value not in _LEVELS:
        raise ValueError(f"{_name} must be 123, 12 or 13, got {_value!r}")
HIF4_ATTN_OPERAND_SCALE_LEVELS = dict.fromkeys(("q", "k", "p", "v"), HIF4_ATTN_SCALE_LEVELS)
for _entry in filter(None, os.environ.get("FAQUANT_HIF4_ATTN_OPERAND_LEVELS", "").split(",")):
    _operand, _, _value = _entry.partition("=")
    if _operand not in HIF4_ATTN_OPERAND_SCALE_LEVELS or _value not in _LEVELS:
        raise ValueError(f"FAQUANT_HIF4_ATTN_OPERAND_LEVELS entries must be q|k|p|v=123|12|13, got {_entry!r}")
    HIF4_ATTN_OPERAND_SCALE_LEVELS[_operand] = _value


@dataclass(frozen=True)
class CompactHiF4Parameters:
    """Per-64-block HiF4 metadata (same fields and shapes as the reference)."""

    scale: torch.Tensor
    reciprocal: torch.Tensor
    scale_lv2_exponent: torch.Tensor
    scale_lv3_exponent: torch.Tensor


@dataclass(frozen=True)
class PackedHiF4:
    """HiF4 storage: 4.5 bits per value.

    ``codes`` [..., C/2] uint8, value 2i in the low nibble (bit 3 sign, bits 0-2 the
    magnitude code c, value = c/4 * scale * 2^(lv2 + lv3)); per 64-block
    ``scale_byte`` = ((e + 48) << 2) | m for scale = 2^e (1 + m/4), ``lv2_bits`` (bit i
    = 8-group i) and ``lv3_bits`` (bit i = 4-group i).
    """

    codes: torch.Tensor
    scale_byte: torch.Tensor
    lv2_bits: torch.Tensor
    lv3_bits: torch.Tensor


def _require_floating_point(x: torch.Tensor) -> None:
    if not x.is_floating_point():
        raise TypeError("HiF4 fake quantization expects a floating-point tensor")


def _resolve(levels: str | None, default: str) -> str:
    levels = levels or default
    if levels not in _LEVELS:
        raise ValueError(f"HiF4 levels must be 123, 12 or 13, got {levels!r}")
    return levels


def _kernel_view(x: torch.Tensor) -> tuple[torch.Tensor, torch.dtype]:
    """The kernel handles fp32 / bf16 / fp16; other float dtypes go through fp32
    (the reference computes in fp32 and casts back, which is exact for HiF4 values)."""
    if x.dtype in (torch.float32, torch.bfloat16, torch.float16):
        return x, x.dtype
    return x.float(), x.dtype


@torch.no_grad()
def fit_hif4_compact_parameters(
    blocks: torch.Tensor,
    *,
    max_scale: torch.Tensor | float = 1.0,
    scale_steps: torch.Tensor | float = 0.0,
    levels: str | None = None,
) -> CompactHiF4Parameters:
    """Compact HiF4 metadata of ``blocks[..., 64]`` (hif4.py:143-219).

    ``max_scale`` / ``scale_steps`` are the reference's GPTQ search knobs; only their
    no-op defaults are part of the attention path.
    """
    _require_floating_point(blocks)
    if blocks.ndim == 0:
        raise ValueError("HiF4 parameter fitting requires at least one dimension")
    if blocks.shape[-1] != HIF4_BLOCK_SIZE:
        raise ValueError(
            f"HiF4 parameter fitting requires a final dimension of {HIF4_BLOCK_SIZE}, got {blocks.shape[-1]}"
        )
    if not (isinstance(max_scale, (int, float)) and max_scale == 1.0) or not (
        isinstance(scale_steps, (int, float)) and scale_steps == 0.0
    ):
        raise NotImplementedError("max_scale / scale_steps (GPTQ scale search) are not part of the HIP path")
    levels = _resolve(levels, HIF4_SCALE_LEVELS)
    x, _ = _kernel_view(blocks)
    _, meta = _ops.qdq_rows(x, levels, compact=True)
    lead = tuple(blocks.shape[:-1])
    return CompactHiF4Parameters(
        scale=meta["scale"].reshape(lead + (1, 1, 1)),
        reciprocal=meta["rec"].reshape(lead + (1, 1, 1)),
        scale_lv2_exponent=meta["lv2"].reshape(lead + (8, 1, 1)),
        scale_lv3_exponent=meta["lv3"].reshape(lead + (8, 2, 1)),
    )


@torch.no_grad()
def fit_hif4_compact_parameters_for_axis(x: torch.Tensor) -> CompactHiF4Parameters:
    """Metadata of the grid ``fake_quantize_hif4`` snaps ``x`` to (zero-padded to 64)."""
    _require_floating_point(x)
    if x.ndim == 0:
        raise ValueError("HiF4 parameter fitting requires at least one dimension")
    if x.shape[-1] == 0:
        raise ValueError("HiF4 parameter fitting does not support an empty axis")
    pad = (-x.shape[-1]) % HIF4_BLOCK_SIZE
    padded = torch.nn.functional.pad(x, (0, pad)) if pad else x
    return fit_hif4_compact_parameters(padded.reshape(*padded.shape[:-1], -1, HIF4_BLOCK_SIZE))


@torch.no_grad()
def fake_quantize_hif4(x: torch.Tensor, *, levels: str | None = None) -> torch.Tensor:
    """Official HiF4 direct-cast fake quantization along the final axis (hif4.py:377-390)."""
    _require_floating_point(x)
    if x.ndim == 0:
        raise ValueError("HiF4 fake quantization requires at least one dimension")
    if x.shape[-1] == 0:
        raise ValueError("HiF4 fake quantization does not support an empty axis")
    levels = _resolve(levels, HIF4_ACT_SCALE_LEVELS)
    xk, dtype = _kernel_view(x)
    y = _ops.qdq_rows(xk, levels)
    return y if y.dtype == dtype else y.to(dtype)


@torch.no_grad()
def encode_hif4(x: torch.Tensor, *, levels: str | None = None) -> PackedHiF4:
    """Packed HiF4 of ``x`` (last axis a multiple of 64); decodes to fake_quantize_hif4(x)."""
    _require_floating_point(x)
    if x.ndim == 0 or x.shape[-1] % HIF4_BLOCK_SIZE:
        raise ValueError("HiF4 packing needs a last axis that is a multiple of 64")
    levels = _resolve(levels, HIF4_ACT_SCALE_LEVELS)
    xk, _ = _kernel_view(x)
    _, meta = _ops.qdq_rows(xk, levels, packed=True)
    return PackedHiF4(meta["codes"], meta["scale_byte"], meta["lv2_bits"], meta["lv3_bits"])


def decode_hif4(packed: PackedHiF4, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Values of a PackedHiF4 (exact): the HIP unpack kernel over its rows."""
    codes = packed.codes
    lead = tuple(codes.shape[:-1])
    cols = codes.shape[-1] * 2
    return _ops.unpack_rows(codes, packed.scale_byte, packed.lv2_bits, packed.lv3_bits, cols, dtype).view(*lead, cols)
