"""Plain HiF4 W4A4 Linear for the Wan2.2 DiT blocks: drop-in for faquant.wan22_hif4.

Reference: src/faquant/wan22_hif4.py:35-92.  ``HiF4Linear`` keeps the reference's
constructor and forward: the weight is quantized once (its HiF4 values are exact in the
Linear's dtype, which is checked), inputs are quantized as they arrive in row chunks,
then ``F.linear`` on the HiF4-exact operands.  ``faquant_qdq(levels)`` returns the HIP row
quantizer; the Wan attention drop-in recognizes it and fuses it into its prologue.
"""

from __future__ import annotations

from typing import Callable

import torch
from torch import nn
from torch.nn import functional as F

from . import _lib
from .wan22_attention import faquant_qdq

BLOCK_LINEARS = (
    "self_attn.q", "self_attn.k", "self_attn.v", "self_attn.o",
    "cross_attn.q", "cross_attn.k", "cross_attn.v", "cross_attn.o",
    "ffn.0", "ffn.2",
)

__all__ = ["BLOCK_LINEARS", "HiF4Linear", "faquant_qdq"]


class HiF4Linear(nn.Module):
    """HiF4 weights (quantized once) and HiF4 inputs (quantized per call), wan22_hif4.py:51-92."""

    def __init__(
        self,
        linear: nn.Linear,
        *,
        weight_qdq: Callable[[torch.Tensor], torch.Tensor],
        input_qdq: Callable[[torch.Tensor], torch.Tensor],
        device: torch.device | str,
        chunk_elements: int = 1 << 26,
        weight: torch.Tensor | None = None,
    ) -> None:
        super().__init__()
        self.in_features, self.out_features = linear.in_features, linear.out_features
        source = linear.weight.detach()
        if weight is None:
            quantized = weight_qdq(source.to(device=device, dtype=torch.float32))
        elif weight.shape != source.shape:
            raise ValueError(f"HiF4 weight of shape {tuple(weight.shape)} for a Linear of {tuple(source.shape)}")
        else:
            quantized = weight.to(device=device, dtype=torch.float32)
        stored = quantized.to(source.dtype)
        if not torch.equal(stored.float(), quantized):
            raise RuntimeError(f"HiF4 weight is not exactly representable in {source.dtype}")
        self.weight = nn.Parameter(stored.to(source.device), requires_grad=False)
        self.bias = None if linear.bias is None else nn.Parameter(linear.bias.detach().clone(), requires_grad=False)
        self.input_qdq = input_qdq
        self.chunk_rows = max(1, chunk_elements // self.in_features)
        # called as collector(module, quantized_rows, first_row_index) for every chunk
        self.collector: Callable[[nn.Module, torch.Tensor, int], None] | None = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.reshape(-1, self.in_features)
        out = None
        for start in range(0, rows.shape[0], self.chunk_rows):
            chunk = rows[start:start + self.chunk_rows]
            part = _lib.forward_only(self.input_qdq(chunk), chunk)
            if self.collector is not None:
                self.collector(self, part, start)
            y = F.linear(part, self.weight, self.bias)
            if out is None:
                out = y.new_empty(rows.shape[0], y.shape[-1])
            out[start:start + part.shape[0]] = y
        return out.reshape(*x.shape[:-1], self.out_features)
