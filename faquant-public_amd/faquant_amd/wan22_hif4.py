"""HiF4 W4A4 Linear of the Wan2.2 DiT blocks on the MI355X: drop-in for faquant.wan22_hif4.

Reference: src/faquant/wan22_hif4.py:35-92 (``BLOCK_LINEARS``, ``faquant_qdq``,
``HiF4Linear``).  The constructor keeps the reference's arguments and errors; the compute is
this build's:

- the weight's HiF4 values are produced once by the quantizer the caller passes (the HIP
  row quantizer for ``faquant_qdq``) and stored in the Linear's own dtype, refusing a dtype
  that cannot hold them exactly;
- a forward call quantizes all its rows in one launch of the HIP row quantizer when
  ``input_qdq`` is ``faquant_qdq`` (its levels are known), or one call of any other
  ``input_qdq``; the reference's row chunks only bounded the fp32 temporaries of a torch
  quantizer, which the kernel does not have (``chunk_elements`` is accepted and unused);
- the product is ``F.linear`` on the HiF4-exact operands (a library GEMM, hipBLASLt).
"""

from __future__ import annotations

from typing import Callable

import torch
from torch import nn
from torch.nn import functional as F

from . import _lib, _ops
from .wan22_attention import faquant_qdq

BLOCK_LINEARS = (
    "self_attn.q", "self_attn.k", "self_attn.v", "self_attn.o",
    "cross_attn.q", "cross_attn.k", "cross_attn.v", "cross_attn.o",
    "ffn.0", "ffn.2",
)

__all__ = ["BLOCK_LINEARS", "HiF4Linear", "faquant_qdq"]


def _hif4_rows(qdq: Callable[[torch.Tensor], torch.Tensor], rows: torch.Tensor) -> torch.Tensor:
    """QDQ of a [rows, in_features] matrix along its rows: one HIP launch for faquant_qdq."""
    if isinstance(qdq, faquant_qdq) and rows.dtype in (torch.float32, torch.bfloat16, torch.float16):
        return _ops.act_qdq_rows(rows.contiguous(), levels=qdq.levels)
    return qdq(rows)


class HiF4Linear(nn.Module):
    """A Linear whose weight holds HiF4 values and whose inputs are HiF4-quantized per call
    (wan22_hif4.py:51-92)."""

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
        del chunk_elements  # the HIP quantizer needs no row chunks
        w = linear.weight.detach()
        self.in_features, self.out_features = linear.in_features, linear.out_features
        if weight is not None and weight.shape != w.shape:
            raise ValueError(f"HiF4 weight of shape {tuple(weight.shape)} for a Linear of {tuple(w.shape)}")
        values = (_hif4_rows(weight_qdq, w.to(device=device, dtype=torch.float32)) if weight is None
                  else weight.to(device=device, dtype=torch.float32))
        held = values.to(w.dtype)
        if not torch.equal(held.float(), values.float()):
            raise RuntimeError(f"HiF4 weight is not exactly representable in {w.dtype}")
        self.weight = nn.Parameter(held.to(w.device), requires_grad=False)
        self.bias = None if linear.bias is None else nn.Parameter(linear.bias.detach().clone(), requires_grad=False)
        self.input_qdq = input_qdq
        # collector(module, quantized_rows, first_row_index): sees every call's quantized inputs
        self.collector: Callable[[nn.Module, torch.Tensor, int], None] | None = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.reshape(-1, self.in_features)
        qx = _lib.forward_only(_hif4_rows(self.input_qdq, rows), rows)
        if self.collector is not None:
            self.collector(self, qx, 0)
        return F.linear(qx, self.weight, self.bias).reshape(*x.shape[:-1], self.out_features)
