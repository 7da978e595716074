"""``fake_quantize`` dispatcher: drop-in for faquant.quantization.fake_quantize (hif4 branch).

Reference: src/faquant/quantization.py:30-57.  The HiF4 branch validates its
arguments with the reference's messages and runs the HIP quantizer.  The int
and MXFP8 formats are not part of the HiF4 attention path and raise
NotImplementedError rather than silently computing something else.
"""

from __future__ import annotations

import torch

from . import _lib
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


class FakeQuantLinear(torch.nn.Module):
    """Linear with HiF4 fake-quantized weights and dynamic HiF4 inputs (W4A4).

    Drop-in for faquant.quantization.FakeQuantLinear (quantization.py:97-276) on the
    HiF4 path: the weight is quantized once at construction (levels
    FAQUANT_HIF4_SCALE_LEVELS); each forward runs the activation prologue in one HIP
    launch (``input_scale`` in the input dtype, the online block Hadamard in fp32 with one
    cast back, the HiF4 QDQ with the ACT levels), then ``F.linear`` on the HiF4-exact
    operands.  The input rotation (signs/permutation), activation clamp, companding and the
    generalized (non-block) online Hadamard raise NotImplementedError.
    """

    faquant_quantizes_input = True

    def __init__(
        self,
        linear: torch.nn.Linear,
        *,
        quant_format: str = "int",
        bits: int,
        weight_group_size: int,
        activation_group_size: int,
        symmetric: bool,
        clip_ratio: float,
        quantize_weight: bool = True,
        online_hadamard: bool = False,
        online_hadamard_block_size: int | None = None,
        input_scale: torch.Tensor | None = None,
        input_rotation_signs: torch.Tensor | None = None,
        input_rotation_permutation: torch.Tensor | None = None,
        input_rotation_block_size: int | None = None,
        weight_override: torch.Tensor | None = None,
        activation_min: float | None = None,
        activation_max: float | None = None,
        activation_compand_log_scale: torch.Tensor | None = None,
    ) -> None:
        super().__init__()
        if quant_format != "hif4":
            raise NotImplementedError(
                f"quant_format={quant_format!r} is outside the HiF4 path of this library"
            )
        check_hif4_arguments(bits=bits, group_size=weight_group_size, symmetric=symmetric, clip_ratio=clip_ratio)
        check_hif4_arguments(bits=bits, group_size=activation_group_size, symmetric=symmetric, clip_ratio=clip_ratio)
        if input_rotation_signs is not None or input_rotation_permutation is not None:
            raise NotImplementedError("the HiSQ input rotation is not implemented on the MI355X")
        if activation_min is not None or activation_max is not None:
            raise NotImplementedError("activation clamping is not implemented on the MI355X")
        if activation_compand_log_scale is not None:
            raise NotImplementedError("activation companding is not implemented on the MI355X")
        if online_hadamard and online_hadamard_block_size is None:
            raise NotImplementedError("the generalized (non-block) online Hadamard is not implemented on the MI355X")
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.quant_format = quant_format
        self.bits = bits
        self.activation_group_size = activation_group_size
        self.symmetric = symmetric
        self.clip_ratio = clip_ratio
        self.online_hadamard = online_hadamard
        self.online_hadamard_block_size = online_hadamard_block_size
        self.input_rotation_block_size = input_rotation_block_size
        self.register_buffer("input_scale", None if input_scale is None else input_scale.detach().float().clone())
        for name in ("input_rotation_signs", "input_rotation_permutation", "activation_min", "activation_max",
                     "activation_compand_log_scale"):
            self.register_buffer(name, None)
        weight = linear.weight.detach() if weight_override is None else weight_override.detach()
        if quantize_weight:
            from .hif4 import HIF4_SCALE_LEVELS

            source_device = weight.device
            gpu = weight if weight.device.type == "cuda" else weight.to("cuda")
            weight = fake_quantize(gpu, quant_format=quant_format, bits=bits, group_size=weight_group_size,
                                   symmetric=symmetric, clip_ratio=clip_ratio, hif4_levels=HIF4_SCALE_LEVELS)
            weight = weight.to(device=source_device, dtype=linear.weight.dtype)
        self.weight = torch.nn.Parameter(weight.detach().clone(), requires_grad=False)
        if linear.bias is None:
            self.register_parameter("bias", None)
        else:
            self.bias = torch.nn.Parameter(linear.bias.detach().clone(), requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from . import _ops
        from .hif4 import HIF4_ACT_SCALE_LEVELS

        block = self.online_hadamard_block_size if self.online_hadamard else 0
        xq = _ops.act_qdq_rows(x, levels=HIF4_ACT_SCALE_LEVELS, hadamard=int(block or 0), col_scale=self.input_scale)
        return torch.nn.functional.linear(_lib.forward_only(xq, x), self.weight, self.bias)
