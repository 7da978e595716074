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
    FAQUANT_HIF4_SCALE_LEVELS); each forward runs the activation path in one HIP launch,
    then ``F.linear`` on the HiF4-exact operands.  Without the HiSQ input rotation,
    clamp or companding that launch is ``act_qdq_rows`` (``input_scale`` in the input
    dtype, the online block Hadamard in fp32 with one cast back, the HiF4 QDQ with the ACT
    levels); with any of them it is ``act_prep_rows``, which adds the rotation (signs,
    permutation, block Hadamard; quantization.py:201-219), the clamp and the companding
    product and quotient around the QDQ (quantization.py:220-276).  The companding scale
    is computed with torch as the reference computes it (clamp to +-2.079, exp, cast to the
    input dtype).  Without a block size the online transform is the generalized one of the
    whole row (rotation.py:53-69), also in ``act_prep_rows``.

    ``packed_weight=True`` (an option of this library; in_features a multiple of 128) also
    keeps the weight as packed HiF4 rows (4.5 bits per weight, packed from the weight before
    its QDQ, so they decode to ``weight``), and inputs of at most ``packed_max_rows`` rows
    (decode steps, small batches) run the contraction from them (``linear_packed``,
    faq_hif4_linear_packed) instead of ``F.linear``: the same operands, fp32 sums in another
    (fixed) order.
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
        packed_weight: bool = False,
        packed_max_rows: int = 4,
    ) -> None:
        super().__init__()
        if quant_format != "hif4":
            raise NotImplementedError(
                f"quant_format={quant_format!r} is outside the HiF4 path of this library"
            )
        check_hif4_arguments(bits=bits, group_size=weight_group_size, symmetric=symmetric, clip_ratio=clip_ratio)
        check_hif4_arguments(bits=bits, group_size=activation_group_size, symmetric=symmetric, clip_ratio=clip_ratio)
        if (input_rotation_signs is None) != (input_rotation_permutation is None):
            raise ValueError("the input rotation needs both signs and permutation")
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
        self.register_buffer(
            "input_rotation_signs",
            None if input_rotation_signs is None else input_rotation_signs.detach().to(torch.int8).clone(),
        )
        self.register_buffer(
            "input_rotation_permutation",
            None if input_rotation_permutation is None else input_rotation_permutation.detach().long().clone(),
        )
        if self.input_rotation_permutation is not None:
            perm = self.input_rotation_permutation.reshape(-1)
            if perm.numel() != self.in_features or not torch.equal(
                    torch.sort(perm.cpu()).values, torch.arange(self.in_features)):
                raise ValueError("the input rotation permutation must be a permutation of the input features")
        self.register_buffer(
            "activation_min", None if activation_min is None else torch.as_tensor(activation_min).detach().float().clone()
        )
        self.register_buffer(
            "activation_max", None if activation_max is None else torch.as_tensor(activation_max).detach().float().clone()
        )
        self.register_buffer(
            "activation_compand_log_scale",
            None if activation_compand_log_scale is None else activation_compand_log_scale.detach().float().clone(),
        )
        weight = linear.weight.detach() if weight_override is None else weight_override.detach()
        self._packed = None
        self.packed_max_rows = int(packed_max_rows)
        if packed_weight and not quantize_weight:
            raise ValueError("packed_weight packs the weight's HiF4 QDQ: it needs quantize_weight=True")
        if packed_weight and not 0 <= self.packed_max_rows <= 8:
            raise ValueError("packed_max_rows must be in 0..8 (the packed contraction takes at most 8 rows)")
        if quantize_weight:
            from . import _ops
            from .hif4 import HIF4_SCALE_LEVELS

            source_device = weight.device
            gpu = weight if weight.device.type == "cuda" else weight.to("cuda")
            if packed_weight:
                # packed from the weight before its QDQ (a second QDQ of the result could
                # choose another scale), with the QDQ's levels: decodes to the weight below
                self._packed = _ops.PackedHiF4Weight(gpu, HIF4_SCALE_LEVELS)
            weight = fake_quantize(gpu, quant_format=quant_format, bits=bits, group_size=weight_group_size,
                                   symmetric=symmetric, clip_ratio=clip_ratio, hif4_levels=HIF4_SCALE_LEVELS)
            weight = weight.to(device=source_device, dtype=linear.weight.dtype)
        self.weight = torch.nn.Parameter(weight.detach().clone(), requires_grad=False)
        if linear.bias is None:
            self.register_parameter("bias", None)
        else:
            self.bias = torch.nn.Parameter(linear.bias.detach().clone(), requires_grad=False)

    def _prep_vectors(self, x: torch.Tensor):
        """The per-feature vectors of the activation path in the kernel's forms (int32
        permutation; the companding scale computed as the reference does: clamp to +-2.079,
        exp, cast to x's dtype, then held as fp32; its reciprocals for the kernel's product
        form of the final division) and the clamp bounds as floats, cached per device and
        dtype and recomputed when a buffer is modified in place or replaced."""
        tensors = (self.input_rotation_permutation, self.activation_compand_log_scale, self.activation_min,
                   self.activation_max)
        key = (x.device, x.dtype) + tuple(None if t is None else t._version for t in tensors)
        cached = getattr(self, "_prep_cache", None)
        # the cache holds the buffer objects themselves, so a replaced buffer never matches
        if cached is not None and cached[0] == key and all(a is b for a, b in zip(cached[2], tensors)):
            return cached[1]
        perm = None
        if self.input_rotation_permutation is not None:
            perm = self.input_rotation_permutation.to(device=x.device, dtype=torch.int32).contiguous()
        compand = rcp = None
        if self.activation_compand_log_scale is not None:
            log_scale = self.activation_compand_log_scale
            if log_scale.numel() != self.in_features:
                if self.in_features % log_scale.numel():
                    raise RuntimeError("invalid activation companding shape")
                log_scale = log_scale.repeat_interleave(self.in_features // log_scale.numel())
            compand = log_scale.clamp(-2.079, 2.079).exp().to(device=x.device, dtype=x.dtype).float().contiguous()
            from . import _ops

            rcp = _ops.act_compand_rcp(compand, x.dtype)
        bounds = (None if self.activation_min is None else float(self.activation_min),
                  None if self.activation_max is None else float(self.activation_max))
        value = (perm, compand, bounds, rcp)
        self._prep_cache = (key, value, tensors)
        return value

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from . import _ops
        from .hif4 import HIF4_ACT_SCALE_LEVELS

        block = int(self.online_hadamard_block_size or 0) if self.online_hadamard else 0
        generalized = bool(self.online_hadamard) and self.online_hadamard_block_size is None
        extra = (self.input_rotation_signs is not None or self.activation_min is not None
                 or self.activation_max is not None or self.activation_compand_log_scale is not None)
        if not extra and not generalized and block <= 512:
            xq = _ops.act_qdq_rows(x, levels=HIF4_ACT_SCALE_LEVELS, hadamard=block, col_scale=self.input_scale)
        else:
            perm, compand, bounds, rcp = self._prep_vectors(x)
            xq = _ops.act_prep_rows(
                x, levels=HIF4_ACT_SCALE_LEVELS, col_scale=self.input_scale, rot_signs=self.input_rotation_signs,
                rot_perm=perm, rot_block=self.input_rotation_block_size, act_min=bounds[0], act_max=bounds[1],
                compand=compand, hadamard=block, hadamard_generalized=generalized, compand_rcp=rcp)
        packed = self._packed
        if (packed is not None and xq.dtype == torch.bfloat16 and xq.device == packed.device
                and xq.numel() <= self.packed_max_rows * self.in_features):
            # few rows: the contraction reads the packed weight (faq_hif4_linear_packed)
            return _lib.forward_only(_ops.linear_packed(xq, packed, self.bias), x)
        return torch.nn.functional.linear(_lib.forward_only(xq, x), self.weight, self.bias)
