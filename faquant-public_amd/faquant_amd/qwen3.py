"""Qwen3 post-RoPE attention core on the MI355X (the hot-path part of faquant.qwen3).

Reference: src/faquant/qwen3.py:90-166, the section of ``_attention_forward``
between RoPE and ``o_proj``:
  * one fp32 excursion over Q and K: key offset, Smooth-QK scale (with optional
    ``exp(delta)``), 128-point or block Hadamard, one cast back   qwen3.py:90-130
  * the simulated flash attention call                            qwen3.py:144-166
``post_rope_qk_transform`` is that excursion as one HIP pass per operand.
``attention_core`` fuses it with the Q/K/V QDQ and runs the attention kernel:
three prologue passes and one attention launch, with the same result as the
reference's excursion followed by ``simulated_flash_attention_forward``.
Module attributes are the reference's (``faquant_qk_smooth_scale``,
``faquant_qk_smooth_delta``, ``faquant_qk_key_offset``, ``faquant_qk_rotation``,
``faquant_qk_rotation_block_size`` plus the simulator's).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib, _ops
from .config import PV_NORMALIZER_MODES
from .hif4 import HIF4_ACT_SCALE_LEVELS, HIF4_ATTN_OPERAND_SCALE_LEVELS
from .hif4 import _resolve as resolve_hif4_levels
from .quantization import check_hif4_arguments, fake_quantize
from .simulated_flash_attention import (
    _hif4_group,
    count_tiles,
    key_ranges,
    kv_operands_and_attend,
    simulated_flash_attention_forward,
)


def _block(rotation: bool, rotation_block_size: Optional[int], head_dim: int) -> int:
    if not rotation:
        return 0
    if rotation_block_size is None or rotation_block_size == head_dim:
        return head_dim
    if rotation_block_size not in (64, 128):
        raise NotImplementedError(f"Hadamard block {rotation_block_size} is not implemented on the MI355X")
    return rotation_block_size


def _smooth(smooth_scale, smooth_delta):
    if smooth_delta is not None:
        if smooth_scale is None:
            raise RuntimeError("Smooth-QK delta requires a frozen base scale")
        smooth_scale = smooth_scale * smooth_delta.float().exp()
    return smooth_scale


def post_rope_qk_transform(
    query: torch.Tensor,
    key: torch.Tensor,
    *,
    smooth_scale: Optional[torch.Tensor] = None,
    smooth_delta: Optional[torch.Tensor] = None,
    key_offset: Optional[torch.Tensor] = None,
    rotation: bool = False,
    rotation_block_size: Optional[int] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Q [B, Hq, L, 128] and K [B, Hkv, L, 128] after the qwen3.py:97-130 excursion."""
    smooth_scale = _smooth(smooth_scale, smooth_delta)
    if smooth_scale is None and key_offset is None and not rotation:
        return query, key
    block = _block(rotation, rotation_block_size, query.shape[-1])
    out = []
    for t, is_key in ((query, False), (key, True)):
        y, rot = _ops.operand_prep(
            t, levels=None, hadamard=block, key_offset=key_offset if is_key else None,
            smooth=smooth_scale, smooth_divide=is_key, round_dtype=t.dtype,
            want_rotated=t.dtype != torch.bfloat16,
        )
        out.append(y if rot is None else rot)
    return out[0], out[1]


def _output_quant_levels(module: torch.nn.Module) -> Optional[str]:
    """HiF4 levels of the attention-output (o_proj input) QDQ of qwen3.py:167-171, or None.

    Validates ``faquant_core_quant_kwargs`` like fake_quantize's HiF4 branch
    (quantization.py:30-57); other formats raise NotImplementedError.
    """
    if not getattr(module, "faquant_attention_output_quant", False):
        return None
    if getattr(getattr(module, "o_proj", None), "faquant_quantizes_input", False):
        return None
    kwargs = dict(module.faquant_core_quant_kwargs)
    if kwargs.get("quant_format", "int") != "hif4":
        fake_quantize(torch.zeros(1, 64), **kwargs)  # raises for formats outside the HiF4 path
        return None
    check_hif4_arguments(**{k: kwargs[k] for k in ("bits", "group_size", "symmetric", "clip_ratio") if k in kwargs})
    return resolve_hif4_levels(kwargs.get("hif4_levels"), HIF4_ACT_SCALE_LEVELS)


def attention_core(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    scaling: Optional[float] = None,
    attention_mask: Optional[torch.Tensor] = None,
    sliding_window: Optional[int] = None,
    cache_position: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Post-RoPE Q/K/V -> attention output [B, L, Hq, 128], fused on the GPU.

    Equivalent to the reference's excursion, the optional Q/K/V input QDQ
    (``faquant_attention_input_quant`` with ``faquant_core_quant_kwargs``, qwen3.py:132-136)
    and ``simulated_flash_attention_forward(module, q, k, v, attention_mask, scaling=scaling,
    sliding_window=sliding_window, cache_position=cache_position)`` (qwen3.py:97-166).  Keys
    past the valid length (a static cache's backing tensor beyond the mask or
    ``cache_position``) are dropped first, as the simulator does (sfa:511-520).  A 2-D
    padding mask and a sliding window run as per-row key ranges in the same fused launch;
    the input QDQ, the PV-normalizer probe and anything else the fused path does not take go
    through the drop-in.  When the module enables the attention-output quantizer
    (``faquant_attention_output_quant`` and o_proj does not quantize its own input,
    qwen3.py:167-171), the HiF4 QDQ of the output rows with ``faquant_core_quant_kwargs``
    runs in the attention kernel's epilogue.
    """
    smooth_scale = _smooth(getattr(module, "faquant_qk_smooth_scale", None),
                           getattr(module, "faquant_qk_smooth_delta", None))
    key_offset = getattr(module, "faquant_qk_key_offset", None)
    rotation = bool(getattr(module, "faquant_qk_rotation", False))
    block = _block(rotation, getattr(module, "faquant_qk_rotation_block_size", None), query.shape[-1])
    qk_quant = bool(module.faquant_qk_matmul_quant)
    pv_quant = bool(module.faquant_pv_matmul_quant)
    mode = getattr(module, "faquant_pv_normalizer_mode", "unquantized")
    if mode not in PV_NORMALIZER_MODES:
        raise ValueError(f"unsupported pv_normalizer_mode {mode!r}; expected one of {PV_NORMALIZER_MODES}")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError("sliding_window must be positive")
    valid = key.shape[-2]
    if attention_mask is not None:
        valid = min(valid, attention_mask.shape[-1])
    if isinstance(cache_position, torch.Tensor) and cache_position.numel():
        valid = min(valid, int(cache_position.max().item()) + 1)
    if valid < key.shape[-2]:
        key = key[:, :, :valid]
        value = value[:, :, :valid]
    input_quant = bool(getattr(module, "faquant_attention_input_quant", False))
    probe = pv_quant and isinstance(getattr(module, "faquant_pv_normalizer_diagnostics", None), dict)
    fused = (not input_quant and not probe and query.dtype == torch.bfloat16
             and int(module.faquant_attention_key_chunk_size) == _ops.KEY_TILE
             and (attention_mask is None or (attention_mask.ndim == 2 and attention_mask.shape[-1] == key.shape[2])))
    if not fused:
        q, k = post_rope_qk_transform(
            query, key, smooth_scale=smooth_scale, key_offset=key_offset, rotation=rotation,
            rotation_block_size=getattr(module, "faquant_qk_rotation_block_size", None),
        )
        v = value
        if input_quant:
            # the excursion's output, then the core quantizer, then the simulator's own
            # operand QDQ (HiF4 QDQ is not idempotent: both run)
            kwargs = module.faquant_core_quant_kwargs
            q, k, v = (fake_quantize(t, **kwargs) for t in (q, k, v))
        out = simulated_flash_attention_forward(module, q, k, v, attention_mask, scaling=scaling,
                                                sliding_window=sliding_window, cache_position=cache_position)[0]
        if _output_quant_levels(module) is not None:
            out = fake_quantize(out.reshape(*out.shape[:2], -1), **module.faquant_core_quant_kwargs).view(out.shape)
        return out
    quant_kwargs = module.faquant_matmul_quant_kwargs
    qk_group = _hif4_group(getattr(module, "faquant_qk_matmul_quant_kwargs", quant_kwargs), "QK") if qk_quant else 64
    pv_group = _hif4_group(getattr(module, "faquant_pv_matmul_quant_kwargs", quant_kwargs), "PV") if pv_quant else 64
    levels = HIF4_ATTN_OPERAND_SCALE_LEVELS
    q_levels = levels["q"] if qk_quant else None
    # bf16 rows without Smooth-QK: the attention kernel applies Q's prologue as it loads them
    q_prep = ((block or 0), q_levels) if smooth_scale is None and _ops.raw_q_operand_ok(query, block) else None
    if q_prep is not None:
        q_op = query
    else:
        q_op, _ = _ops.operand_prep(query, levels=q_levels, hadamard=block, smooth=smooth_scale,
                                    round_dtype=torch.bfloat16)
    B, Hq, Lq, D = query.shape
    Lk = key.shape[2]
    scale = float(scaling if scaling is not None else D**-0.5)
    causal = bool(getattr(module, "is_causal", True))
    out = torch.empty((B, Lq, Hq, D), device=query.device, dtype=query.dtype)
    ranges, masked = key_ranges(module, attention_mask, batch=B, query_length=Lq, key_length=Lk, causal=causal,
                                sliding_window=sliding_window, device=query.device)
    # K and V through the decode QDQ cache of the module (sfa:243-289), K with the same
    # post-RoPE prologue as Q
    k_prep = dict(hadamard=block, key_offset=key_offset, smooth=smooth_scale, smooth_divide=True,
                  round_dtype=torch.bfloat16)
    kv_operands_and_attend(module, q_op, key, value, query_length=Lq, qk_quant=qk_quant, pv_quant=pv_quant,
                           levels=levels, k_prep=k_prep, q_prep=q_prep, causal=causal, scale=scale, quant_p=pv_quant,
                           p_levels=levels["p"], norm_same=mode == "quantized_same", out=out.transpose(1, 2),
                           out_levels=_output_quant_levels(module), ranges=ranges)
    count_tiles(
        module.faquant_simulated_attention_stats, batch=B, query_heads=Hq, query_length=Lq, key_length=Lk,
        head_dim=D, query_chunk=int(module.faquant_attention_query_chunk_size), key_chunk=_ops.KEY_TILE,
        causal=causal,
        skip_fully_masked=bool(getattr(module, "faquant_skip_fully_masked_tiles", True)) and not masked
        and sliding_window is None,
        qk_quant=qk_quant, pv_quant=pv_quant, qk_group=qk_group, pv_group=pv_group,
    )
    return _lib.forward_only(out, query, key, value)
