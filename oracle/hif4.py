"""numpy restatement of the reference HiF4 codec (test oracle, never shipped).

Follows ``src/faquant/hif4.py`` of the reference:
  * ``_round_to_bfloat16``               hif4.py:87-88
  * ``_e6m2_scale``                      hif4.py:91-115
  * ``fit_hif4_compact_parameters``      hif4.py:143-219 (no-op max_scale/scale_steps)
  * ``expand_hif4_parameters``           hif4.py:222-243
  * ``quantize_hif4_with_parameters``    hif4.py:255-271
  * ``_group_for_hif4`` / ``fake_quantize_hif4``  hif4.py:346-390
and the int branch of ``fake_quantize`` (quantization.py:30-94) so that the
reference's own simulator tests, which mostly run the int format, can pin the
attention oracle as well.

Every step is an IEEE float32 operation in the reference's order, so the
result is bit-exact with the reference for finite inputs.  bf16 tensors are
represented as float32 arrays whose values are bf16-representable; HiF4
outputs have at most six significant bits and are therefore exact in bf16.

Parity pins (tests/test_oracle_hif4.py): the known-answer vector of
tests/test_quantization.py:51-74 (levels 123, fp32 and bf16), golden vectors
written by the reference (tests/golden), an exhaustive sweep of the E6M2
scale over every positive finite bf16 block maximum against a closed form,
block locality and tail padding (test_quantization.py:77-85).
"""

from __future__ import annotations

import numpy as np

BLOCK = 64
LEVELS = ("123", "12", "13")

_F32 = np.float32


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32, as ``Tensor.to(bfloat16)``."""
    x = np.asarray(x, dtype=_F32)
    u = x.view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + bias) & 0xFFFF0000).astype(np.uint32)
    out = r.view(_F32)
    # NaN stays NaN (quiet); the rounding above could carry a NaN payload into inf.
    return np.where(np.isnan(x), x, out).astype(_F32)


def fp16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=_F32).astype(np.float16).astype(_F32)


def _require_levels(levels: str) -> None:
    if levels not in LEVELS:
        raise ValueError(f"HiF4 levels must be 123, 12 or 13, got {levels!r}")


def divisor_reciprocal(levels: str) -> np.float32:
    """``bf16(1 / divisor)``; divisor 7 for levels 123, 3.5 otherwise (hif4.py:102, 192)."""
    _require_levels(levels)
    divisor = 7.0 if levels == "123" else 3.5
    return bf16_round(np.array([_F32(1.0) / _F32(divisor)], dtype=_F32))[0]


def e6m2_scale(maximum: np.ndarray, levels: str = "123") -> tuple[np.ndarray, np.ndarray]:
    """E6M2 base scale and its bf16 reciprocal for block maxima (hif4.py:91-115).

    Steps: s = bf16(max * bf16(1/div)); clamp to [2^-48, 49152]; round the
    significand to two bits with ties-to-even (carry into the exponent); the
    reciprocal is the correctly rounded fp32 1/s rounded once more to bf16.
    """
    maximum = np.asarray(maximum, dtype=_F32)
    r = divisor_reciprocal(levels)
    s = bf16_round(maximum * r)
    s = np.minimum(np.maximum(s, _F32(2.0**-48)), _F32(49152.0))
    # floor(log2(s)) of a positive normal float is its unbiased exponent field.
    e = ((s.view(np.uint32) >> 23) & 0xFF).astype(np.int32) - 127
    # The explicit bf16-significand rounding (hif4.py:108-110) is the identity
    # on the bf16 value s; apply it anyway, with the same arithmetic.
    p_up = np.ldexp(_F32(1.0), 7 - e).astype(_F32)
    p_dn = np.ldexp(_F32(1.0), e - 7).astype(_F32)
    s = (np.rint(s * p_up) * p_dn).astype(_F32)
    e = ((s.view(np.uint32) >> 23) & 0xFF).astype(np.int32) - 127
    p_up = np.ldexp(_F32(1.0), 2 - e).astype(_F32)
    p_dn = np.ldexp(_F32(1.0), e - 2).astype(_F32)
    s = (np.rint(s * p_up) * p_dn).astype(_F32)  # np.rint: round half to even
    rec = bf16_round(_F32(1.0) / s)
    return s.astype(_F32), rec.astype(_F32)


def fit_compact(blocks: np.ndarray, levels: str = "123") -> dict[str, np.ndarray]:
    """Compact HiF4 metadata of ``blocks[..., 64]`` (hif4.py:143-219).

    Returns ``scale``/``reciprocal`` with shape (..., 1, 1, 1), ``lv2``
    (..., 8, 1, 1) and ``lv3`` (..., 8, 2, 1) as int8 exponents, the reference's
    ``CompactHiF4Parameters`` layout.
    """
    _require_levels(levels)
    blocks = np.asarray(blocks, dtype=_F32)
    if blocks.ndim == 0:
        raise ValueError("HiF4 parameter fitting requires at least one dimension")
    if blocks.shape[-1] != BLOCK:
        raise ValueError(
            f"HiF4 parameter fitting requires a final dimension of {BLOCK}, got {blocks.shape[-1]}"
        )
    work = blocks.reshape(*blocks.shape[:-1], 8, 2, 4)
    mag = np.abs(work)
    m3 = mag.max(axis=-1, keepdims=True)
    m2 = m3.max(axis=-2, keepdims=True)
    m1 = m2.max(axis=-3, keepdims=True)
    scale, rec = e6m2_scale(m1, levels)
    if levels == "123":
        lv2 = np.floor(np.clip(m2 * rec, 0.0, 4.0).astype(_F32) / _F32(4.0))
        lv3 = np.floor(np.clip((m3 * rec) / np.exp2(lv2).astype(_F32), 0.0, 2.0).astype(_F32) / _F32(2.0))
    elif levels == "12":
        lv2 = np.floor(np.clip(m2 * rec, 0.0, 2.0).astype(_F32) / _F32(2.0))
        lv3 = np.zeros_like(m3)
    else:
        lv2 = np.zeros_like(m2)
        lv3 = np.floor(np.clip(m3 * rec, 0.0, 2.0).astype(_F32) / _F32(2.0))
    return {
        "scale": scale,
        "reciprocal": rec,
        "lv2": lv2.astype(np.int8),
        "lv3": lv3.astype(np.int8),
    }


def quantize_blocks(blocks: np.ndarray, levels: str = "123") -> np.ndarray:
    """QDQ of ``blocks[..., 64]`` (fp32 math, fp32 result; hif4.py:222-271)."""
    blocks = np.asarray(blocks, dtype=_F32)
    p = fit_compact(blocks, levels)
    work_shape = (*blocks.shape[:-1], 8, 2, 4)
    sc2 = np.exp2(p["lv2"].astype(_F32)).astype(_F32)
    sc3 = np.exp2(p["lv3"].astype(_F32)).astype(_F32)
    qm = np.broadcast_to((p["reciprocal"] / sc2 / sc3).astype(_F32), work_shape)
    ds = np.broadcast_to((p["scale"] * sc2 * sc3).astype(_F32), work_shape)
    work = blocks.reshape(work_shape)
    t = (np.abs(work) * qm).astype(_F32)
    t = (t * _F32(4.0)).astype(_F32)
    mant = (np.floor((t + _F32(0.5)).astype(_F32)) / _F32(4.0)).astype(_F32)
    mant = np.minimum(mant, _F32(1.75))
    y = (mant * ds).astype(_F32)
    # torch.sign(x) * y: negative x gives -y (so -0.0 when the code is 0), while
    # +0.0 and -0.0 inputs give +0.0.
    y = np.where(work < 0, -y, y).astype(_F32)
    return y.reshape(blocks.shape)


def fake_quantize_hif4(x: np.ndarray, levels: str = "123", dtype: str = "float32") -> np.ndarray:
    """``fake_quantize_hif4`` along the last axis (hif4.py:377-390).

    ``x`` holds values already representable in ``dtype`` ("float32",
    "bfloat16" or "float16").  The last axis is zero-padded to a multiple of 64,
    quantized, and sliced back.  The result is returned as float32 holding
    ``dtype`` values (HiF4 results are exact in all three).
    """
    _require_levels(levels)
    x = np.asarray(x, dtype=_F32)
    if x.ndim == 0:
        raise ValueError("HiF4 fake quantization requires at least one dimension")
    size = x.shape[-1]
    if size == 0:
        raise ValueError("HiF4 fake quantization does not support an empty axis")
    pad = (-size) % BLOCK
    if pad:
        x = np.concatenate([x, np.zeros((*x.shape[:-1], pad), dtype=_F32)], axis=-1)
    grouped = x.reshape(*x.shape[:-1], -1, BLOCK)
    y = quantize_blocks(grouped, levels).reshape(x.shape)[..., :size]
    if dtype == "bfloat16":
        y = bf16_round(y)
    elif dtype == "float16":
        y = fp16_round(y)
    return np.ascontiguousarray(y, dtype=_F32)


def encode(x: np.ndarray, levels: str = "123") -> dict[str, np.ndarray]:
    """Packed HiF4 view of ``fake_quantize_hif4`` for rows whose width is a multiple of 64.

    Per value a 4-bit code (bit 3 = sign, bits 0-2 = magnitude 0..7); per
    64-block one E6M2 byte ``((e + 48) << 2) | m`` with ``scale = 2^e (1 + m/4)``,
    one byte of level-2 exponent bits (bit i = 8-group i) and 16 bits of level-3
    exponent bits (bit i = 4-group i).  ``decode`` inverts it exactly.
    """
    x = np.asarray(x, dtype=_F32)
    if x.shape[-1] % BLOCK:
        raise ValueError("encode requires a width that is a multiple of 64")
    grouped = x.reshape(*x.shape[:-1], -1, BLOCK)
    p = fit_compact(grouped, levels)
    s = p["scale"].reshape(*grouped.shape[:-1])
    bits = s.view(np.uint32)
    e = ((bits >> 23) & 0xFF).astype(np.int32) - 127
    m = ((bits >> 21) & 3).astype(np.int32)
    scale_byte = (((e + 48) << 2) | m).astype(np.uint8)
    lv2 = p["lv2"].reshape(*grouped.shape[:-1], 8).astype(np.uint32)
    lv3 = p["lv3"].reshape(*grouped.shape[:-1], 16).astype(np.uint32)
    lv2_bits = np.zeros(grouped.shape[:-1], dtype=np.uint32)
    for i in range(8):
        lv2_bits |= lv2[..., i] << i
    lv3_bits = np.zeros(grouped.shape[:-1], dtype=np.uint32)
    for i in range(16):
        lv3_bits |= lv3[..., i] << i
    y = quantize_blocks(grouped, levels)
    k = np.repeat(lv2, 8, axis=-1) + np.repeat(lv3, 4, axis=-1)
    ds = (s[..., None] * np.exp2(k.astype(_F32))).astype(_F32)
    mag = np.rint(np.abs(y) / ds * _F32(4.0)).astype(np.uint8)
    sign = (y.view(np.uint32) >> 31).astype(np.uint8)
    codes = (sign << 3) | mag
    return {
        "codes": codes.reshape(x.shape),
        "scale_byte": scale_byte,
        "lv2_bits": lv2_bits.astype(np.uint8),
        "lv3_bits": lv3_bits.astype(np.uint16),
    }


def decode(packed: dict[str, np.ndarray]) -> np.ndarray:
    """Inverse of ``encode``: float32 values of the HiF4 tensor."""
    codes = packed["codes"]
    grouped = codes.reshape(*codes.shape[:-1], -1, BLOCK)
    sb = packed["scale_byte"].astype(np.int32)
    e = (sb >> 2) - 48
    m = sb & 3
    s = np.ldexp((1.0 + m / 4.0), e).astype(_F32)
    lv2 = (packed["lv2_bits"].astype(np.uint32)[..., None] >> np.arange(8)) & 1
    lv3 = (packed["lv3_bits"].astype(np.uint32)[..., None] >> np.arange(16)) & 1
    k = np.repeat(lv2, 8, axis=-1) + np.repeat(lv3, 4, axis=-1)
    mag = (grouped & 7).astype(_F32)
    y = (mag / _F32(4.0) * s[..., None] * np.exp2(k.astype(_F32))).astype(_F32)
    y = np.where((grouped >> 3) & 1, -y, y).astype(_F32)
    return y.reshape(codes.shape)


def fake_quantize_int(
    x: np.ndarray, *, bits: int, group_size: int, symmetric: bool = True, clip_ratio: float = 1.0
) -> np.ndarray:
    """The int branch of ``fake_quantize`` (quantization.py:74-94), float32."""
    x = np.asarray(x, dtype=_F32)
    if bits >= 16:
        return x
    shape = x.shape
    g = shape[-1] if group_size == -1 else group_size
    if g <= 0 or shape[-1] % g:
        raise ValueError(f"last dimension {shape[-1]} must be divisible by group_size={group_size}")
    work = x.reshape(*shape[:-1], shape[-1] // g, g)
    eps = np.finfo(np.float32).eps
    if symmetric:
        qmax = 2 ** (bits - 1) - 1
        qmin = -(2 ** (bits - 1))
        absmax = (np.abs(work).max(axis=-1, keepdims=True) * _F32(clip_ratio)).astype(_F32)
        scale = np.maximum((absmax / _F32(qmax)).astype(_F32), _F32(eps))
        quant = np.clip(np.rint((work / scale).astype(_F32)), qmin, qmax)
        out = (quant * scale).astype(_F32)
    else:
        qmin, qmax = 0, 2**bits - 1
        xmin = np.minimum((work.min(axis=-1, keepdims=True) * _F32(clip_ratio)).astype(_F32), 0)
        xmax = np.maximum((work.max(axis=-1, keepdims=True) * _F32(clip_ratio)).astype(_F32), 0)
        scale = np.maximum(((xmax - xmin) / _F32(qmax)).astype(_F32), _F32(eps))
        zero = np.clip(np.rint((-xmin / scale).astype(_F32)), qmin, qmax)
        quant = np.clip(np.rint((work / scale + zero).astype(_F32)), qmin, qmax)
        out = ((quant - zero) * scale).astype(_F32)
    return out.reshape(shape).astype(_F32)


def fake_quantize(
    x: np.ndarray,
    *,
    quant_format: str = "int",
    bits: int = 4,
    group_size: int = -1,
    symmetric: bool = True,
    clip_ratio: float = 1.0,
    hif4_levels: str = "123",
    dtype: str = "float32",
) -> np.ndarray:
    """Dispatcher mirroring quantization.py:30-94 (hif4 and int formats)."""
    if quant_format == "hif4":
        if bits != 4:
            raise ValueError("HiF4 requires bits=4")
        if group_size not in (-1, BLOCK):
            raise ValueError("HiF4 requires group_size=64 (or -1 for direct use)")
        if not symmetric:
            raise ValueError("HiF4 does not support asymmetric quantization")
        if clip_ratio != 1.0:
            raise ValueError("HiF4 direct-cast does not support clipping")
        return fake_quantize_hif4(x, hif4_levels, dtype)
    if quant_format != "int":
        raise ValueError(f"unsupported quant_format={quant_format!r}")
    y = fake_quantize_int(x, bits=bits, group_size=group_size, symmetric=symmetric, clip_ratio=clip_ratio)
    if dtype == "bfloat16":
        y = bf16_round(y)
    elif dtype == "float16":
        y = fp16_round(y)
    return y
