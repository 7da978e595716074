"""numpy restatement of the quantized Linear's activation path (test oracle only).

Follows ``FakeQuantLinear.forward`` in src/faquant/quantization.py:199-276, before the
``F.linear``:
  1. ``x * input_scale.to(x.dtype)``                                   (200-201)
  2. the HiSQ input rotation: fp32 ``x * signs``, ``index_select`` by the permutation, the
     per-block fp32 Hadamard when a block size is set, one cast back   (202-219;
     hisq_rotation.py:50-71)
  3. ``x.clamp(min, max)``: the bounds are 0-d fp32 tensors, so torch clamps in x's
     dtype with the bounds rounded to it, and NaN stays NaN             (220-221)
  4. ``x * compand_scale`` with the scale already cast to x's dtype     (222-234)
  5. the online block Hadamard in fp32 with one cast back (without a block size the
     generalized transform of the whole row, rotation.py:53-69), then the HiF4 fake
     quantizer in x's dtype, or the quantizer alone                    (235-266)
  6. ``x / compand_scale``                                             (267-268)
Every elementwise torch op on a bf16 / fp16 tensor computes in fp32 and rounds to the
dtype; on fp32 tensors the rounding is the identity.

Parity pins (tests/test_oracle_linear.py): golden vectors that the reference's
FakeQuantLinear wrote with an identity weight (tests/golden/linear_act.npz), for the
rotation with and without its block Hadamard, the clamp, companding and the online
Hadamard, in bf16 and fp32; and closed forms (the rotation is orthogonal, so it keeps
row norms in fp32 up to rounding; an all-ones sign vector with the identity permutation
and no block is the identity).
"""

from __future__ import annotations

import numpy as np

from . import hadamard as OH
from . import hif4 as OQ

_F32 = np.float32


def _rounder(dtype: str):
    if dtype == "bfloat16":
        return OQ.bf16_round
    if dtype == "float16":
        return lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    return lambda a: np.asarray(a, np.float32)


def fake_quant_linear_input(
    x: np.ndarray,
    dtype: str,
    *,
    levels: str | None = "123",
    input_scale: np.ndarray | None = None,
    rot_signs: np.ndarray | None = None,
    rot_perm: np.ndarray | None = None,
    rot_block: int | None = None,
    act_min: float | None = None,
    act_max: float | None = None,
    compand: np.ndarray | None = None,
    hadamard: int = 0,
    hadamard_generalized: bool = False,
) -> np.ndarray:
    """The activation F.linear receives, for x of values of ``dtype`` ("bfloat16",
    "float16" or "float32") given as float32.  ``compand`` is the companding scale already
    in x's dtype (the reference's ``log_scale.clamp(-2.079, 2.079).exp().to(x.dtype)``)."""
    rnd = _rounder(dtype)
    v = np.asarray(x, _F32)
    if input_scale is not None:
        v = rnd(v * rnd(np.asarray(input_scale, _F32)))
    if rot_signs is not None:
        w = v * np.asarray(rot_signs, _F32)
        w = np.take(w, np.asarray(rot_perm, np.int64), axis=-1)
        if rot_block:
            w = OH.block_hadamard_transform(w, rot_block)
        v = rnd(w)
    if act_min is not None or act_max is not None:
        lo = rnd(np.float32(act_min)) if act_min is not None else None
        hi = rnd(np.float32(act_max)) if act_max is not None else None
        nan = np.isnan(v)
        if lo is not None:
            v = np.where(v < lo, lo, v)
        if hi is not None:
            v = np.where(v > hi, hi, v)
        v = np.where(nan, np.nan, v).astype(_F32)
    c = None if compand is None else np.asarray(compand, _F32)
    if c is not None:
        v = rnd(v * c)
    if hadamard:
        v = rnd(OH.block_hadamard_transform(v, hadamard))
    elif hadamard_generalized:
        v = rnd(OH.generalized_hadamard_transform(v))
    if levels:
        v = OQ.fake_quantize_hif4(v, levels, dtype=dtype)
    if c is not None:
        v = rnd(v / c)
    return np.asarray(v, _F32)
