"""numpy restatement of the reference's normalized Walsh-Hadamard transform (test oracle).

Follows ``src/faquant/rotation.py``:
  * ``hadamard_transform``                rotation.py:14-29
  * ``generalized_hadamard_transform``    rotation.py:53-69 (12 * 2^k sizes)
  * ``chunked_block_hadamard_transform``  rotation.py:117-135
and the two post-RoPE callers that wrap it in one fp32 excursion with a single
cast back:
  * Qwen3 attention prologue              qwen3.py:97-130
  * Wan ``rotate_heads``                  wan22_attention.py:186-192

Stage order is part of the result in floating point: strides 1, 2, ..., n/2,
each stage writing ``(left + right, left - right)`` with the left half at the
lower index, then a true fp32 division by ``fp32(sqrt(n))`` (CPU torch divides
by a Python float scalar rather than multiplying by its reciprocal).

Parity pins (tests/test_oracle_hadamard.py): the dense Sylvester-matrix closed
form in float64 (as tests/test_hisq_rotation.py:29-43 builds it), orthogonality
and self-inverse (tests/test_rotation.py:10-18), chunked-equals-full, the exact
64-point case, and golden vectors written by the reference (fp32, and bf16 / fp16
tensors with their per-stage rounding); the generalized transform by the Kronecker
closed form H12 (x) H_b in float64, its orthogonality, and activations the reference's
FakeQuantLinear wrote with it (tests/golden/linear_act.npz).
"""

from __future__ import annotations

import math

import numpy as np

_F32 = np.float32


def _is_power_of_two(v: int) -> bool:
    return v > 0 and v & (v - 1) == 0


def hadamard_transform(x: np.ndarray, stage_round=None) -> np.ndarray:
    """Normalized FWHT over the last axis, computed in x's float32 values.

    ``stage_round`` (e.g. ``hif4.bf16_round``) is the transform on a bf16 / fp16 tensor:
    torch computes each ``left + right``, ``left - right`` and the final division in
    fp32 and rounds the result to the tensor's dtype (rotation.py:21-28 in that dtype).
    """
    x = np.asarray(x, dtype=_F32)
    rnd = stage_round if stage_round is not None else (lambda a: a)
    n = x.shape[-1]
    if not _is_power_of_two(n):
        raise ValueError(f"Hadamard dimension must be a power of two, got {n}")
    out = x.reshape(-1, n).copy()
    stride = 1
    while stride < n:
        v = out.reshape(-1, n // (2 * stride), 2, stride)
        left = v[:, :, 0, :]
        right = v[:, :, 1, :]
        out = np.concatenate(((left + right)[:, :, None, :], (left - right)[:, :, None, :]), axis=2)
        out = rnd(out.reshape(-1, n).astype(_F32))
        stride *= 2
    out = rnd((out / _F32(math.sqrt(n))).astype(_F32))
    return out.reshape(x.shape)


def block_hadamard_transform(x: np.ndarray, block_size: int) -> np.ndarray:
    """``chunked_block_hadamard_transform`` before its cast back (fp32 result)."""
    x = np.asarray(x, dtype=_F32)
    if not _is_power_of_two(block_size) or x.shape[-1] % block_size:
        raise ValueError(
            f"dimension {x.shape[-1]} must be divisible by power-of-two block_size={block_size}"
        )
    return hadamard_transform(x.reshape(-1, block_size)).reshape(x.shape)


# The 12-point Hadamard matrix of rotation.py:32-50, row r as a mask of its -1 entries
# (bit h set: entry (r, h) is -1).
H12_NEG_MASKS = (0xFFE, 0x474, 0x8E8, 0x1D2, 0x3A4, 0x748, 0xE90, 0xD22, 0xA46, 0x48E, 0x91C, 0x23A)


def hadamard12() -> np.ndarray:
    """The reference's 12-point Hadamard matrix (float32 entries +-1)."""
    return np.array([[(-1.0 if (m >> h) & 1 else 1.0) for h in range(12)] for m in H12_NEG_MASKS], dtype=_F32)


def generalized_hadamard_transform(x: np.ndarray, stage_round=None) -> np.ndarray:
    """``generalized_hadamard_transform`` (rotation.py:53-69) in float32 over the last axis.

    A power-of-two size is ``hadamard_transform``.  For n = 12 b (b a power of two) the
    reference's loop pairs elements 2i, 2i + 1 and concatenates sums before differences,
    which is the unnormalized FWHT of every b-block with the stages in ``hadamard_transform``'s
    order; then the 12 x 12 matrix mixes the blocks (out[r b + c] = sum_h H12[r, h] W[h b + c]),
    summed in h order from 0 as the CPU matmul does (an fma chain: each step one rounding),
    then a true division by fp32(sqrt(n)).

    ``stage_round`` (e.g. ``hif4.bf16_round``) is the transform on a bf16 / fp16 tensor: each
    butterfly stage rounded to the dtype, the matmul's fp32 sum rounded once to it, the
    division computed in fp32 and rounded to it.
    """
    x = np.asarray(x, dtype=_F32)
    rnd = stage_round if stage_round is not None else (lambda a: a)
    n = x.shape[-1]
    if _is_power_of_two(n):
        return hadamard_transform(x, stage_round=stage_round)
    if n % 12 or not _is_power_of_two(n // 12):
        raise ValueError(f"unsupported generalized Hadamard dimension: {n}")
    b = n // 12
    w = x.reshape(-1, b).copy()
    stride = 1
    while stride < b:
        v = w.reshape(-1, b // (2 * stride), 2, stride)
        left = v[:, :, 0, :]
        right = v[:, :, 1, :]
        w = np.concatenate(((left + right)[:, :, None, :], (left - right)[:, :, None, :]), axis=2)
        w = rnd(w.reshape(-1, b).astype(_F32))
        stride *= 2
    w = w.reshape(-1, 12, b)
    h12 = hadamard12()
    out = np.zeros_like(w)
    for h in range(12):
        out = (out + h12[None, :, h, None] * w[:, h : h + 1, :]).astype(_F32)
    out = rnd(out)
    out = rnd((out.reshape(x.shape) / _F32(math.sqrt(n))).astype(_F32))
    return out


def sylvester_matrix(n: int) -> np.ndarray:
    """Unnormalized Sylvester Hadamard matrix H_n (float64), H_2n = [[H, H], [H, -H]]."""
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def qk_rotation(
    x: np.ndarray,
    *,
    block_size: int | None = None,
    smooth_scale: np.ndarray | None = None,
    smooth_is_key: bool = False,
    key_offset: np.ndarray | None = None,
    rotate: bool = True,
    out_round=None,
) -> np.ndarray:
    """The post-RoPE fp32 excursion of qwen3.py:97-130 for one operand.

    ``x`` [..., D] float32 values of the bf16 input.  Key offset (keys only) is
    subtracted, then Q is multiplied / K divided by the Smooth-QK scale, then the
    (block) Hadamard is applied, and ``out_round`` (e.g. ``bf16_round``) is the
    single cast back.
    """
    w = np.asarray(x, dtype=_F32)
    if key_offset is not None:
        w = (w - np.asarray(key_offset, dtype=_F32)).astype(_F32)
    if smooth_scale is not None:
        s = np.asarray(smooth_scale, dtype=_F32)
        w = (w / s if smooth_is_key else w * s).astype(_F32)
    if rotate:
        d = w.shape[-1]
        if block_size is None or block_size == d:
            w = hadamard_transform(w)
        else:
            w = block_hadamard_transform(w, block_size)
    return out_round(w) if out_round is not None else w
