"""Tensor-level launchers over the C ABI: allocate outputs, check shapes, launch.

All tensors must live on a ROCm device; every launch is enqueued on the current
torch stream of that device.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

HEAD_DIM = 128
KEY_TILE = 128


def _checked_out(out: torch.Tensor | None, like: torch.Tensor, shape=None, dtype=None, unit_last_only=False):
    """``out`` if it can take the result (device, dtype, shape, and contiguous or, with
    ``unit_last_only``, a unit last stride), else a ValueError; a new tensor when None."""
    shape = tuple(like.shape) if shape is None else tuple(shape)
    dtype = like.dtype if dtype is None else dtype
    if out is None:
        return torch.empty(shape, device=like.device, dtype=dtype)
    if out.device != like.device or out.dtype != dtype or tuple(out.shape) != shape:
        raise ValueError(f"out must be a {dtype} tensor of shape {shape} on {like.device}")
    if not (out.stride(-1) == 1 if unit_last_only else out.is_contiguous()):
        raise ValueError("out must be contiguous" if not unit_last_only else "out must have a unit last stride")
    return out

def _pad_keys(length: int) -> int:
    return max(KEY_TILE, (length + KEY_TILE - 1) // KEY_TILE * KEY_TILE)


def qdq_rows(
    x: torch.Tensor,
    levels: str,
    *,
    out: torch.Tensor | None = None,
    compact: bool = False,
    packed: bool = False,
):
    """HiF4 QDQ of ``x`` along its last axis (any leading shape); returns y (and metadata).

    ``compact`` adds (scale, rec, lv2, lv3) shaped like the reference's
    CompactHiF4Parameters for the grouped view [..., groups, 64]; ``packed`` adds
    (codes [..., C/2] uint8, scale_byte, lv2_bits, lv3_bits).
    """
    _lib.require_device(x)
    lib = _lib.load()
    cols = x.shape[-1]
    if x.ndim == 0:
        raise ValueError("HiF4 fake quantization requires at least one dimension")
    if cols == 0:
        raise ValueError("HiF4 fake quantization does not support an empty axis")
    xc = x.contiguous()
    rows = xc.numel() // cols
    y = _checked_out(out, xc)
    groups = (cols + 63) // 64
    lead = tuple(x.shape[:-1])
    extra = {}
    if compact:
        extra["scale"] = torch.empty(lead + (groups, 1, 1, 1), device=x.device, dtype=torch.float32)
        extra["rec"] = torch.empty_like(extra["scale"])
        extra["lv2"] = torch.empty(lead + (groups, 8, 1, 1), device=x.device, dtype=torch.int8)
        extra["lv3"] = torch.empty(lead + (groups, 8, 2, 1), device=x.device, dtype=torch.int8)
    if packed:
        if cols % 64:
            raise ValueError("packed HiF4 codes need a width that is a multiple of 64")
        extra["codes"] = torch.empty(lead + (cols // 2,), device=x.device, dtype=torch.uint8)
        extra["scale_byte"] = torch.empty(lead + (groups,), device=x.device, dtype=torch.uint8)
        extra["lv2_bits"] = torch.empty(lead + (groups,), device=x.device, dtype=torch.uint8)
        extra["lv3_bits"] = torch.empty(lead + (groups,), device=x.device, dtype=torch.uint16)
    g = extra.get
    _lib.check(
        lib.faq_hif4_qdq_rows(
            xc.data_ptr(), y.data_ptr(), rows, cols, _lib.dtype_code(x.dtype), int(levels),
            _lib.ptr(g("scale")), _lib.ptr(g("rec")), _lib.ptr(g("lv2")), _lib.ptr(g("lv3")),
            _lib.ptr(g("codes")), _lib.ptr(g("scale_byte")), _lib.ptr(g("lv2_bits")), _lib.ptr(g("lv3_bits")),
            _lib.stream_ptr(x.device),
        )
    )
    y = y.view(x.shape)
    if not extra:
        return y
    return y, extra


def unpack_rows(codes, scale_byte, lv2_bits, lv3_bits, cols: int, dtype: torch.dtype) -> torch.Tensor:
    """Packed HiF4 rows -> values [rows, cols] in ``dtype`` (exact)."""
    _lib.require_device(codes, scale_byte, lv2_bits, lv3_bits)
    lib = _lib.load()
    if cols % 64:
        raise ValueError("HiF4 packing needs a last axis that is a multiple of 64")
    c = codes.contiguous()
    rows = c.numel() // (cols // 2) if cols else 0
    y = torch.empty((rows, cols), device=codes.device, dtype=dtype)
    parts = [t.contiguous() for t in (scale_byte, lv2_bits, lv3_bits)]
    _lib.check(
        lib.faq_hif4_unpack_rows(
            c.data_ptr(), parts[0].data_ptr(), parts[1].data_ptr(), parts[2].data_ptr(), rows, cols,
            _lib.dtype_code(dtype), y.data_ptr(), _lib.stream_ptr(codes.device),
        )
    )
    return y


def hadamard_rows(x: torch.Tensor, block: int, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Block Hadamard over the last axis in fp32, rounded once to ``out_dtype``."""
    _lib.require_device(x)
    lib = _lib.load()
    xc = x.contiguous()
    cols = x.shape[-1]
    rows = xc.numel() // cols if cols else 0
    y = torch.empty(x.shape, device=x.device, dtype=out_dtype or x.dtype)
    _lib.check(
        lib.faq_hadamard_rows(
            xc.data_ptr(), y.data_ptr(), rows, cols, int(block), _lib.dtype_code(x.dtype),
            _lib.dtype_code(y.dtype), _lib.stream_ptr(x.device),
        )
    )
    return y


def hadamard_rows_native(x: torch.Tensor) -> torch.Tensor:
    """Normalized Hadamard over the last axis of a bf16 / fp16 tensor computed in that dtype
    (every butterfly stage rounded to it, rotation.py:14-29 on such a tensor)."""
    _lib.require_device(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("hadamard_rows_native takes bf16 or fp16")
    xc = x.contiguous()
    y = torch.empty_like(xc)
    cols = x.shape[-1]
    _lib.check(_lib.load().faq_hadamard_rows_native(xc.data_ptr(), y.data_ptr(), xc.numel() // max(cols, 1), cols,
                                                     _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device)))
    return y.view(x.shape)


def act_prep_rows(
    x: torch.Tensor,
    *,
    levels: str | None,
    col_scale: torch.Tensor | None = None,
    rot_signs: torch.Tensor | None = None,
    rot_perm: torch.Tensor | None = None,
    rot_block: int | None = None,
    act_min: float | None = None,
    act_max: float | None = None,
    compand: torch.Tensor | None = None,
    hadamard: int = 0,
    hadamard_generalized: bool = False,
    out: torch.Tensor | None = None,
    compand_rcp: torch.Tensor | None = None,
    stage_round: bool = False,
) -> torch.Tensor:
    """The full activation path of a quantized Linear along the last axis of ``x``
    (faq_act_prep_rows): x * dtype(col_scale); the HiSQ input rotation (fp32 x times
    ``rot_signs``, gathered by ``rot_perm``, the per-block fp32 Hadamard of ``rot_block``
    values when set, one cast back); the clamp to [act_min, act_max] in x's dtype; x times
    ``compand`` (already in x's dtype); the online block Hadamard of ``hadamard`` values, or
    with ``hadamard_generalized`` the generalized transform of the whole row (rotation.py:
    53-69: a power of two or 12 times one); HiF4 QDQ with ``levels``; x / ``compand``.
    Output in x's dtype.  ``compand_rcp`` is ``act_compand_rcp(compand, x.dtype)``, computed
    here when not given (callers that keep the scale keep it too).  ``stage_round`` runs the
    online transform in x's dtype (each butterfly stage and the 12-point mix rounded to it,
    as the reference's transforms on a bf16 / fp16 tensor)."""
    _lib.require_device(x, col_scale, rot_signs, rot_perm, compand, compand_rcp)
    lib = _lib.load()
    if x.ndim == 0:
        raise ValueError("HiF4 fake quantization requires at least one dimension")
    cols = x.shape[-1]
    xc = x.contiguous()
    rows = xc.numel() // cols if cols else 0
    y = _checked_out(out, xc)
    keep = []

    def vec(t, dtype, name):
        if t is None:
            return None
        v = t.to(device=x.device, dtype=dtype).reshape(-1).contiguous()
        if v.numel() != cols:
            raise ValueError(f"{name} must hold {cols} values, got {v.numel()}")
        if v.data_ptr() % 16:  # the kernel reads these vectors 16 bytes at a time
            v = v.clone()
        keep.append(v)
        return v.data_ptr()

    if (rot_signs is None) != (rot_perm is None):
        raise ValueError("the input rotation needs both signs and permutation")
    if compand is not None and compand_rcp is None and rows > 0:
        compand_rcp = act_compand_rcp(compand.to(device=x.device, dtype=torch.float32).reshape(-1), x.dtype)
    opts = _lib.ActOpts(
        col_scale=vec(col_scale, torch.float32, "input scale"),
        rot_signs=vec(rot_signs, torch.int8, "rotation signs"),
        rot_perm=vec(rot_perm, torch.int32, "rotation permutation"),
        rot_block=int(rot_block or 0),
        has_min=int(act_min is not None),
        has_max=int(act_max is not None),
        act_min=float(act_min) if act_min is not None else 0.0,
        act_max=float(act_max) if act_max is not None else 0.0,
        compand=vec(compand, torch.float32, "companding scale"),
        hadamard=int(hadamard or 0),
        hadamard_generalized=int(bool(hadamard_generalized)),
        compand_rcp=vec(compand_rcp, torch.float32, "companding reciprocal") if compand is not None else None,
        stage_round=int(bool(stage_round)),
    )
    _lib.check(
        lib.faq_act_prep_rows(
            xc.data_ptr(), y.data_ptr(), rows, cols, _lib.dtype_code(x.dtype), ctypes.byref(opts),
            int(levels) if levels else 0, _lib.stream_ptr(x.device),
        )
    )
    del keep
    return y.view(x.shape)


def act_compand_rcp(compand: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """fp32 reciprocals of a companding scale (fp32 values of ``dtype``) where the activation
    kernel's product form of x / scale is exact for ``dtype``, 0 elsewhere
    (faq_act_compand_rcp)."""
    _lib.require_device(compand)
    lib = _lib.load()
    c = compand.to(torch.float32).reshape(-1).contiguous()
    rcp = torch.empty_like(c)
    _lib.check(lib.faq_act_compand_rcp(c.data_ptr(), rcp.data_ptr(), c.numel(), _lib.dtype_code(dtype),
                                       _lib.stream_ptr(c.device)))
    return rcp


def act_qdq_rows(
    x: torch.Tensor,
    *,
    levels: str | None,
    hadamard: int = 0,
    col_scale: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Activation prologue of a W4A4 Linear along the last axis of ``x`` (any leading
    shape, fp32 / bf16 / fp16): x * dtype(col_scale), optional block Hadamard in fp32 with
    one cast back, HiF4 QDQ with ``levels`` (None: none).  Output in x's dtype."""
    _lib.require_device(x, col_scale)
    lib = _lib.load()
    if x.ndim == 0:
        raise ValueError("HiF4 fake quantization requires at least one dimension")
    cols = x.shape[-1]
    xc = x.contiguous()
    rows = xc.numel() // cols if cols else 0
    y = _checked_out(out, xc)
    sc = None
    if col_scale is not None:
        sc = col_scale.to(device=x.device, dtype=torch.float32).reshape(-1).contiguous()
        if sc.numel() != cols:
            raise ValueError(f"input scale must hold {cols} values, got {sc.numel()}")
    _lib.check(
        lib.faq_act_qdq_rows(
            xc.data_ptr(), y.data_ptr(), rows, cols, _lib.dtype_code(x.dtype), _lib.ptr(sc), int(hadamard),
            int(levels) if levels else 0, _lib.stream_ptr(x.device),
        )
    )
    return y.view(x.shape)


def pquant_groups(p: torch.Tensor, levels: str) -> torch.Tensor:
    """The attention kernel's in-register P quantizer on given non-negative fp32 values
    ``p[..., 64 n]`` (contiguous), in 64-value groups along the last axis: the HiF4 QDQ of P
    along keys (sfa:801-806) through the same device code as attention_fwd."""
    _lib.require_device(p)
    if p.dtype != torch.float32 or not p.is_contiguous() or p.ndim == 0 or p.shape[-1] % 64:
        raise ValueError("pquant_groups needs a contiguous fp32 tensor whose last axis is a multiple of 64")
    out = torch.empty_like(p)
    _lib.check(_lib.load().faq_pquant_groups(p.data_ptr(), out.data_ptr(), p.numel() // 64, int(levels),
                                              _lib.stream_ptr(p.device)))
    return out


def _bhld_strides(x: torch.Tensor) -> tuple[int, int, int]:
    if x.stride(-1) != 1:
        raise ValueError("operands need a unit stride along head_dim")
    return x.stride(0), x.stride(1), x.stride(2)


def operand_prep(
    x: torch.Tensor,
    *,
    levels: str | None,
    hadamard: int = 0,
    key_offset: torch.Tensor | None = None,
    smooth: torch.Tensor | None = None,
    smooth_divide: bool = False,
    round_dtype: torch.dtype | None = None,
    want_rotated: bool = False,
    out: torch.Tensor | None = None,
):
    """Q/K operand prologue on x [B, H, L, 128] (any strides, unit last stride).

    Returns the bf16 operand [B, H, L, 128] (or writes ``out``) and, when
    ``want_rotated``, the rotated tensor in ``round_dtype`` before quantization.
    """
    _lib.require_device(x, key_offset, smooth)
    lib = _lib.load()
    if x.ndim != 4 or x.shape[-1] != HEAD_DIM:
        raise NotImplementedError("the HIP operand prologue supports [B, H, L, 128] tensors")
    B, H, L, _ = x.shape
    sb, sh, sl = _bhld_strides(x)
    rdt = round_dtype or x.dtype
    y = _checked_out(out, x, (B, H, L, HEAD_DIM), torch.bfloat16, unit_last_only=True)
    rot = torch.empty((B, H, L, HEAD_DIM), device=x.device, dtype=rdt) if want_rotated else None

    def per_head(t):
        if t is None:
            return None, 0
        t = t.to(device=x.device, dtype=torch.float32).contiguous()
        if t.numel() == HEAD_DIM:
            return t.reshape(HEAD_DIM), 0
        if t.numel() == H * HEAD_DIM:
            return t.reshape(H, HEAD_DIM), HEAD_DIM
        raise ValueError(f"per-dim tensor must hold 128 or H*128 values, got shape {tuple(t.shape)}")

    off, off_sh = per_head(key_offset)
    sm, sm_sh = per_head(smooth)
    _lib.check(
        lib.faq_operand_prep(
            x.data_ptr(), _lib.dtype_code(x.dtype), sb, sh, sl, B, H, L,
            _lib.ptr(off), off_sh, _lib.ptr(sm), sm_sh, int(bool(smooth_divide)), int(hadamard),
            _lib.dtype_code(rdt), _lib.ptr(rot), y.data_ptr(), y.stride(0), y.stride(1), y.stride(2),
            int(levels) if levels else 0, _lib.stream_ptr(x.device),
        )
    )
    return y, rot


class PackedHiF4KV:
    """A packed HiF4 K or V cache (faq_hif4_kv): one row of 128 values per (batch, head,
    position) at 4.5 bits per value, ``codes`` int32 [B, H, capacity, 16] and ``meta`` int32
    [B, H, capacity, 2]; rows 0..length-1 are valid.  Written by ``pack_operand``, read by
    ``attention_decode``; it decodes to the bf16 HiF4 QDQ values of the same prologue."""

    def __init__(self, batch: int, heads: int, capacity: int, device, levels: str) -> None:
        self.codes = torch.empty((batch, heads, capacity, 16), device=device, dtype=torch.int32)
        self.meta = torch.empty((batch, heads, capacity, 2), device=device, dtype=torch.int32)
        self.length = 0
        self.levels = levels

    @property
    def shape(self) -> tuple:
        """Logical shape [B, H, length, 128] of the values held."""
        return (self.codes.shape[0], self.codes.shape[1], self.length, HEAD_DIM)

    @property
    def capacity(self) -> int:
        return self.codes.shape[2]

    @property
    def device(self) -> torch.device:
        return self.codes.device

    def nbytes(self) -> int:
        """Bytes of the valid rows (72 per row: 4.5 bits per value)."""
        return self.codes.shape[0] * self.codes.shape[1] * self.length * 72

    def grow(self, capacity: int) -> "PackedHiF4KV":
        """A copy with room for `capacity` rows (the valid rows copied)."""
        B, H = self.codes.shape[:2]
        g = PackedHiF4KV(B, H, capacity, self.device, self.levels)
        g.codes[:, :, : self.length].copy_(self.codes[:, :, : self.length])
        g.meta[:, :, : self.length].copy_(self.meta[:, :, : self.length])
        g.length = self.length
        return g

    def descriptor(self) -> "_lib.HiF4KV":
        if self.codes.stride(3) != 1 or self.codes.stride(2) != 16 or self.meta.stride(2) != 2:
            raise ValueError("packed HiF4 rows must be contiguous")
        rows_b, rows_h = self.codes.stride(0) // 16, self.codes.stride(1) // 16
        if (self.meta.stride(0) // 2, self.meta.stride(1) // 2) != (rows_b, rows_h):
            raise ValueError("packed HiF4 codes and meta must share row strides")
        return _lib.HiF4KV(self.codes.data_ptr(), self.meta.data_ptr(), rows_b, rows_h)


def pack_operand(
    x: torch.Tensor,
    *,
    levels: str,
    out: PackedHiF4KV,
    start: int = 0,
    hadamard: int = 0,
    key_offset: torch.Tensor | None = None,
    smooth: torch.Tensor | None = None,
    smooth_divide: bool = False,
    round_dtype: torch.dtype | None = None,
) -> PackedHiF4KV:
    """The operand prologue of ``operand_prep`` on x [B, H, L, 128] with the HiF4 QDQ
    written packed into rows start .. start + L - 1 of ``out`` (faq_operand_prep_hif4_kv)."""
    _lib.require_device(x, key_offset, smooth)
    lib = _lib.load()
    if x.ndim != 4 or x.shape[-1] != HEAD_DIM:
        raise NotImplementedError("the HIP operand prologue supports [B, H, L, 128] tensors")
    B, H, L, _ = x.shape
    if tuple(out.codes.shape[:2]) != (B, H) or start < 0 or start + L > out.capacity:
        raise ValueError(f"rows {start}..{start + L} of a packed cache of shape {tuple(out.codes.shape[:3])}")
    if not levels:
        raise ValueError("the packed HiF4 form needs HiF4 levels")
    sb, sh, sl = _bhld_strides(x)
    rdt = round_dtype or x.dtype
    off, off_sh = _per_head(key_offset, H, x.device)
    sm, sm_sh = _per_head(smooth, H, x.device)
    d = out.descriptor()
    _lib.check(
        lib.faq_operand_prep_hif4_kv(
            x.data_ptr(), _lib.dtype_code(x.dtype), sb, sh, sl, B, H, L,
            _lib.ptr(off), off_sh, _lib.ptr(sm), sm_sh, int(bool(smooth_divide)), int(hadamard),
            _lib.dtype_code(rdt), int(levels), d.codes + start * 64, d.meta + start * 8, d.sb, d.sh,
            _lib.stream_ptr(x.device),
        )
    )
    out.length = max(out.length, start + L)
    return out


class PackedHiF4Weight:
    """A Linear weight W [N, K] kept as packed HiF4 rows (4.5 bits per weight) for
    ``linear_packed``: row n * (K / 128) + j of ``rows`` (a PackedHiF4KV of one batch and head)
    holds columns 128 j .. 128 j + 127 of output feature n.  Packed from the weight before its
    QDQ (``pack_operand`` with the weight's levels), so it decodes to the HiF4 weight QDQ of
    FakeQuantLinear (quantization.py:164-191) bitwise; packing an already quantized weight
    would not (a second QDQ can pick a finer E6M2 scale)."""

    def __init__(self, weight: torch.Tensor, levels: str) -> None:
        _lib.require_device(weight)
        if weight.ndim != 2 or weight.shape[1] % HEAD_DIM:
            raise NotImplementedError("packed HiF4 weights need [out_features, in_features] with in_features a "
                                      "multiple of 128")
        N, K = weight.shape
        self.shape = (N, K)
        self.levels = levels
        self.rows = PackedHiF4KV(1, 1, N * (K // HEAD_DIM), weight.device, levels)
        w = weight.detach().contiguous()
        pack_operand(w.view(1, 1, N * (K // HEAD_DIM), HEAD_DIM), levels=levels, out=self.rows, round_dtype=w.dtype)

    @property
    def device(self) -> torch.device:
        return self.rows.device

    def nbytes(self) -> int:
        return self.rows.nbytes()


LINEAR_PACKED_MAX_ROWS = 8  # faq_hif4_linear_packed takes at most this many rows of x


def linear_packed(x: torch.Tensor, weight: PackedHiF4Weight, bias: torch.Tensor | None = None, *,
                  out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y = x W^T (+ bias) with W packed (faq_hif4_linear_packed): x bf16 [..., K] (the HiF4
    activation QDQ) with at most LINEAR_PACKED_MAX_ROWS rows, y [..., N] in ``out_dtype``
    (default x's dtype; fp32 or bf16).  fp32 sums in a fixed order on every call; not bitwise
    the library GEMM of F.linear, whose fp32 sums run in another order."""
    _lib.require_device(x, bias)
    lib = _lib.load()
    N, K = weight.shape
    if x.dtype != torch.bfloat16:
        raise NotImplementedError("the packed-weight Linear takes bf16 activations")
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} features, the weight {K}")
    out_dtype = out_dtype or x.dtype
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        # a fresh copy: contiguous() returns a contiguous view that starts off alignment as is
        x2 = x2.clone(memory_format=torch.contiguous_format)
    M = x2.shape[0]
    y = torch.empty((M, N), device=x.device, dtype=out_dtype)
    if M:
        b = None if bias is None else bias.detach().contiguous()
        d = weight.rows.descriptor()
        _lib.check(
            lib.faq_hif4_linear_packed(
                x2.data_ptr(), x2.stride(0), d.codes, d.meta, None if b is None else b.data_ptr(),
                0 if b is None else _lib.dtype_code(b.dtype), y.data_ptr(), _lib.dtype_code(out_dtype), y.stride(0),
                M, N, K, _lib.stream_ptr(x.device),
            )
        )
    return y.view(*x.shape[:-1], N)


def _per_head(t, H: int, device):
    """A per-dim fp32 tensor of 128 or H*128 values as (tensor, head stride)."""
    if t is None:
        return None, 0
    t = t.to(device=device, dtype=torch.float32).contiguous()
    if t.numel() == HEAD_DIM:
        return t.reshape(HEAD_DIM), 0
    if t.numel() == H * HEAD_DIM:
        return t.reshape(H, HEAD_DIM), HEAD_DIM
    raise ValueError(f"per-dim tensor must hold 128 or H*128 values, got shape {tuple(t.shape)}")


def operand_prep_vt(v: torch.Tensor, *, levels: str | None) -> torch.Tensor:
    """V [B, H, L, 128] -> HiF4-QDQ'd, transposed bf16 [B, H, 128, Lpad] (zero padded)."""
    _lib.require_device(v)
    lib = _lib.load()
    if v.ndim != 4 or v.shape[-1] != HEAD_DIM:
        raise NotImplementedError("the HIP operand prologue supports [B, H, L, 128] tensors")
    B, H, L, _ = v.shape
    sb, sh, sl = _bhld_strides(v)
    lpad = _pad_keys(L)
    vt = torch.empty((B, H, HEAD_DIM, lpad), device=v.device, dtype=torch.bfloat16)
    _lib.check(
        lib.faq_operand_prep_vt(
            v.data_ptr(), _lib.dtype_code(v.dtype), sb, sh, sl, B, H, L, lpad, vt.data_ptr(),
            int(levels) if levels else 0, _lib.stream_ptr(v.device),
        )
    )
    return vt


@dataclass
class KeyRanges:
    """Per-row key ranges and valid-key bits of the attention kernel's key-range mode:
    query position p of batch b sees the keys k in [row_lo[b, p], row_hi[b, p]] whose bit
    k % 32 of key_bits[b, k // 32] is set."""

    row_lo: torch.Tensor      # int32 [B, Lq]
    row_hi: torch.Tensor      # int32 [B, Lq]
    row_blocks: torch.Tensor  # int32 [B, ceil(Lq / 32), 4]: per-32-position summaries
    key_bits: torch.Tensor    # int32 [B, key_words], key_words = 4 * ceil(Lk / 128)


def attention_key_ranges(
    mask: torch.Tensor | None,
    batch: int,
    query_length: int,
    key_length: int,
    *,
    causal: bool,
    window: int | None = None,
    device: torch.device | None = None,
) -> KeyRanges:
    """Key ranges of a 2-D attention mask (sfa:341-368 plus the rank form of sfa:371-427):
    ``mask`` holds the last ``key_length`` columns of the caller's [B, L] mask (nonzero =
    valid; a leading dimension of 1 broadcasts over the batch), or None for every key
    valid.  ``window`` is the sliding window (None: none)."""
    lib = _lib.load()
    if mask is not None:
        _lib.require_device(mask)
        device = mask.device
        if mask.ndim != 2 or mask.shape[-1] != key_length:
            raise ValueError("the 2-D mask slice must be [B, key_length]")
        if mask.shape[0] not in (1, batch):
            raise ValueError("2-D attention mask batch does not match the query batch")
        mask = mask.to(torch.bool)
        if mask.shape[0] != batch:
            mask = mask.expand(batch, key_length)
        if mask.stride(-1) != 1 or (batch > 1 and mask.stride(0) < key_length):
            mask = mask.contiguous()
    if device is None:
        raise ValueError("attention_key_ranges needs a device when mask is None")
    if window is not None and window <= 0:
        raise ValueError("sliding_window must be positive")
    words = 4 * max(1, -(-key_length // KEY_TILE))
    row_lo = torch.empty((batch, query_length), device=device, dtype=torch.int32)
    row_hi = torch.empty_like(row_lo)
    row_blocks = torch.empty((batch, -(-query_length // 32), 4), device=device, dtype=torch.int32)
    key_bits = torch.empty((batch, words), device=device, dtype=torch.int32)
    _lib.check(
        lib.faq_attention_mask_bounds(
            _lib.ptr(mask), mask.stride(0) if mask is not None and batch > 1 else key_length,
            batch, query_length, key_length, int(bool(causal)), int(window or 0),
            row_lo.data_ptr(), row_hi.data_ptr(), row_blocks.data_ptr(), key_bits.data_ptr(), words,
            _lib.stream_ptr(device),
        )
    )
    return KeyRanges(row_lo, row_hi, row_blocks, key_bits)


def dense_attention_mask(mask: torch.Tensor, batch: int, heads: int, query_length: int,
                         key_length: int) -> torch.Tensor:
    """The kernel's form of a 3-D/4-D attention mask (sfa:430-454): fp32
    [B or 1, Hq or 1, Lq or 1, Lpad], 0 / the additive value where allowed, -inf where the
    reference masks (boolean False, -inf, or <= finfo.min / 2), -inf past key_length.
    Query rows are the mask's last query_length rows (one row broadcasts); keys are its
    first key_length columns."""
    if mask.ndim == 3:
        mask = mask[:, None]
    if mask.ndim != 4:
        raise ValueError("attention mask must be rank 2, 3, or 4")
    mq = mask.shape[-2]
    if mq == 1:
        rows = slice(0, 1)
    elif mq >= query_length:
        rows = slice(mq - query_length, mq)
    else:
        raise ValueError("4-D attention mask is shorter than the query sequence")
    if mask.shape[0] not in (1, batch) or mask.shape[1] not in (1, heads) or mask.shape[-1] < key_length:
        raise ValueError("4-D attention mask does not broadcast to the attention scores")
    m = mask[..., rows, :key_length]
    if m.dtype == torch.bool or not m.is_floating_point():
        add = torch.zeros(m.shape, device=m.device, dtype=torch.float32).masked_fill(~m.to(torch.bool), -math.inf)
    else:
        invalid = torch.isneginf(m) | (m <= torch.finfo(m.dtype).min / 2)
        add = m.to(torch.float32).masked_fill(invalid, -math.inf)
    out = torch.full((*m.shape[:-1], _pad_keys(key_length)), -math.inf, device=m.device, dtype=torch.float32)
    out[..., :key_length] = add
    return out


def raw_q_operand_ok(q: torch.Tensor, hadamard: int | None) -> bool:
    """Whether attention_fwd's q_prep can take these query rows as they are: bf16 [B, H, L,
    128] with unit stride along head_dim, strides of multiples of 8 elements, 16-byte
    aligned, and a Hadamard block of 0, 64 or 128."""
    return (q.dtype == torch.bfloat16 and q.ndim == 4 and q.shape[-1] == HEAD_DIM and q.stride(-1) == 1
            and all(q.stride(i) % 8 == 0 for i in range(3)) and q.data_ptr() % 16 == 0
            and int(hadamard or 0) in (0, 64, 128))


def _attn_opts(ranges: KeyRanges | None, softcap: float | None, pv_probe: torch.Tensor | None = None,
               dense_mask: torch.Tensor | None = None, p_dump: torch.Tensor | None = None,
               q_prep: tuple[int, str | None] | None = None):
    if (ranges is None and not softcap and pv_probe is None and dense_mask is None and p_dump is None
            and q_prep is None):
        return None
    opts = _lib.AttnOpts()
    if q_prep is not None:
        opts.q_prep = 1
        opts.q_hadamard = int(q_prep[0] or 0)
        opts.q_levels = int(q_prep[1]) if q_prep[1] else 0
    opts.pv_probe = _lib.ptr(pv_probe)
    if p_dump is not None:
        opts.p_dump = p_dump.data_ptr()
        opts.p_dump_stride = p_dump.shape[-1]
    if dense_mask is not None:
        opts.dense_mask = dense_mask.data_ptr()
        sb, sh, sq = (dense_mask.stride(i) if dense_mask.shape[i] > 1 else 0 for i in range(3))
        opts.dm_sb, opts.dm_sh, opts.dm_sq = sb, sh, sq
    if ranges is not None:
        opts.row_lo = ranges.row_lo.data_ptr()
        opts.row_hi = ranges.row_hi.data_ptr()
        opts.row_blocks = ranges.row_blocks.data_ptr()
        opts.key_bits = ranges.key_bits.data_ptr()
        opts.key_words = ranges.key_bits.shape[-1]
    opts.softcap = float(softcap or 0.0)
    return ctypes.byref(opts), opts


def attention_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    vt: torch.Tensor,
    key_length: int,
    *,
    causal: bool,
    scale: float,
    quant_p: bool,
    p_levels: str,
    norm_same: bool,
    out: torch.Tensor,
    row_den: torch.Tensor | None = None,
    out_levels: str | None = None,
    split: int | None = None,
    ranges: KeyRanges | None = None,
    softcap: float | None = None,
    pv_probe: torch.Tensor | None = None,
    dense_mask: torch.Tensor | None = None,
    p_dump: torch.Tensor | None = None,
    q_prep: tuple[int, str | None] | None = None,
) -> torch.Tensor:
    """Attention over bf16 operands q [B, Hq, Lq, 128], k [B, Hkv, Lk, 128] and
    vt [B, Hkv, 128, Lpad]; writes ``out`` (a [B, Hq, Lq, 128] view, fp32 or bf16).
    ``out_levels`` adds a HiF4 QDQ of each 64-value half of every output row, after its
    rounding to the output dtype (the o_proj-input quantizer, qwen3.py:167-171).
    ``ranges`` (attention_key_ranges) replaces the causal flag by per-row key ranges;
    ``softcap`` > 0 caps the scores (sfa:725-727).  ``pv_probe`` (fp32 [B, Hq, Lq, 5],
    needs ``quant_p``) receives the PV-normalizer probe's per-row sums: sum P^, sum P,
    #(P^ = 0 < P), sum (P^ - P)^2, sum P^2 (sfa:36-185, 835-869); it runs one pass.
    ``dense_mask`` (dense_attention_mask) is a 3-D/4-D mask: added to the scaled scores in
    place of the causal rule (sfa:730-757).  ``p_dump`` (fp32 [B, Hq, Lq, 2, W], W a
    multiple of 4 and >= 128 * ceil(Lk / 128), needs ``quant_p``) receives the kernel's P
    and P^ for every key of every key tile a row processes (verification of the in-register
    quantizer); it runs one pass.  ``q_prep = (hadamard, levels)`` takes the raw bf16 query
    rows and applies ``operand_prep(q, levels=levels, hadamard=hadamard,
    round_dtype=torch.bfloat16)``'s steps inside the kernel as each work item loads them
    (hadamard 0, 64 or 128; levels None for no QDQ): the same bits without the separate pass
    over Q."""
    _lib.require_device(q, k, vt, out, row_den)
    if softcap is not None and softcap < 0:
        raise ValueError("softcap must be non-negative")
    if dense_mask is not None:
        _lib.require_device(dense_mask)
        if ranges is not None:
            raise ValueError("a dense mask and key ranges are exclusive")
        if (dense_mask.dtype != torch.float32 or dense_mask.ndim != 4 or dense_mask.stride(-1) != 1
                or dense_mask.shape[-1] < _pad_keys(int(key_length))):
            raise ValueError("dense_mask must be fp32 [B|1, Hq|1, Lq|1, Lpad] with unit key stride")
    if ranges is None and softcap and dense_mask is None:
        ranges = attention_key_ranges(None, q.shape[0], q.shape[2], int(key_length), causal=causal,
                                      device=q.device)
    if ranges is not None:
        _lib.require_device(ranges.row_lo, ranges.row_hi, ranges.key_bits)
        if tuple(ranges.row_lo.shape) != (q.shape[0], q.shape[2]) or tuple(ranges.row_hi.shape) != tuple(
            ranges.row_lo.shape
        ):
            raise ValueError("key ranges must be [B, Lq]")
    if pv_probe is not None:
        _lib.require_device(pv_probe)
        if pv_probe.dtype != torch.float32 or tuple(pv_probe.shape) != (q.shape[0], q.shape[1], q.shape[2], 5) \
                or not pv_probe.is_contiguous():
            raise ValueError("pv_probe must be a contiguous fp32 [B, Hq, Lq, 5] tensor")
        split = 1
    if p_dump is not None:
        _lib.require_device(p_dump)
        width = p_dump.shape[-1] if p_dump.ndim == 5 else -1
        if (p_dump.dtype != torch.float32 or tuple(p_dump.shape[:4]) != (q.shape[0], q.shape[1], q.shape[2], 2)
                or not p_dump.is_contiguous() or width % 4 or width < _pad_keys(int(key_length))):
            raise ValueError("p_dump must be a contiguous fp32 [B, Hq, Lq, 2, W] tensor, W >= 128 * ceil(Lk / 128)")
        split = 1
    held = _attn_opts(ranges, softcap, pv_probe, dense_mask, p_dump, q_prep)
    opts = held[0] if held else None
    lib = _lib.load()
    B, Hq, Lq, D = q.shape
    Hkv = k.shape[1]
    if D != HEAD_DIM or k.shape[-1] != HEAD_DIM:
        raise NotImplementedError(f"the HIP attention kernel supports head_dim 128, got {D}")
    _check_attention_tensors(q, out, row_den, B, Hq, Lq)
    if k.shape[0] != B or k.shape[2] < int(key_length) or tuple(vt.shape[:3]) != (B, Hkv, HEAD_DIM):
        raise ValueError("k must be [B, Hkv, >= key_length, 128] and vt [B, Hkv, 128, Lpad]")
    for t in (q, k, vt):
        if t.dtype != torch.bfloat16:
            raise TypeError("attention operands must be bf16")
    if out.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("attention output must be fp32 or bf16")
    qs, ks_, vs = _bhld_strides(q), _bhld_strides(k), _bhld_strides(vt)
    os_ = (out.stride(0), out.stride(1), out.stride(2))
    if out.stride(3) != 1:
        raise ValueError("attention output needs a unit stride along head_dim")
    nsplit = _split_count(B, Hq, Hkv, Lq, int(key_length), _device_cus(q.device)) if split is None else int(split)
    if nsplit > 1 and not out_levels:
        ws_bytes = lib.faq_attention_split_workspace(B, Hq, Lq, int(key_length), nsplit)
        ws = torch.empty(max(int(ws_bytes), 16), device=q.device, dtype=torch.uint8)
        _lib.check(
            lib.faq_attention_fwd_split(
                q.data_ptr(), *qs, k.data_ptr(), *ks_, vt.data_ptr(), *vs, vt.shape[-1],
                out.data_ptr(), _lib.dtype_code(out.dtype), *os_,
                B, Hq, Hkv, Lq, int(key_length), int(bool(causal)), float(scale),
                int(bool(quant_p)), int(p_levels), int(bool(norm_same)), _lib.ptr(row_den),
                nsplit, ws.data_ptr(), ws.numel(), opts, _lib.stream_ptr(q.device),
            )
        )
        return out
    _lib.check(
        lib.faq_attention_fwd(
            q.data_ptr(), *qs, k.data_ptr(), *ks_, vt.data_ptr(), *vs, vt.shape[-1],
            out.data_ptr(), _lib.dtype_code(out.dtype), *os_,
            B, Hq, Hkv, Lq, int(key_length), int(bool(causal)), float(scale),
            int(bool(quant_p)), int(p_levels), int(bool(norm_same)), _lib.ptr(row_den),
            int(out_levels) if out_levels else 0, opts, _lib.stream_ptr(q.device),
        )
    )
    return out



GENERAL_MAX_DIM = 256
GENERAL_MAX_TILE = 1024


def attention_general(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    key_tile: int,
    causal: bool,
    scale: float,
    quant_p: bool,
    p_levels: str,
    norm_same: bool,
    out: torch.Tensor,
    row_den: torch.Tensor | None = None,
    ranges: KeyRanges | None = None,
    softcap: float | None = None,
    pv_probe: torch.Tensor | None = None,
    dense_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """The simulator's recurrence (sfa:457-909) for what attention_fwd does not take: any
    head_dim up to 256, key tiles of 1..1024 keys, and fp32, bf16 or fp16 operands multiplied
    in fp32.  q [B, Hq, Lq, D], k and v [B, Hkv, Lk, D] (natural layout, already quantized
    where the caller quantizes), ``out`` a [B, Hq, Lq, D] view (fp32 or bf16).  The masking
    arguments and ``pv_probe`` mean what they mean for attention_fwd."""
    _lib.require_device(q, k, v, out, row_den)
    if softcap is not None and softcap < 0:
        raise ValueError("softcap must be non-negative")
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    if k.shape != v.shape or k.shape[0] != B or k.shape[-1] != D:
        raise ValueError("k and v must be [B, Hkv, Lk, D] with the query's batch and head_dim")
    if D > GENERAL_MAX_DIM:
        raise NotImplementedError(f"the MI355X attention supports head_dim up to {GENERAL_MAX_DIM}, got {D}")
    if not 1 <= key_tile <= GENERAL_MAX_TILE:
        raise NotImplementedError(f"the MI355X attention supports key chunks of 1 to {GENERAL_MAX_TILE} keys, "
                                  f"got {key_tile}")
    for t in (q, k, v):
        if t.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise TypeError("attention operands must be fp32, bf16 or fp16")
        if t.stride(-1) != 1:
            raise ValueError("attention operands need a unit stride along head_dim")
    if out.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError("attention output must be fp32, bf16 or fp16")
    if tuple(out.shape) != (B, Hq, Lq, D) or out.stride(-1) != 1:
        raise ValueError("out must be a [B, Hq, Lq, D] view with a unit stride along head_dim")
    if row_den is not None and (row_den.dtype != torch.float32 or tuple(row_den.shape) != (B, Hq, Lq)
                                or not row_den.is_contiguous()):
        raise ValueError("row_den must be a contiguous fp32 [B, Hq, Lq] tensor")
    if dense_mask is not None:
        _lib.require_device(dense_mask)
        if ranges is not None:
            raise ValueError("a dense mask and key ranges are exclusive")
        if (dense_mask.dtype != torch.float32 or dense_mask.ndim != 4 or dense_mask.stride(-1) != 1
                or dense_mask.shape[-1] < Lk):
            raise ValueError("dense_mask must be fp32 [B|1, Hq|1, Lq|1, >= Lk] with unit key stride")
    if ranges is not None:
        _lib.require_device(ranges.row_lo, ranges.row_hi, ranges.key_bits)
        if tuple(ranges.row_lo.shape) != (B, Lq) or tuple(ranges.row_hi.shape) != (B, Lq):
            raise ValueError("key ranges must be [B, Lq]")
    if pv_probe is not None:
        _lib.require_device(pv_probe)
        if pv_probe.dtype != torch.float32 or tuple(pv_probe.shape) != (B, Hq, Lq, 5) \
                or not pv_probe.is_contiguous():
            raise ValueError("pv_probe must be a contiguous fp32 [B, Hq, Lq, 5] tensor")
    held = _attn_opts(ranges, softcap, pv_probe, dense_mask)
    opts = held[0] if held else None
    lib = _lib.load()
    code = _lib.dtype_code
    _lib.check(
        lib.faq_attention_fwd_general(
            q.data_ptr(), code(q.dtype), *_bhld_strides(q), k.data_ptr(), code(k.dtype), *_bhld_strides(k),
            v.data_ptr(), code(v.dtype), *_bhld_strides(v), out.data_ptr(), code(out.dtype),
            out.stride(0), out.stride(1), out.stride(2),
            B, Hq, Hkv, Lq, Lk, D, int(key_tile), int(bool(causal)), float(scale),
            int(bool(quant_p)), int(p_levels), int(bool(norm_same)), _lib.ptr(row_den), opts,
            _lib.stream_ptr(q.device),
        )
    )
    return out


def _check_attention_tensors(q, out, row_den, B, Hq, Lq):
    """The output and row denominators must cover every query row the kernels write."""
    if tuple(out.shape) != (B, Hq, Lq, HEAD_DIM):
        raise ValueError(f"attention output must be [B, Hq, Lq, 128] = {(B, Hq, Lq, HEAD_DIM)}, got {tuple(out.shape)}")
    if row_den is not None and (row_den.dtype != torch.float32 or not row_den.is_contiguous()
                                or tuple(row_den.shape) != (B, Hq, Lq)):
        raise ValueError("row_den must be a contiguous fp32 [B, Hq, Lq] tensor")

def decode_shaped(Hq: int, Hkv: int, Lq: int) -> bool:
    """Whether faq_attention_decode takes a call: all query rows of a KV head (G heads x Lq
    positions) fit one wave's 32 MFMA columns, so every K/V tile is read once."""
    G = Hq // Hkv
    return G <= 32 and Lq * G <= 32


def decode_split_count(B: int, Hkv: int, Lk: int, cus: int = 256, packed: bool = False) -> int:
    """Key ranges of faq_attention_decode: about eight waves per CU (two per SIMD) over all
    (batch, KV head, range) work, at least one key tile per range, no empty range.  For
    bf16 K/V a range of one tile becomes two where that still leaves four waves per CU: the
    second tile's loads then fly during the first one's work.  Packed K/V (a quarter of the
    bytes per tile) keep one tile per range.  Measured at 32k keys, Qwen3-8B heads: bf16
    36.6 us with two tiles per range against 42.7 with one; packed 31.5 us with one against
    34.3 with two; at 8k, with two waves per CU left, one tile per range stays faster."""
    ntiles = -(-Lk // KEY_TILE)
    if ntiles == 0:
        return 1
    work = max(1, B * Hkv)
    want = max(1, min(ntiles, 4096, -(-8 * cus // work)))
    tps = -(-ntiles // want)
    if not packed and tps == 1 and work * -(-ntiles // 2) >= 4 * cus:
        tps = 2
    return -(-ntiles // tps)


def attention_decode(
    q: torch.Tensor,
    key_length: int,
    *,
    causal: bool,
    scale: float,
    quant_p: bool,
    p_levels: str,
    norm_same: bool,
    out: torch.Tensor,
    k: torch.Tensor | None = None,
    v: torch.Tensor | None = None,
    packed: tuple[PackedHiF4KV, PackedHiF4KV] | None = None,
    row_den: torch.Tensor | None = None,
    split: int | None = None,
) -> torch.Tensor:
    """Decode-shaped attention (faq_attention_decode): q [B, Hq, Lq, 128] bf16 against bf16
    k and v [B, Hkv, Lk, 128] (natural rows, any strides with a unit last stride), or against
    ``packed`` = (K cache, V cache) of PackedHiF4KV; masks none or bottom-right causal.  Same
    results as attention_fwd's split path with the same ``split``, bitwise, for either form
    of K/V."""
    tensors = (q, out, row_den) + ((k, v) if packed is None else (packed[0].codes, packed[1].codes))
    _lib.require_device(*tensors)
    lib = _lib.load()
    B, Hq, Lq, D = q.shape
    if D != HEAD_DIM or q.dtype != torch.bfloat16:
        raise NotImplementedError("the decode kernel takes bf16 queries with head_dim 128")
    _check_attention_tensors(q, out, row_den, B, Hq, Lq)
    if out.dtype not in (torch.float32, torch.bfloat16) or out.stride(3) != 1:
        raise ValueError("attention output must be fp32 or bf16 with a unit stride along head_dim")
    Lk = int(key_length)
    if packed is None:
        if k is None or v is None or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise TypeError("bf16 k and v are required without packed K/V")
        if (k.shape[-2] < Lk or v.shape[-2] < Lk or k.shape[-1] != HEAD_DIM or v.shape[-1] != HEAD_DIM
                or k.shape[0] != B or v.shape[0] != B or v.shape[1] != k.shape[1]):
            raise ValueError("k and v must be [B, Hkv, >= key_length, 128]")
        Hkv = k.shape[1]
        kargs = (k.data_ptr(), *_bhld_strides(k), v.data_ptr(), *_bhld_strides(v))
        kp = vp = None
    else:
        kc, vc = packed
        Hkv = kc.codes.shape[1]
        if (kc.length < Lk or vc.length < Lk or vc.codes.shape[1] != Hkv or kc.codes.shape[0] != B
                or vc.codes.shape[0] != B):
            raise ValueError("the packed K/V caches must hold key_length rows of the same heads")
        kargs = (0, 0, 0, 0, 0, 0, 0, 0)
        kp, vp = kc.descriptor(), vc.descriptor()
    nsplit = decode_split_count(B, Hkv, Lk, _device_cus(q.device), packed is not None) if split is None else int(split)
    ws_bytes = lib.faq_attention_decode_workspace(B, Hq, Lq, Lk, nsplit)
    ws = torch.empty(max(int(ws_bytes), 16), device=q.device, dtype=torch.uint8)
    _lib.check(
        lib.faq_attention_decode(
            q.data_ptr(), *_bhld_strides(q), *kargs,
            None if kp is None else ctypes.byref(kp), None if vp is None else ctypes.byref(vp),
            out.data_ptr(), _lib.dtype_code(out.dtype), out.stride(0), out.stride(1), out.stride(2),
            B, Hq, Hkv, Lq, Lk, int(bool(causal)), float(scale), int(bool(quant_p)), int(p_levels),
            int(bool(norm_same)), _lib.ptr(row_den), nsplit, ws.data_ptr(), ws.numel(), _lib.stream_ptr(q.device),
        )
    )
    return out


_CUS: dict = {}
SPLIT_MAX_TILES = 16384  # the split path's scan holds one row's tile maxima in LDS


def _device_cus(device) -> int:
    """Compute units of a device (cached): the attention kernel runs one workgroup per CU."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _CUS:
        _CUS[key] = int(torch.cuda.get_device_properties(key).multi_processor_count)
    return _CUS[key]


def _split_count(B: int, Hq: int, Hkv: int, Lq: int, Lk: int, cus: int = 256) -> int:
    """Key ranges for decode-sized queries (Lq <= 64) whose work items cannot fill the CUs:
    the one-pass kernel runs one 256-row work item per (KV head group, 256/hpw positions).
    The split count gives each CU one item (cus / items ranges), each range at least one key
    tile.  Longer query blocks keep the one-pass kernel, so a prefill fed in chunks stays
    bitwise equal to one pass."""
    G = Hq // Hkv
    hpw = 8 if G % 8 == 0 else 4 if G % 4 == 0 else 2 if G % 2 == 0 else 1
    wgs = B * Hkv * (G // hpw) * -(-Lq // (256 // hpw))
    ntiles = -(-Lk // KEY_TILE)
    if Lq > 64 or 2 * wgs > cus or ntiles < 4 or ntiles > SPLIT_MAX_TILES:
        return 1
    return max(2, min(cus // wgs, ntiles))


def attention_pairs(query_length: int, key_length: int, causal: bool) -> int:
    """Unmasked (query, key) pairs; causal rows p see keys <= p + Lk - Lq."""
    if not causal:
        return query_length * key_length
    seen = np.clip(np.arange(query_length, dtype=np.int64) + (key_length - query_length) + 1, 0, key_length)
    return int(seen.sum())


def attention_flops(batch: int, heads: int, query_length: int, key_length: int, causal: bool,
                    head_dim: int = HEAD_DIM) -> float:
    """Algorithmic QK + PV FLOPs: 4 B H D N_pairs (masked-out pairs not counted)."""
    return 4.0 * batch * heads * head_dim * attention_pairs(query_length, key_length, causal)


def default_scale(head_dim: int = HEAD_DIM) -> float:
    return head_dim**-0.5


def log2e() -> float:
    return 1.0 / math.log(2.0)
