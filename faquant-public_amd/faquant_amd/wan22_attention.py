"""HiF4 QK/PV attention for the Wan2.2 DiT on the MI355X: drop-in for faquant.wan22_attention.

Reference: src/faquant/wan22_attention.py.  Same public names and signatures:
  * ``qdq_rows_128(x, block_rows=64)``                 :97-102 (3-level HiF4 of [R, 128] fp32)
  * ``hif4_attention(q, k, v, *, softmax_scale, quantize_p, quantized_normalizer,
    block_m, num_warps, num_stages)``                   :165-183 (non-causal, [L, H, 128] bf16)
  * ``rotate_heads(x, chunk_rows)``                     :186-192 (128-point Hadamard, one bf16 cast)
  * ``make_flash_attention(input_qdq, *, quantized_normalizer, qk_rotation, fallback)``
                                                         :195-228 (drop-in for Wan's flash_attention)
``block_m``, ``num_warps`` and ``num_stages`` were Triton tuning knobs; they are
accepted and ignored.  P is quantized with the three-level format, as the
reference kernel's in-register quantizer is.

``make_flash_attention`` fuses rotation, Q/K/V QDQ and attention into two HIP
launches when ``input_qdq`` comes from ``faquant_qdq`` (it carries its levels);
any other callable is applied as given between the rotation and the kernel.

``patch_attention_modules(model_module, collector)`` (:231-270) installs the same
per-module settings on Wan's attention classes.  A self-attention's
``faquant_qk_smooth_scale`` multiplies Q and divides K in fp32 after RoPE; when the
module's ``flash_attention`` is this drop-in, that step runs inside its fused prologue
(fp32 smooth, Hadamard, one bf16 cast, QDQ in one pass per operand) instead of as a
separate elementwise pass, with the same result.
"""

from __future__ import annotations

import contextvars
from typing import Callable

import torch

from . import _lib, _ops
from .hif4 import fake_quantize_hif4

KEY_TILE = _ops.KEY_TILE
R7 = 0.142578125  # bf16(1/7), the three-level divisor reciprocal
_BF16_ATTENTION = contextvars.ContextVar("faquant_bf16_attention", default=False)
# Smooth-QK scale handed from a patched self-attention to this module's flash_attention
_SMOOTH_QK = contextvars.ContextVar("faquant_smooth_qk", default=None)


class faquant_qdq:  # noqa: N801 - named after the reference's factory (wan22_hif4.py:35-36)
    """HiF4 QDQ callable with known levels, so the attention prologue can fuse it."""

    def __init__(self, levels: str) -> None:
        self.levels = levels

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return fake_quantize_hif4(x, levels=self.levels)


def qdq_rows_128(x: torch.Tensor, block_rows: int = 64) -> torch.Tensor:
    """Three-level HiF4 QDQ of an [R, 128] tensor in fp32 (the in-kernel quantizer)."""
    del block_rows
    x = x.contiguous().float()
    return _ops.qdq_rows(x, "123")


def _as_bhld(t: torch.Tensor) -> torch.Tensor:
    """[L, H, D] or [B, L, H, D] -> a [B, H, L, D] view."""
    return t.unsqueeze(0).transpose(1, 2) if t.ndim == 3 else t.transpose(1, 2)


def hif4_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    softmax_scale: float | None = None,
    quantize_p: bool = True,
    quantized_normalizer: bool = False,
    block_m: int = 128,
    num_warps: int = 8,
    num_stages: int = 1,
) -> torch.Tensor:
    """Non-causal attention of [L, H, D] bf16 tensors (Q/K/V already quantized); bf16 out."""
    del block_m, num_warps, num_stages
    lq, heads, dim = q.shape
    lk = k.shape[0]
    assert dim == 128 and k.shape == v.shape and k.shape[1:] == (heads, dim)
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16 and q.stride(-1) == k.stride(-1) == v.stride(-1) == 1
    scale = float(softmax_scale if softmax_scale is not None else dim**-0.5)
    out = torch.empty_like(q)
    vt = _ops.operand_prep_vt(_as_bhld(v), levels=None)
    _ops.attention_fwd(
        _as_bhld(q), _as_bhld(k), vt, lk, causal=False, scale=scale, quant_p=quantize_p,
        p_levels="123", norm_same=quantized_normalizer, out=_as_bhld(out),
    )
    return _lib.forward_only(out, q, k, v)


def rotate_heads(x: torch.Tensor, chunk_rows: int = 1 << 16) -> torch.Tensor:
    """Normalized Hadamard over head_dim in fp32, cast once to bf16."""
    del chunk_rows
    return _ops.hadamard_rows(x, x.shape[-1], torch.bfloat16)


def make_flash_attention(
    input_qdq: Callable[[torch.Tensor], torch.Tensor],
    *,
    quantized_normalizer: bool = False,
    qk_rotation: bool = False,
    fallback: Callable | None = None,
) -> Callable:
    """A drop-in for ``wan.modules.attention.flash_attention`` with HiF4 Q/K/P/V."""

    def flash_attention(q, k, v, q_lens=None, k_lens=None, dropout_p=0., softmax_scale=None, q_scale=None,
                        causal=False, window_size=(-1, -1), deterministic=False, dtype=torch.bfloat16,
                        version=None):
        fused_prologue = (isinstance(input_qdq, faquant_qdq) and dtype == torch.bfloat16
                          and q.shape[-1] == _ops.HEAD_DIM)
        smooth = _SMOOTH_QK.get()
        # Q diag(s), K diag(s)^-1 ahead of everything else (exact for Q K^T).  The fused
        # prologue computes it in fp32, which is the reference's q * s for an fp32 scale (the
        # product promotes to fp32); any other case scales here, in the reference's dtypes.
        out_dtype = q.dtype if smooth is None else torch.promote_types(q.dtype, smooth.dtype)
        if smooth is not None and (not fused_prologue or smooth.dtype != torch.float32
                                   or (fallback is not None and _BF16_ATTENTION.get())):
            q, k = q * smooth, k / smooth
            smooth = None
        if fallback is not None and _BF16_ATTENTION.get():
            return fallback(q, k, v, q_lens=q_lens, k_lens=k_lens, dropout_p=dropout_p, softmax_scale=softmax_scale,
                            q_scale=q_scale, causal=causal, window_size=window_size, deterministic=deterministic,
                            dtype=dtype, version=version)
        assert dropout_p == 0 and q_scale is None and not causal and tuple(window_size) == (-1, -1)
        inputs = (q, k, v)
        batch, lq, lk = q.size(0), q.size(1), k.size(1)
        for lens, full in ((q_lens, lq), (k_lens, lk)):
            if lens is not None and any(int(n) != full for n in lens.tolist()):
                raise NotImplementedError("variable sequence lengths are not supported")
        dim = q.shape[-1]
        scale = float(softmax_scale if softmax_scale is not None else dim**-0.5)
        if fused_prologue:
            # (Smooth-QK) -> rotation (fp32) -> one bf16 cast -> HiF4 QDQ, in one pass per operand
            rot = _ops.HEAD_DIM if qk_rotation else 0
            qh, _ = _ops.operand_prep(_as_bhld(q), levels=input_qdq.levels, hadamard=rot, smooth=smooth,
                                      round_dtype=torch.bfloat16)
            kh, _ = _ops.operand_prep(_as_bhld(k), levels=input_qdq.levels, hadamard=rot, smooth=smooth,
                                      smooth_divide=True, round_dtype=torch.bfloat16)
            vt = _ops.operand_prep_vt(_as_bhld(v.to(dtype)), levels=input_qdq.levels)
        else:
            if qk_rotation:
                q, k = rotate_heads(q), rotate_heads(k)
            q, k, v = (input_qdq(t.to(dtype)) for t in (q, k, v))
            qh = _as_bhld(q.to(torch.bfloat16))
            kh = _as_bhld(k.to(torch.bfloat16))
            vt = _ops.operand_prep_vt(_as_bhld(v.to(torch.bfloat16)), levels=None)
        out = torch.empty((batch, lq, q.shape[2], dim), device=q.device, dtype=torch.bfloat16)
        _ops.attention_fwd(
            qh, kh, vt, lk, causal=False, scale=scale, quant_p=True, p_levels="123",
            norm_same=quantized_normalizer, out=_as_bhld(out),
        )
        return _lib.forward_only(out.type(out_dtype), *inputs)

    flash_attention.faquant_fuses_smooth_qk = True
    return flash_attention


def patch_attention_modules(model_module, collector: Callable | None = None) -> None:
    """Per-module attention settings for ``wan.modules.model`` (wan22_attention.py:231-270):

    - ``faquant_qk_smooth_scale`` (head_dim, or [heads, head_dim]) on a WanSelfAttention:
      Q times it and K divided by it after RoPE, in fp32 before the Hadamard and the bf16
      cast.  With this module's ``flash_attention`` installed the step runs in its fused
      prologue; any other ``flash_attention`` receives the scaled fp32 Q/K, as in the
      reference;
    - ``faquant_attention_bf16 = True`` routes that module's attention to the fallback;
    - ``collector(module, q, k)`` sees every self-attention call's post-RoPE Q/K.
    """
    rope_apply = model_module.rope_apply

    def attend(module, smooth, *args, **kwargs):
        fa = model_module.flash_attention
        if smooth is not None and not getattr(fa, "faquant_fuses_smooth_qk", False):
            q, k = kwargs["q"], kwargs["k"]
            kwargs["q"], kwargs["k"] = q * smooth, k / smooth
            smooth = None
        t_bf16 = _BF16_ATTENTION.set(bool(getattr(module, "faquant_attention_bf16", False)))
        t_smooth = _SMOOTH_QK.set(smooth)
        try:
            return fa(*args, **kwargs)
        finally:
            _SMOOTH_QK.reset(t_smooth)
            _BF16_ATTENTION.reset(t_bf16)

    def self_forward(self, x, seq_lens, grid_sizes, freqs):
        b, s, n, d = *x.shape[:2], self.num_heads, self.head_dim
        q = rope_apply(self.norm_q(self.q(x)).view(b, s, n, d), grid_sizes, freqs)
        k = rope_apply(self.norm_k(self.k(x)).view(b, s, n, d), grid_sizes, freqs)
        v = self.v(x).view(b, s, n, d)
        if collector is not None:
            collector(self, q, k)
        y = attend(self, getattr(self, "faquant_qk_smooth_scale", None), q=q, k=k, v=v, k_lens=seq_lens,
                   window_size=self.window_size)
        return self.o(y.flatten(2))

    def cross_forward(self, x, context, context_lens):
        b, n, d = x.size(0), self.num_heads, self.head_dim
        q = self.norm_q(self.q(x)).view(b, -1, n, d)
        k = self.norm_k(self.k(context)).view(b, -1, n, d)
        v = self.v(context).view(b, -1, n, d)
        return self.o(attend(self, None, q, k, v, k_lens=context_lens).flatten(2))

    model_module.WanSelfAttention.forward = self_forward
    model_module.WanCrossAttention.forward = cross_forward
