"""Wan self-attention patching (wan22_attention.py:231-270) with Smooth-QK fused into the
attention prologue.

A stand-in for ``wan.modules.model`` (same attribute names: q, k, v, o, norm_q, norm_k,
num_heads, head_dim, window_size; ``rope_apply``; ``flash_attention``) runs the patched
forward three ways: the drop-in's fused prologue (fp32 smooth, Hadamard, one bf16 cast,
QDQ in one pass), the same drop-in with a non-fusible quantizer (the scale applied as
q * s, k / s first, as the reference does), and an opaque flash_attention wrapper (the
patch scales before the call).  All three agree bitwise, keep the reference's fp32
output dtype, and match the oracle of the whole recipe; the bf16 fallback receives the
scaled Q/K, and the collector sees the unscaled post-RoPE Q/K.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from oracle import attention as OA
from oracle import hadamard as OH
from oracle import hif4 as OQ
from tests.test_gpu_attention import assert_close_attention

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

HEADS, DIM, L = 3, 128, 300


def _model_module():
    nn = torch.nn

    class SelfAttn(nn.Module):
        def __init__(self):
            super().__init__()
            d = HEADS * DIM
            self.q, self.k, self.v, self.o = (nn.Linear(d, d) for _ in range(4))
            self.norm_q, self.norm_k = nn.Identity(), nn.Identity()
            self.num_heads, self.head_dim, self.window_size = HEADS, DIM, (-1, -1)

    class CrossAttn(SelfAttn):
        pass

    def rope_apply(x, grid_sizes, freqs):  # a fixed position-dependent sign pattern
        return x * freqs[None, : x.shape[1], None, None]

    return SimpleNamespace(WanSelfAttention=SelfAttn, WanCrossAttention=CrossAttn, rope_apply=rope_apply,
                           flash_attention=None)


@torch.no_grad()
def test_smooth_qk_fused_equals_reference_order(dev):
    from faquant_amd.hif4 import fake_quantize_hif4
    from faquant_amd.wan22_attention import faquant_qdq, make_flash_attention, patch_attention_modules

    torch.manual_seed(3)
    mm = _model_module()
    seen = []
    patch_attention_modules(mm, collector=lambda m, q, k: seen.append((q.clone(), k.clone())))
    att = mm.WanSelfAttention().to(dev, torch.bfloat16)
    att.faquant_qk_smooth_scale = (torch.rand(HEADS, DIM, device=dev) * 1.5 + 0.5)  # fp32 buffer
    x = torch.randn(1, L, HEADS * DIM, device=dev).to(torch.bfloat16)
    freqs = torch.where(torch.arange(L, device=dev) % 3 == 0, -1.0, 1.0).to(torch.bfloat16)
    args = (x, torch.tensor([L], device=dev), None, freqs)

    fused = make_flash_attention(faquant_qdq("123"), quantized_normalizer=True, qk_rotation=True)
    unfusible = make_flash_attention(lambda t: fake_quantize_hif4(t, levels="123"), quantized_normalizer=True,
                                     qk_rotation=True)
    outs, inner = [], []
    for fa in (fused, unfusible, lambda *a, **kw: fused(*a, **kw)):
        def capture(*a, _fa=fa, **kw):
            y = _fa(*a, **kw)
            inner.append(y)
            return y
        capture.faquant_fuses_smooth_qk = getattr(fa, "faquant_fuses_smooth_qk", False)
        mm.flash_attention = capture
        with torch.autocast("cuda", dtype=torch.bfloat16):
            outs.append(att(*args))
    assert all(y.dtype == torch.float32 for y in inner)  # bf16 q times an fp32 scale: fp32, as in the reference
    assert torch.equal(inner[0], inner[1]) and torch.equal(inner[0], inner[2])
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])

    # the recipe in the oracle: q s, k / s in fp32, 128-point Hadamard, one bf16 cast, HiF4 QDQ
    q, k = (t.float().cpu().numpy() for t in seen[0])
    v = att.v(x).view(1, L, HEADS, DIM).float().cpu().numpy()
    s = att.faquant_qk_smooth_scale.cpu().numpy()
    qr = OQ.bf16_round(OH.hadamard_transform((q * s[None, None]).astype(np.float32)))
    kr = OQ.bf16_round(OH.hadamard_transform((k / s[None, None]).astype(np.float32)))
    t = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))  # noqa: E731
    ref = OA.simulated_flash_attention(t(qr), t(kr), t(v), OA.SimConfig(pv_normalizer_mode="quantized_same",
                                                                          is_causal=False), dtype="bfloat16")
    assert_close_attention(inner[0].float().cpu().numpy(), ref, "wan smooth-qk recipe")


@torch.no_grad()
def test_bf16_fallback_receives_scaled_qk(dev):
    from faquant_amd.wan22_attention import faquant_qdq, make_flash_attention, patch_attention_modules

    torch.manual_seed(4)
    mm = _model_module()
    patch_attention_modules(mm)
    att = mm.WanSelfAttention().to(dev, torch.bfloat16)
    att.faquant_qk_smooth_scale = torch.rand(DIM, device=dev) + 0.5
    att.faquant_attention_bf16 = True
    got = {}

    def fallback(q, k, v, **kw):
        got.update(q=q, k=k)
        return torch.zeros_like(q)

    mm.flash_attention = make_flash_attention(faquant_qdq("123"), fallback=fallback)
    x = torch.randn(1, 40, HEADS * DIM, device=dev).to(torch.bfloat16)
    freqs = torch.ones(40, device=dev, dtype=torch.bfloat16)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        att(x, torch.tensor([40], device=dev), None, freqs)
        q = att.q(x).view(1, 40, HEADS, DIM)
        k = att.k(x).view(1, 40, HEADS, DIM)
    s = att.faquant_qk_smooth_scale
    assert got["q"].dtype == torch.float32
    assert torch.equal(got["q"], q * s) and torch.equal(got["k"], k / s)
