"""Bit-exactness of the attention kernel's in-register P quantizer.

The reference quantizes each 128-key tile of P along keys in 64-groups with
``fake_quantize_hif4`` (simulated_flash_attention.py:801-806, hif4.py:143-271).  The kernel
computes its own P (exp2 of the fma-scaled score, a few ulp from torch.exp), so P-hat is
checked against the oracle quantizer applied to the kernel's own P:
- ``faq_pquant_groups`` runs the kernel's device code on chosen values: groups built on and
  around the rounding thresholds of floor(fp32(fp32(p qm) 4) + 0.5) (ties, products that
  round onto a half-integer, u = 0.5 - 2^-25), and softmax-like groups;
- the probe form of ``faq_attention_fwd`` writes P and P-hat of every processed key, and
  every tile's P-hat must equal the oracle's QDQ of that tile's P, bit for bit, over causal,
  non-causal, GQA and ragged shapes and all three level sets.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hif4 as OQ
from tests.pquant_cases import single_rounding_codes, softmax_groups, tie_groups

torch = pytest.importorskip("torch")

LEVELS = ("123", "12", "13")


@pytest.mark.parametrize("levels", LEVELS)
def test_tie_groups_separate_the_two_rounding_rules(levels):
    # the constructed groups contain codes where the reference's two roundings (ties up)
    # and one rounding with ties to even disagree: the GPU test below can tell them apart
    g = tie_groups(levels, seed=7)
    ref = OQ.fake_quantize_hif4(g, levels, "float32")
    alt = single_rounding_codes(g, levels)
    assert int((ref.view(np.uint32) != alt.view(np.uint32)).sum()) > 100


@pytest.mark.gpu
@pytest.mark.parametrize("levels", LEVELS)
def test_pquant_groups_bit_exact(dev, levels):
    from faquant_amd import _ops

    for name, groups in (("ties", tie_groups(levels, seed=11)), ("softmax", softmax_groups(seed=12)),
                         ("softmax_wide", softmax_groups(seed=13, spread=12.0))):
        got = _ops.pquant_groups(torch.from_numpy(groups).to(dev), levels).cpu().numpy()
        ref = OQ.fake_quantize_hif4(groups, levels, "float32")
        diff = int((got.view(np.uint32) != ref.view(np.uint32)).sum())
        print(f"pquant {levels} {name}: {diff} of {groups.size} codes differ", flush=True)
        assert diff == 0, name


@pytest.mark.gpu
def test_pquant_groups_special_blocks(dev):
    from faquant_amd import _ops

    blocks = np.zeros((4, 64), np.float32)
    blocks[1] = 1.0                       # all equal
    blocks[2, ::7] = 2.0**-60             # tiny maxima: the scale clamps at 2^-48
    blocks[3] = np.linspace(0, 1, 64, dtype=np.float32)
    for levels in LEVELS:
        got = _ops.pquant_groups(torch.from_numpy(blocks).to(dev), levels).cpu().numpy()
        ref = OQ.fake_quantize_hif4(blocks, levels, "float32")
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), levels


def _p_dump(dev, seed, B, Hq, Hkv, Lq, Lk, causal, levels):
    from faquant_amd import _ops

    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal((B, Hq, Lq, 128), dtype=np.float32) * 1.5).to(dev).to(torch.bfloat16)
    k = torch.from_numpy(rng.standard_normal((B, Hkv, Lk, 128), dtype=np.float32) * 1.5).to(dev).to(torch.bfloat16)
    v = torch.from_numpy(rng.standard_normal((B, Hkv, Lk, 128), dtype=np.float32)).to(dev).to(torch.bfloat16)
    qh, _ = _ops.operand_prep(q, levels=levels)
    kh, _ = _ops.operand_prep(k, levels=levels)
    vt = _ops.operand_prep_vt(v, levels=levels)
    width = -(-Lk // 128) * 128
    dump = torch.full((B, Hq, Lq, 2, width), float("nan"), device=dev, dtype=torch.float32)
    out = torch.empty((B, Hq, Lq, 128), device=dev, dtype=torch.float32)
    scale = 128**-0.5
    _ops.attention_fwd(qh, kh, vt, Lk, causal=causal, scale=scale, quant_p=True, p_levels=levels, norm_same=True,
                       out=out, p_dump=dump)
    return qh.float().cpu().numpy(), kh.float().cpu().numpy(), dump.cpu().numpy(), scale


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B,Hq,Hkv,Lq,Lk,causal,levels",
    [
        (1, 4, 1, 300, 300, True, "123"),
        (1, 4, 1, 300, 300, False, "12"),
        (2, 2, 2, 130, 333, True, "13"),
        (1, 8, 2, 257, 640, False, "123"),
    ],
)
def test_attention_p_hat_bit_exact_per_tile(dev, B, Hq, Hkv, Lq, Lk, causal, levels):
    qh, kh, dump, scale = _p_dump(dev, 5 + Lq, B, Hq, Hkv, Lq, Lk, causal, levels)
    G = Hq // Hkv
    nt = -(-Lk // 128)
    off = Lk - Lq
    P = dump[:, :, :, 0].reshape(B, Hq, Lq, nt, 128)
    Ph = dump[:, :, :, 1].reshape(B, Hq, Lq, nt, 128)
    done = ~np.isnan(P).any(axis=-1)  # tiles the kernel processed for the row
    pos = np.arange(Lq)
    last = np.minimum(nt - 1, (pos + off) // 128) if causal else np.full(Lq, nt - 1)
    need = np.arange(nt)[None, :] <= last[:, None]  # [Lq, nt]: tiles the row must see
    assert done[..., need].all(), "a tile the row sees was not processed"
    ref = OQ.fake_quantize_hif4(np.where(done[..., None], P, 0.0).astype(np.float32), levels, "float32")
    bad = (ref.view(np.uint32) != Ph.view(np.uint32)) & done[..., None]
    # the kernel's P is exp(S scale - running max) within the fp32 accumulation error of S
    kk = np.repeat(kh, G, axis=1).astype(np.float64)
    s = np.einsum("bhqd,bhkd->bhqk", qh.astype(np.float64), kk) * scale
    keys = np.arange(Lk)
    if causal:
        s = np.where(keys[None, :] > (pos + off)[:, None], -np.inf, s)
    sp = np.full((B, Hq, Lq, nt * 128), -np.inf)
    sp[..., :Lk] = s
    sp = sp.reshape(B, Hq, Lq, nt, 128)
    m = np.maximum.accumulate(sp.max(axis=-1), axis=-1)  # running maximum after each tile
    with np.errstate(invalid="ignore"):
        want = np.where(np.isfinite(sp), np.exp(sp - m[..., None]), 0.0)
    worst_p = float(np.abs(np.where(done[..., None], P - want, 0.0)).max())
    print(f"P-hat codes checked {int(done.sum()) * 128}, mismatched {int(bad.sum())}; "
          f"max |P - exp(S - m)| {worst_p:.2e}", flush=True)
    assert done.any() and int(bad.sum()) == 0
    assert worst_p < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("causal,levels", [(True, "123"), (False, "12")])
def test_p_hat_flip_rate_against_the_oracle_softmax(dev, causal, levels):
    """How many P-hat codes differ from the reference's own tile computation (fp32 S from
    a float32 matmul, s scale, running max, numpy exp, then the oracle quantizer): the
    codes only differ where the two P values straddle a rounding boundary."""
    B, Hq, Hkv, L = 1, 8, 2, 640
    qh, kh, dump, scale = _p_dump(dev, 77, B, Hq, Hkv, L, L, causal, levels)
    G = Hq // Hkv
    nt = L // 128
    s = np.matmul(qh, np.swapaxes(np.repeat(kh, G, axis=1), -1, -2)).astype(np.float32)
    s = (s * np.float32(scale)).astype(np.float32)
    if causal:
        s = np.where(np.arange(L)[None, :] > np.arange(L)[:, None], -np.inf, s).astype(np.float32)
    t = s.reshape(B, Hq, L, nt, 128)
    m = np.maximum.accumulate(t.max(axis=-1), axis=-1).astype(np.float32)
    with np.errstate(invalid="ignore"):
        p = np.where(np.isfinite(t), np.exp((t - m[..., None]).astype(np.float32)), 0.0).astype(np.float32)
    ref = OQ.fake_quantize_hif4(p, levels, "float32")
    ph = dump[:, :, :, 1].reshape(B, Hq, L, nt, 128)
    done = ~np.isnan(ph).any(axis=-1)
    flips = int(((ref != ph) & done[..., None]).sum())
    total = int(done.sum()) * 128
    rel_p = float(np.nanmax(np.abs(dump[:, :, :, 0].reshape(p.shape) - p)[done]))
    print(f"P-hat flips vs the oracle's exp: {flips} of {total} ({flips / total:.2e}); max |dP| {rel_p:.2e}", flush=True)
    assert flips / total < 1e-3
