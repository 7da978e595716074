"""The Q operand prologue inside the attention kernel (faq_attn_opts.q_prep).

The kernel loads the raw bf16 query rows and applies faq_operand_prep's steps for Q (the
per-block fp32 Hadamard, one bf16 cast, the HiF4 QDQ; qwen3.py:97-130) to each wave's
fragment as a work item starts.  It must give the attention of the separately prepared
operand bit for bit: outputs and row denominators, across the head groupings (8, 4, 2, 1
query heads per workgroup), Hadamard blocks 0 / 64 / 128, levels 123 / 12 / 13 and none,
causal and not, key-range masks, the split-key path, and query rows holding NaN, infinities
and values near the E6M2 clamp.
"""

from __future__ import annotations

import zlib

import pytest

from faquant_amd import _ops

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _inputs(seed, B, Hq, Hkv, L, dev, q_scale=2.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = (torch.randn(B, Hq, L, 128, generator=g) * q_scale).to(torch.bfloat16).to(dev)
    k = torch.randn(B, Hkv, L, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, Hkv, L, 128, generator=g).to(torch.bfloat16).to(dev)
    kh, _ = _ops.operand_prep(k, levels="123", hadamard=64, round_dtype=torch.bfloat16)
    vt = _ops.operand_prep_vt(v, levels="123")
    return q, kh, vt


def _attend(q, kh, vt, L, causal, *, q_prep=None, ranges=None, split=1):
    B, Hq = q.shape[0], q.shape[1]
    out = torch.empty((B, L, Hq, 128), device=q.device, dtype=torch.float32)
    den = torch.empty((B, Hq, L), device=q.device, dtype=torch.float32)
    _ops.attention_fwd(q, kh, vt, L, causal=causal, scale=128**-0.5, quant_p=True, p_levels="123", norm_same=True,
                       out=out.transpose(1, 2), row_den=den, ranges=ranges, split=split, q_prep=q_prep)
    return out, den


def _bits_equal(a, b):
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


CASES = [
    # B, Hq, Hkv, L, causal, hadamard, levels
    (1, 32, 8, 1000, True, 64, "123"),
    (2, 16, 16, 700, False, 128, "12"),
    (1, 16, 2, 513, True, 0, "13"),
    (1, 8, 4, 300, True, 64, None),
    (2, 12, 6, 777, True, 128, "123"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_fused_q_prologue_equals_separate_prologue(dev, case):
    B, Hq, Hkv, L, causal, had, lv = case
    print(f"[q_prep] {case}", flush=True)
    q, kh, vt = _inputs(zlib.crc32(repr(case).encode()) & 0xFFFF, B, Hq, Hkv, L, dev)
    qh, _ = _ops.operand_prep(q, levels=lv, hadamard=had, round_dtype=torch.bfloat16)
    want = _attend(qh, kh, vt, L, causal)
    got = _attend(q, kh, vt, L, causal, q_prep=(had, lv))
    assert _bits_equal(got[0], want[0]) and _bits_equal(got[1], want[1])


def test_fused_q_prologue_with_masks_split_and_special_values(dev):
    B, Hq, Hkv, L = 2, 16, 4, 650
    q, kh, vt = _inputs(5, B, Hq, Hkv, L, dev, q_scale=3.0)
    # special rows: a NaN, infinities, values at the top of the E6M2 range and tiny ones
    q[0, 1, 7, 3] = float("nan")
    q[1, 2, 100, 70] = float("inf")
    q[1, 2, 101, 0:64] = -float("inf")
    q[0, 5, 300, :] = 60000.0
    q[0, 6, 301, :] = 1e-30
    mask = torch.ones((B, L), dtype=torch.bool, device=dev)
    mask[1, :40] = False
    ranges = _ops.attention_key_ranges(mask, B, L, L, causal=True, window=300, device=dev)
    for had, lv in ((64, "123"), (128, "13")):
        qh, _ = _ops.operand_prep(q, levels=lv, hadamard=had, round_dtype=torch.bfloat16)
        for split, rng in ((1, None), (1, ranges), (3, None)):
            print(f"[q_prep] masks/split had={had} lv={lv} split={split} ranges={rng is not None}", flush=True)
            want = _attend(qh, kh, vt, L, True, ranges=rng, split=split)
            got = _attend(q, kh, vt, L, True, q_prep=(had, lv), ranges=rng, split=split)
            assert _bits_equal(got[0], want[0]) and _bits_equal(got[1], want[1])
