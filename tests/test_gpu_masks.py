"""2-D padding masks, sliding windows and the logit softcap (sfa:341-427, 561-586, 725-727).

The kernel runs a mask as per-row key ranges [row_lo, row_hi] plus valid-key bits.
faq_attention_mask_bounds computes them from the mask with the reference's rank rule
(unpadded FlashAttention alignment).  Its result must reproduce the oracle's allowed
matrix bit for bit.  The oracle's mask code is pinned on the CPU against the reference's
closed forms: padding equals unpadded batches, decode with padding and a window, the
non-causal window.  The attention through the drop-in then matches the oracle within the
attention tolerance, with the same stats counters.  An all-valid mask, which the kernel
runs in key-range mode, equals the mask-free causal path bitwise.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import assert_close_attention, module, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def make_mask(kind: str, batch: int, length: int, seed: int) -> np.ndarray:
    g = OI.rng(seed)
    m = np.ones((batch, length), dtype=np.int64)
    for b in range(batch):
        n = int(g.integers(0, length // 2)) if b else 0  # batch row 0 stays unpadded
        if kind == "left":
            m[b, :n] = 0
        elif kind == "right":
            m[b, length - n:] = 0
        elif kind == "holes":
            m[b] = g.random(length) > 0.15
        elif kind == "empty_row":
            m[b] = 0 if b == batch - 1 else 1
        else:
            raise KeyError(kind)
    return m


def allowed_oracle(mask, batch, lq, lk, causal, window):
    qv = kv = None
    if mask is not None:
        qv, kv = OA._two_dimensional_mask(mask, lq, lk)
    a = OA.streaming_mask(batch=batch, q0=0, q1=lq, k0=0, k1=lk, query_length=lq, key_length=lk, is_causal=causal,
                          sliding_window=window, query_valid=qv, key_valid=kv)
    return np.broadcast_to(a, (batch, 1, lq, lk))[:, 0]


def allowed_kernel(ranges, lk):
    lo, hi = ranges.row_lo.cpu().numpy(), ranges.row_hi.cpu().numpy()
    bits = ranges.key_bits.cpu().numpy().view(np.uint32)
    k = np.arange(lk)
    valid = ((bits[:, k // 32] >> (k % 32).astype(np.uint32)) & 1).astype(bool)
    return (k[None, None, :] >= lo[:, :, None]) & (k[None, None, :] <= hi[:, :, None]) & valid[:, None, :]


BOUND_CASES = [
    # (mask kind or None, B, Lq, Lk, causal, window)
    ("left", 3, 300, 300, True, None),
    ("right", 3, 300, 300, True, None),
    ("holes", 3, 300, 300, True, None),
    ("holes", 2, 5, 777, True, None),        # multi-token decode over a padded cache
    ("left", 4, 1, 1000, True, 64),          # decode with a window
    ("holes", 2, 600, 300, True, None),      # Lq > Lk: leading queries see no key
    ("holes", 2, 300, 300, False, None),
    ("right", 2, 300, 300, False, 40),
    ("empty_row", 3, 200, 200, True, None),
    (None, 2, 700, 700, True, 100),
    (None, 1, 500, 300, False, 60),          # non-causal window with Lq > Lk, no mask
    (None, 1, 500, 300, True, None),         # causal, Lq > Lk: the first 200 queries see no key
    (None, 1, 129, 1000, True, 1),
]


@pytest.mark.parametrize("case", BOUND_CASES, ids=lambda c: "_".join(map(str, c)))
def test_key_ranges_reproduce_the_reference_allowed_matrix(dev, case):
    from faquant_amd import _ops

    kind, batch, lq, lk, causal, window = case
    mask = make_mask(kind, batch, lk, seed=lq + lk) if kind else None
    ranges = _ops.attention_key_ranges(None if mask is None else torch.from_numpy(mask).to(dev), batch, lq, lk,
                                       causal=causal, window=window, device=dev)
    print(f"[bounds] {case}", flush=True)
    got = allowed_kernel(ranges, lk)
    assert np.array_equal(got, allowed_oracle(mask, batch, lq, lk, causal, window))
    words = ranges.key_bits.shape[-1]
    assert words == 4 * -(-lk // 128)
    tail = ranges.key_bits.cpu().numpy().view(np.uint32)
    k = np.arange(lk, words * 32)
    assert not ((tail[:, k // 32] >> (k % 32).astype(np.uint32)) & 1).any()  # zero past Lk


def _qkv(seed, batch, hq, hkv, lq, lk):
    g = OI.rng(seed)
    q = OQ.bf16_round(g.standard_normal((batch, hq, lq, 128), dtype=np.float32) * 2)
    k = OQ.bf16_round(g.standard_normal((batch, hkv, lk, 128), dtype=np.float32))
    v = OQ.bf16_round(g.standard_normal((batch, hkv, lk, 128), dtype=np.float32))
    return q, k, v


def _run(dev, q, k, v, mask, *, mode="quantized_same", causal=True, window=None, softcap=None):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    mod = module(mode=mode, causal=causal)
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    out, _ = simulated_flash_attention_forward(mod, qt, kt, vt, None if mask is None else torch.from_numpy(mask).to(dev),
                                               sliding_window=window, softcap=softcap)
    cfg = OA.SimConfig(pv_normalizer_mode=mode, is_causal=causal)
    stats = OA.new_stats()
    ref = OA.simulated_flash_attention(q, k, v, cfg, attention_mask=mask, sliding_window=window, softcap=softcap,
                                       dtype="bfloat16", stats=stats)
    return out.float().cpu().numpy(), ref, mod.faquant_simulated_attention_stats, stats


@pytest.mark.parametrize("mode", ["quantized_same", "unquantized"])
@pytest.mark.parametrize("kind,lq,lk", [("left", 300, 300), ("right", 300, 300), ("holes", 260, 260),
                                        ("left", 1, 400), ("left", 3, 400), ("empty_row", 130, 130)])
def test_padded_batches_through_drop_in(dev, kind, lq, lk, mode):
    q, k, v = _qkv(lq + lk, 3, 8, 2, lq, lk)
    mask = make_mask(kind, 3, lk, seed=lk)
    got, ref, stats, ref_stats = _run(dev, q, k, v, mask, mode=mode)
    assert_close_attention(got, ref, f"mask {kind} {lq}x{lk} {mode}")
    assert stats == ref_stats
    if kind == "empty_row":
        assert np.count_nonzero(got[-1]) == 0  # a batch row without any valid key gives zeros


@pytest.mark.parametrize("lq,window", [(1, 64), (5, 200)])
def test_padded_decode_with_window_through_drop_in(dev, lq, window):
    """Decode steps over a left-padded cache with a sliding window
    (test_simulated_flash_attention.py:235-265, 329-359)."""
    q, k, v = _qkv(900 + lq, 3, 8, 2, lq, 777)
    mask = make_mask("left", 3, 777, seed=lq)
    got, ref, stats, ref_stats = _run(dev, q, k, v, mask, window=window)
    assert_close_attention(got, ref, f"padded decode lq={lq} window={window}")
    assert stats == ref_stats


def test_left_padding_position_ids_are_not_mistaken_for_packing(dev):
    """With a 2-D mask, position ids that restart inside the padding are left-padding ids,
    not packing (test_simulated_flash_attention.py:380-396): the call equals the call
    without them.  Without a mask the same ids are rejected as packed (sfa:485-510)."""
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(11, 1, 4, 2, 300, 300))
    mask = torch.ones((1, 300), dtype=torch.bool)
    mask[0, :100] = False
    pos = torch.cat([torch.ones(100, dtype=torch.long), torch.arange(200)])[None].to(dev)
    a, _ = simulated_flash_attention_forward(module(), q, k, v, mask.to(dev), position_ids=pos)
    b, _ = simulated_flash_attention_forward(module(), q, k, v, mask.to(dev))
    assert torch.equal(a, b)
    with pytest.raises(NotImplementedError):
        simulated_flash_attention_forward(module(), q, k, v, None, position_ids=pos)


@pytest.mark.parametrize("causal,window,lq,lk", [(True, 100, 700, 700), (False, 150, 500, 500),
                                                 (True, 300, 2, 900), (False, 1, 200, 200)])
def test_sliding_window_through_drop_in(dev, causal, window, lq, lk):
    q, k, v = _qkv(window + lq, 1, 4, 1, lq, lk)
    got, ref, stats, ref_stats = _run(dev, q, k, v, None, causal=causal, window=window)
    assert_close_attention(got, ref, f"window {window} causal={causal} {lq}x{lk}")
    assert stats == ref_stats


def test_padding_with_window(dev):
    q, k, v = _qkv(77, 2, 8, 2, 400, 400)
    mask = make_mask("left", 2, 400, seed=5)
    got, ref, stats, ref_stats = _run(dev, q, k, v, mask, window=90)
    assert_close_attention(got, ref, "left padding + window 90")
    assert stats == ref_stats


@pytest.mark.parametrize("softcap,causal", [(0.5, True), (2.0, True), (3.0, False)])
def test_softcap_through_drop_in(dev, softcap, causal):
    q, k, v = _qkv(int(softcap * 10), 1, 4, 1, 300, 300)
    got, ref, _, _ = _run(dev, q, k, v, None, causal=causal, softcap=softcap)
    assert_close_attention(got, ref, f"softcap {softcap} causal={causal}")
    plain, _, _, _ = _run(dev, q, k, v, None, causal=causal)
    assert not np.allclose(got, plain)  # the cap changes the result at these score magnitudes


def test_all_valid_mask_equals_mask_free_path_bitwise(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(3, 2, 8, 2, 300, 300))
    ones = torch.ones((2, 300), device=dev, dtype=torch.int64)
    masked_mod = module()
    a, _ = simulated_flash_attention_forward(masked_mod, q, k, v, ones)  # B = 2: the rank form runs
    b, _ = simulated_flash_attention_forward(module(), q, k, v, None)
    assert torch.equal(a, b)
    # the reference does not skip future tiles once a mask is in force (sfa:676-681)
    assert masked_mod.faquant_simulated_attention_stats["qk_tiles"] == 2 * 3
    # a single prompt with an all-valid mask is the mask-free case, skipping included
    one = module()
    c, _ = simulated_flash_attention_forward(one, q[:1], k[:1], v[:1], ones[:1])
    assert torch.equal(c, b[:1])
    assert one.faquant_simulated_attention_stats["qk_tiles"] == 5  # 2 + 3: key tile 2 skipped for rows < 256


def test_split_key_path_with_ranges_equals_one_pass(dev):
    from faquant_amd import _ops

    B, Hq, Hkv, Lq, Lk = 2, 8, 2, 3, 1000
    q, k, v = _qkv(9, B, Hq, Hkv, Lq, Lk)
    mask = make_mask("holes", B, Lk, seed=9)
    qh, _ = _ops.operand_prep(to_dev(q, dev, torch.bfloat16), levels="123")
    kh, _ = _ops.operand_prep(to_dev(k, dev, torch.bfloat16), levels="123")
    vt = _ops.operand_prep_vt(to_dev(v, dev, torch.bfloat16), levels="123")
    for window in (None, 200):
        ranges = _ops.attention_key_ranges(torch.from_numpy(mask).to(dev), B, Lq, Lk, causal=True, window=window)
        outs = []
        for split in (1, 5):
            out = torch.empty((B, Lq, Hq, 128), device=dev, dtype=torch.float32)
            _ops.attention_fwd(qh, kh, vt, Lk, causal=True, scale=128**-0.5, quant_p=True, p_levels="123",
                               norm_same=True, out=out.transpose(1, 2), split=split, ranges=ranges)
            outs.append(out.cpu().numpy())
        print(f"[split ranges] window={window}", flush=True)
        np.testing.assert_allclose(outs[1], outs[0], rtol=1e-5, atol=1e-6 * np.abs(outs[0]).max())
        cfg = OA.SimConfig(pv_normalizer_mode="quantized_same")
        ref = OA.simulated_flash_attention(q, k, v, cfg, attention_mask=mask, sliding_window=window)
        assert_close_attention(outs[1], ref, f"split ranges window={window}")


def _dense_case(kind, batch, hq, lq, lk, seed):
    """(torch mask, numpy mask for the oracle) of the 3-D/4-D forms of sfa:430-454."""
    g = OI.rng(seed)
    causal = np.tril(np.ones((lq, lk), bool), k=lk - lq)
    if kind == "bool_causal":
        m = np.broadcast_to(causal, (batch, 1, lq, lk)).copy()
        return torch.from_numpy(m), m
    if kind == "additive_heads":
        m = (g.uniform(-3, 0, size=(batch, hq, lq, lk))).astype(np.float32)
        m[g.random(m.shape) < 0.1] = -np.inf
        m[g.random(m.shape) < 0.05] = np.finfo(np.float32).min
        m[:, :, 3] = -np.inf  # a fully masked row
        return torch.from_numpy(m), m
    if kind == "f32_min_row":  # test_simulated_flash_attention.py:208-220: finfo.min rows
        m = np.full((batch, 1, lq, lk), np.finfo(np.float32).min, dtype=np.float32)
        m[..., 1:, : lk // 3] = 0.0  # row 0 stays fully masked by finfo.min (not -inf)
        return torch.from_numpy(m), m
    if kind == "fp16_all_min":  # test_simulated_flash_attention.py:222-233: every row masked
        m = np.full((batch, 1, lq, lk), np.finfo(np.float16).min, dtype=np.float16)
        return torch.from_numpy(m), m
    if kind == "fp16_min":
        m = np.where(causal, 0.0, np.finfo(np.float16).min).astype(np.float16)[None, None]
        m = np.broadcast_to(m, (batch, 1, lq, lk)).copy()
        return torch.from_numpy(m), m
    if kind == "bf16_longer_rows":  # more mask rows than queries: the last lq rows are used
        full = np.tril(np.ones((lq + 7, lk), bool), k=lk - lq - 7)
        m = np.where(full, 0.0, -1e30).astype(np.float32)[None, None]
        m = np.broadcast_to(m, (batch, 1, lq + 7, lk)).copy()
        t = torch.from_numpy(m).to(torch.bfloat16)
        return t, t.float().numpy()
    if kind == "one_row":
        m = g.random((batch, 1, 1, lk)) > 0.2
        return torch.from_numpy(m), m
    if kind == "three_d":
        m = (g.random((batch, lq, lk)) > 0.1) & causal
        m[:, :, 0] = True
        return torch.from_numpy(m), m
    raise KeyError(kind)


@pytest.mark.parametrize("kind,batch,lq,lk", [("bool_causal", 2, 300, 300), ("additive_heads", 1, 200, 260),
                                              ("fp16_min", 1, 256, 300), ("bf16_longer_rows", 1, 130, 300),
                                              ("one_row", 2, 1, 500), ("three_d", 2, 150, 150),
                                              ("f32_min_row", 1, 140, 300), ("fp16_all_min", 1, 70, 200)])
@pytest.mark.parametrize("softcap", [None, 2.5])
def test_dense_masks_through_drop_in(dev, kind, batch, lq, lk, softcap):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    hq = 4
    q, k, v = _qkv(lq + lk, batch, hq, 2, lq, lk)
    tmask, nmask = _dense_case(kind, batch, hq, lq, lk, seed=lk)
    mod = module()
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    out, _ = simulated_flash_attention_forward(mod, qt, kt, vt, tmask.to(dev), softcap=softcap)
    stats = OA.new_stats()
    ref = OA.simulated_flash_attention(q, k, v, OA.SimConfig(pv_normalizer_mode="quantized_same"),
                                       attention_mask=nmask, softcap=softcap, dtype="bfloat16", stats=stats)
    got = out.float().cpu().numpy()
    assert_close_attention(got, ref, f"dense {kind} softcap={softcap}")
    assert mod.faquant_simulated_attention_stats == stats
    assert np.isfinite(got).all()
    if kind == "additive_heads":
        assert np.count_nonzero(got[:, 3]) == 0  # fully masked rows give zeros
    if kind == "f32_min_row":
        assert np.count_nonzero(got[:, 0]) == 0 and np.count_nonzero(got[:, 1:]) > 0
    if kind == "fp16_all_min":
        assert np.count_nonzero(got) == 0


def test_attention_core_with_padding_mask_equals_drop_in(dev):
    """qwen3.attention_core runs a 2-D mask in its fused launch; the result equals the
    reference composition: excursion, then the drop-in with the same mask."""
    from faquant_amd.qwen3 import attention_core, post_rope_qk_transform
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(61, 3, 8, 2, 330, 330))
    mask = torch.from_numpy(make_mask("left", 3, 330, seed=61)).to(dev)

    def mk():
        m = module()
        m.faquant_qk_rotation = True
        m.faquant_qk_rotation_block_size = 64
        return m

    fused_mod, ref_mod = mk(), mk()
    got = attention_core(fused_mod, q, k, v, attention_mask=mask)
    qr, kr = post_rope_qk_transform(q, k, rotation=True, rotation_block_size=64)
    ref, _ = simulated_flash_attention_forward(ref_mod, qr, kr, v, mask)
    assert torch.equal(got, ref)
    assert fused_mod.faquant_simulated_attention_stats == ref_mod.faquant_simulated_attention_stats
