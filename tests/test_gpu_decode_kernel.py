"""The decode kernel (faq_attention_decode) and packed HiF4 K/V caches.

- ``pack_operand`` rows, decoded by ``unpack_rows`` below (the packed format restated in
  integer arithmetic: (nibble - 8) (4 + m) 2^(e + lv2 + lv3 - 4)), equal operand_prep's
  bf16 HiF4 values bitwise: levels 123/12/13, the Qwen post-RoPE prologue (r64 Hadamard,
  Smooth-QK, key offset), zero rows, tiny negatives (-0), a NaN group;
- decode over bf16 K/V gives faq_attention_fwd_split's output and row denominators with
  the same number of key ranges, bitwise (GQA 1..16 heads per KV head, 1..5 positions,
  ragged and single-key ranges, more ranges than tiles, P quantization off, both
  normalizer modes);
- decode over packed K/V gives the bf16 decode's bits;
- the drop-in with ``faquant_kv_cache_packed`` grows a packed cache over decode steps,
  with the same output as bf16 caches, bitwise, and matches the oracle.
The split path these are compared with is itself checked against the oracle
(test_gpu_decode.py).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import TIGHT, _oracle, assert_close_attention, module, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def unpack_rows(codes: np.ndarray, meta: np.ndarray) -> np.ndarray:
    """Values of packed HiF4 rows: codes uint32 [..., 16], meta uint32 [..., 2] -> fp32
    [..., 128].  Dims 8u .. 8u + 7 sit in word (u & 1) 8 + u / 2, dim 8u + i in nibble i."""
    codes = codes.astype(np.int64) & 0xFFFFFFFF
    meta = meta.astype(np.int64) & 0xFFFFFFFF
    out = np.empty(codes.shape[:-1] + (128,), dtype=np.float64)
    for u in range(16):
        word = codes[..., (u & 1) * 8 + u // 2]
        m = meta[..., u // 8]
        sb = m & 0xFF
        e, mant = (sb >> 2) - 48, sb & 3
        g8 = u % 8
        lv2 = (m >> (8 + g8)) & 1
        for i in range(8):
            nib = (word >> (4 * i)) & 0xF
            lv3 = (m >> (16 + 2 * g8 + i // 4)) & 1
            val = (nib - 8) * (4 + mant) * np.exp2((e + lv2 + lv3 - 4).astype(np.float64))
            out[..., 8 * u + i] = np.where(sb == 0xFF, np.nan, val)
    return out.astype(np.float32)


def _packed_values(cache) -> np.ndarray:
    n = cache.length
    return unpack_rows(cache.codes[:, :, :n].cpu().numpy(), cache.meta[:, :, :n].cpu().numpy())


@pytest.mark.parametrize("levels", ["123", "12", "13"])
@pytest.mark.parametrize("prologue", ["plain", "qwen_r64", "hadamard128"])
def test_packed_rows_decode_to_operand_prep(dev, levels, prologue):
    from faquant_amd import _ops

    g = OI.rng(int(levels) + len(prologue))
    B, H, L = 2, 3, 77
    x = g.standard_normal((B, H, L, 128)).astype(np.float32) * 3
    x[0, 1, 5] = 0.0                          # an all-zero row
    x[1, 0, 9, :64] = -1e-30                  # a group of tiny negatives: codes 0 (-0 in bf16)
    x[1, 2, 11, 64:] *= 1e4                   # a large group
    x[0, 0, 13, 70] = np.nan                  # a NaN group (its 64 values become NaN)
    xt = to_dev(x, dev, torch.bfloat16)
    prep = {}
    if prologue == "qwen_r64":
        prep = dict(hadamard=64, smooth=to_dev(g.uniform(0.5, 2.0, size=(128,)), dev),
                    key_offset=to_dev(g.standard_normal((H, 1, 128)) * 0.3, dev), smooth_divide=True,
                    round_dtype=torch.bfloat16)
    elif prologue == "hadamard128":
        prep = dict(hadamard=128, round_dtype=torch.bfloat16)
    want, _ = _ops.operand_prep(xt, levels=levels, **prep)
    cache = _ops.PackedHiF4KV(B, H, 200, dev, levels)
    cache.codes.fill_(0x5A5A5A5A)
    _ops.pack_operand(xt[:, :, :40], levels=levels, out=cache, **prep)
    _ops.pack_operand(xt[:, :, 40:], levels=levels, out=cache, start=40, **prep)  # rows are token-local
    assert cache.length == L
    got = _packed_values(cache)
    ref = want.float().cpu().numpy()
    print(f"[pack] levels {levels} {prologue}", flush=True)
    assert np.array_equal(got, ref, equal_nan=True)
    # the NaN reaches its Hadamard block, then its 64-value HiF4 group
    assert np.isnan(got[0, 0, 13]).sum() == (128 if prologue == "hadamard128" else 64)
    assert (cache.codes[:, :, L:] == 0x5A5A5A5A).all()  # rows past the end untouched
    assert cache.nbytes() == B * H * L * 72  # 4.5 bits per value


DECODE_CASES = [
    # (B, Hq, Hkv, Lq, Lk, causal, mode, quant_p, levels, nsplit)
    (1, 32, 8, 1, 5000, True, "quantized_same", True, "123", 40),    # Qwen3-8B decode step
    (1, 64, 8, 1, 16384, True, "quantized_same", True, "12", 64),    # Qwen3-32B decode step
    (2, 8, 2, 3, 1000, True, "quantized_same", True, "123", 6),      # G 4 x 3 positions
    (1, 4, 1, 5, 900, True, "unquantized", True, "123", 4),          # G 4 x 5 positions
    (1, 16, 1, 2, 3000, True, "quantized_same", True, "123", 7),     # G 16 x 2: 32 columns
    (1, 40, 40, 1, 2000, False, "quantized_same", True, "123", 8),   # MHA, non-causal
    (3, 12, 4, 1, 129, True, "quantized_same", True, "13", 2),       # G 3: 30 of 32 columns live
    (1, 4, 4, 1, 777, False, "quantized_same", True, "12", 3),       # ragged last tile
    (1, 2, 1, 1, 300, True, "quantized_same", True, "13", 16),       # more ranges than tiles
    (1, 8, 2, 1, 1, True, "quantized_same", True, "123", 1),         # one key
    (1, 4, 1, 2, 640, True, "quantized_same", False, "123", 5),      # P not quantized
    (1, 8, 2, 2, 2000, True, "quantized_same", True, "123", 9),      # G 4 x 2 positions: 8 columns
    (2, 4, 2, 3, 1500, True, "quantized_same", True, "12", 5),       # G 2 x 3 positions: 6 of 8 live
]


def _decode_inputs(case, dev):
    from faquant_amd import _ops

    B, Hq, Hkv, Lq, Lk, causal, mode, qp, lv, nsplit = case
    g = OI.rng(7 * Lk + Lq + Hq)
    q = OQ.bf16_round(g.standard_normal((B, Hq, Lq, 128), dtype=np.float32) * 2)
    k = OQ.bf16_round(g.standard_normal((B, Hkv, Lk, 128), dtype=np.float32))
    v = OQ.bf16_round(g.standard_normal((B, Hkv, Lk, 128), dtype=np.float32))
    qh, _ = _ops.operand_prep(to_dev(q, dev, torch.bfloat16), levels=lv)
    kh, _ = _ops.operand_prep(to_dev(k, dev, torch.bfloat16), levels=lv)
    vh, _ = _ops.operand_prep(to_dev(v, dev, torch.bfloat16), levels=lv if qp else None)  # natural rows
    vt = _ops.operand_prep_vt(to_dev(v, dev, torch.bfloat16), levels=lv if qp else None)  # the split path's V^T
    kw = dict(causal=causal, scale=128**-0.5, quant_p=qp, p_levels=lv, norm_same=mode == "quantized_same")
    return (q, k, v), (qh, kh, vh, vt), kw


def _run(fn, case, dev, **extra):
    B, Hq, Hkv, Lq = case[:4]
    out = torch.empty((B, Lq, Hq, 128), device=dev, dtype=torch.float32)
    den = torch.empty((B, Hq, Lq), device=dev, dtype=torch.float32)
    fn(out=out.transpose(1, 2), row_den=den, **extra)
    return out, den


@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"_{c[6]}_{c[8]}_{c[9]}")
def test_decode_equals_split_path_bitwise(dev, case):
    from faquant_amd import _ops

    B, Hq, Hkv, Lq, Lk, causal, mode, qp, lv, nsplit = case
    (q, k, v), (qh, kh, vh, vt), kw = _decode_inputs(case, dev)
    print(f"[decode] {case}", flush=True)
    split_o, split_l = _run(lambda **a: _ops.attention_fwd(qh, kh, vt, Lk, split=nsplit, **kw, **a), case, dev)
    dec_o, dec_l = _run(lambda **a: _ops.attention_decode(qh, Lk, k=kh, v=vh, split=nsplit, **kw, **a), case, dev)
    assert torch.equal(dec_o, split_o)
    assert torch.equal(dec_l, split_l)
    if qp:
        kc = _ops.pack_operand(to_dev(k, dev, torch.bfloat16), levels=lv,
                               out=_ops.PackedHiF4KV(B, Hkv, Lk + 5, dev, lv))
        vc = _ops.pack_operand(to_dev(v, dev, torch.bfloat16), levels=lv,
                               out=_ops.PackedHiF4KV(B, Hkv, Lk + 5, dev, lv))
        pk_o, pk_l = _run(lambda **a: _ops.attention_decode(qh, Lk, packed=(kc, vc), split=nsplit, **kw, **a),
                          case, dev)
        assert torch.equal(pk_o, dec_o)
        assert torch.equal(pk_l, dec_l)
    if case[4] == 5000 or Lq > 1:
        ref = _oracle(q, k, v, causal=causal, levels=lv, mode=mode, qk=True, pv=qp)
        assert_close_attention(dec_o.cpu().numpy(), ref, f"decode {case}", **TIGHT)


@pytest.mark.parametrize("case", [DECODE_CASES[0], DECODE_CASES[2], DECODE_CASES[7], DECODE_CASES[8], DECODE_CASES[9]],
                         ids=lambda c: "x".join(map(str, c[:5])) + f"_{c[9]}")
def test_packed_scores_without_lds_equal_staged_scores(dev, case, monkeypatch):
    """Packed K rows: the scores pass that unpacks each lane's A operand from HBM (the
    default) gives the staged pass's output and row denominators bitwise (ragged last
    tile, more ranges than tiles, one key, several positions)."""
    from faquant_amd import _ops

    B, Hq, Hkv, Lq, Lk, causal, mode, qp, lv, nsplit = case
    (q, k, v), (qh, kh, vh, vt), kw = _decode_inputs(case, dev)
    kc = _ops.pack_operand(to_dev(k, dev, torch.bfloat16), levels=lv, out=_ops.PackedHiF4KV(B, Hkv, Lk, dev, lv))
    vc = _ops.pack_operand(to_dev(v, dev, torch.bfloat16), levels=lv, out=_ops.PackedHiF4KV(B, Hkv, Lk, dev, lv))
    print(f"[scores] {case}", flush=True)
    monkeypatch.setenv("FAQ_DECODE_FUSED", "0")
    runs = {}
    for form in ("direct", "lds"):
        monkeypatch.delenv("FAQ_DEC_SCORES", raising=False)
        if form == "lds":
            monkeypatch.setenv("FAQ_DEC_SCORES", "lds")
        runs[form] = _run(lambda **a: _ops.attention_decode(qh, Lk, packed=(kc, vc), split=nsplit, **kw, **a),
                          case, dev)
    assert torch.equal(runs["direct"][0], runs["lds"][0])
    assert torch.equal(runs["direct"][1], runs["lds"][1])


FUSED_CASES = [
    # decode steps the one-pass kernel takes (P quantized, quantized-same, G x positions <= 8,
    # one key tile per split, at most 64 tiles)
    (1, 32, 8, 1, 5000, True, "quantized_same", True, "123", 40),   # G 4, ragged last tile
    (1, 64, 8, 1, 8192, True, "quantized_same", True, "12", 64),    # G 8
    (1, 8, 2, 2, 2000, True, "quantized_same", True, "13", 16),     # 8 columns over two positions
    (3, 12, 4, 1, 129, True, "quantized_same", True, "123", 2),     # G 3, batch 3
    (1, 2, 1, 1, 300, True, "quantized_same", True, "13", 16),      # empty splits past the last tile
    (1, 40, 40, 1, 2000, False, "quantized_same", True, "123", 16), # MHA, non-causal
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"_{c[8]}_{c[9]}")
def test_one_pass_decode_equals_two_passes_bitwise(dev, case, monkeypatch):
    """The one-pass decode (look-back over the earlier splits' published maxima) gives the
    two passes' output and row denominators bitwise, for bf16 and packed K/V, and so does
    its fallback that computes every earlier split's maxima from K (wait bound < 0)."""
    from faquant_amd import _ops

    B, Hq, Hkv, Lq, Lk, causal, mode, qp, lv, nsplit = case
    (q, k, v), (qh, kh, vh, vt), kw = _decode_inputs(case, dev)
    kc = _ops.pack_operand(to_dev(k, dev, torch.bfloat16), levels=lv, out=_ops.PackedHiF4KV(B, Hkv, Lk, dev, lv))
    vc = _ops.pack_operand(to_dev(v, dev, torch.bfloat16), levels=lv, out=_ops.PackedHiF4KV(B, Hkv, Lk, dev, lv))
    print(f"[fused] {case}", flush=True)
    for name, extra in (("bf16", dict(k=kh, v=vh)), ("packed", dict(packed=(kc, vc)))):
        runs = {}
        for path, env in (("two_pass", {"FAQ_DECODE_FUSED": "0"}), ("one_pass", {"FAQ_DECODE_FUSED": "force"}),
                          ("fallback", {"FAQ_DECODE_FUSED": "force", "FAQ_DECODE_SPIN": "-1"})):
            monkeypatch.delenv("FAQ_DECODE_FUSED", raising=False)
            monkeypatch.delenv("FAQ_DECODE_SPIN", raising=False)
            for key, val in env.items():
                monkeypatch.setenv(key, val)
            runs[path] = _run(lambda **a: _ops.attention_decode(qh, Lk, split=nsplit, **extra, **kw, **a), case, dev)
        for path in ("one_pass", "fallback"):
            assert torch.equal(runs[path][0], runs["two_pass"][0]), (name, path)
            assert torch.equal(runs[path][1], runs["two_pass"][1]), (name, path)
    # and a call right after another one over the same maxima slots (a new epoch) ignores the
    # maxima the first left: keys scaled by 2 (HiF4 values stay exact) change every split
    # maximum, and the second call must still equal its own two-pass result
    monkeypatch.delenv("FAQ_DECODE_SPIN", raising=False)
    kh2 = kh * 2
    monkeypatch.setenv("FAQ_DECODE_FUSED", "0")
    want = _run(lambda **a: _ops.attention_decode(qh, Lk, k=kh2, v=vh, split=nsplit, **kw, **a), case, dev)
    monkeypatch.setenv("FAQ_DECODE_FUSED", "force")
    _run(lambda **a: _ops.attention_decode(qh, Lk, k=kh, v=vh, split=nsplit, **kw, **a), case, dev)
    second = _run(lambda **a: _ops.attention_decode(qh, Lk, k=kh2, v=vh, split=nsplit, **kw, **a), case, dev)
    assert not torch.equal(second[1], runs["two_pass"][1])  # the maxima did change
    assert torch.equal(second[0], want[0]) and torch.equal(second[1], want[1])


def test_decode_captured_in_a_graph_replays_with_new_keys(dev, monkeypatch):
    """A decode step recorded into a HIP graph (torch.cuda.graph) and replayed over new K
    contents gives each replay's two-pass result bitwise: on a capturing stream the entry
    takes the two passes, which keep no state between calls (a recorded one-pass launch would
    keep its epoch and could accept an earlier replay's published maxima).  Each replay is
    followed by eager work and a synchronization before it is checked."""
    from faquant_amd import _ops

    case = (1, 32, 8, 1, 5000, True, "quantized_same", True, "123", 40)  # a one-pass case when eager
    B, Hq, Hkv, Lq, Lk, causal, mode, qp, lv, nsplit = case
    (q, k, v), (qh, kh, vh, vt), kw = _decode_inputs(case, dev)
    monkeypatch.delenv("FAQ_DECODE_FUSED", raising=False)
    monkeypatch.delenv("FAQ_DECODE_SPIN", raising=False)
    kbuf = kh.clone()
    out = torch.empty((B, Lq, Hq, 128), device=dev, dtype=torch.float32)
    den = torch.empty((B, Hq, Lq), device=dev, dtype=torch.float32)
    call = lambda: _ops.attention_decode(qh, Lk, k=kbuf, v=vh, split=nsplit, out=out.transpose(1, 2),  # noqa: E731
                                         row_den=den, **kw)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep, factor in enumerate((1.0, 2.0, 0.5, 4.0, 1.0)):
        kbuf.copy_(kh * factor)
        graph.replay()
        torch.cuda.synchronize()
        got_o, got_l = out.clone(), den.clone()
        monkeypatch.setenv("FAQ_DECODE_FUSED", "0")
        want = _run(lambda **a: _ops.attention_decode(qh, Lk, k=kbuf, v=vh, split=nsplit, **kw, **a), case, dev)
        monkeypatch.delenv("FAQ_DECODE_FUSED")
        torch.cuda.synchronize()
        print(f"[graph] replay {rep} keys x{factor}", flush=True)
        assert torch.equal(got_o, want[0]) and torch.equal(got_l, want[1]), rep


def test_one_pass_decode_is_refused_where_it_does_not_apply(dev, monkeypatch):
    """The force hook reports calls outside the one pass's cases (two tiles per split)."""
    from faquant_amd import _ops

    case = (1, 32, 8, 1, 4096, True, "quantized_same", True, "123", 16)
    (q, k, v), (qh, kh, vh, vt), kw = _decode_inputs(case, dev)
    monkeypatch.setenv("FAQ_DECODE_FUSED", "force")
    with pytest.raises(NotImplementedError, match="one-pass"):
        _run(lambda **a: _ops.attention_decode(qh, 4096, k=kh, v=vh, split=16, **kw, **a), case, dev)


def test_packed_nan_groups_match_bf16_rows(dev):
    """A NaN in K or V makes its 64-value HiF4 group NaN (E6M2 byte 0xFF in the packed
    rows): the packed decode gives NaN exactly where the bf16 rows do, and the same bits
    elsewhere."""
    from faquant_amd import _ops

    case = (1, 32, 8, 1, 1000, True, "quantized_same", True, "123", 8)
    B, Hq, Hkv, Lq, Lk = case[:5]
    (q, k, v), _, kw = _decode_inputs(case, dev)
    k = k.copy()
    v = v.copy()
    k[0, 2, 300, 17] = np.nan   # K group of KV head 2: its query heads' scores at key 300
    v[0, 5, 700, 100] = np.nan  # V group of KV head 5: its rows once key 700 has weight
    kd, vd = to_dev(k, dev, torch.bfloat16), to_dev(v, dev, torch.bfloat16)
    qh, _ = _ops.operand_prep(to_dev(q, dev, torch.bfloat16), levels="123")
    kh, _ = _ops.operand_prep(kd, levels="123")
    vh, _ = _ops.operand_prep(vd, levels="123")
    kc = _ops.pack_operand(kd, levels="123", out=_ops.PackedHiF4KV(B, Hkv, Lk, dev, "123"))
    vc = _ops.pack_operand(vd, levels="123", out=_ops.PackedHiF4KV(B, Hkv, Lk, dev, "123"))
    bf_o, _ = _run(lambda **a: _ops.attention_decode(qh, Lk, k=kh, v=vh, split=8, **kw, **a), case, dev)
    pk_o, _ = _run(lambda **a: _ops.attention_decode(qh, Lk, packed=(kc, vc), split=8, **kw, **a), case, dev)
    nan = torch.isnan(bf_o)
    assert nan.any() and not nan.all()
    assert torch.equal(nan, torch.isnan(pk_o))
    assert torch.equal(bf_o[~nan], pk_o[~nan])


def test_drop_in_runs_decode_steps_on_the_decode_kernel(dev):
    """A decode step through the drop-in (no mask beyond the causal rule) is the decode
    kernel with its automatic range count, bitwise, and matches the oracle."""
    from faquant_amd import _ops
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    case = (1, 32, 8, 1, 5000, True, "quantized_same", True, "123", None)
    (q, k, v), (qh, kh, vh, _), kw = _decode_inputs(case, dev)
    assert _ops.decode_shaped(32, 8, 1) and not _ops.decode_shaped(32, 8, 9)
    got, _ = simulated_flash_attention_forward(module(), *(to_dev(a, dev, torch.bfloat16) for a in (q, k, v)), None)
    n = _ops.decode_split_count(1, 8, 5000, _ops._device_cus(qh.device))
    out = torch.empty((1, 1, 32, 128), device=dev, dtype=torch.bfloat16)
    _ops.attention_decode(qh, 5000, k=kh, v=vh, split=n, out=out.transpose(1, 2), **kw)
    assert torch.equal(got, out)
    ref = _oracle(q, k, v, causal=True, levels="123", dtype="bfloat16")
    assert_close_attention(got.float().cpu().numpy(), ref, "drop-in decode step", **TIGHT)


@pytest.mark.parametrize("core", [False, True], ids=["sdpa", "qwen_core"])
def test_packed_cache_decode_steps_match_bf16_cache(dev, core):
    """Decode steps through the drop-in with packed caches: the packed rows grow by one
    position per step (and past the capacity), the output equals the bf16 caches' output
    bitwise at every step, and the last step matches the oracle."""
    from faquant_amd.qwen3 import attention_core
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    g = OI.rng(91)
    L0, steps = 1020, 6  # crosses the 1024-row capacity of the first packed buffer
    q, k, v = (OQ.bf16_round(g.standard_normal((1, h, L0 + steps, 128), dtype=np.float32)) for h in (8, 2, 2))
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))

    def mk(packed):
        m = module()
        m.faquant_kv_cache_packed = packed
        if core:
            m.faquant_qk_rotation = True
            m.faquant_qk_rotation_block_size = 64
        return m

    def call(m, lq, lk):
        if core:
            return attention_core(m, qt[:, :, lk - lq : lk], kt[:, :, :lk], vt[:, :, :lk])
        return simulated_flash_attention_forward(m, qt[:, :, lk - lq : lk], kt[:, :, :lk], vt[:, :, :lk], None)[0]

    packed, plain = mk(True), mk(False)
    a, b = call(packed, L0, L0), call(plain, L0, L0)  # prefill: bf16 operands for both
    assert torch.equal(a, b)
    cache0 = packed.faquant_k_matmul_qdq_cache
    for lk in range(L0 + 1, L0 + steps + 1):
        print(f"[packed decode] core={core} length {lk}", flush=True)
        a, b = call(packed, 1, lk), call(plain, 1, lk)
        assert torch.equal(a, b)
        kc = packed.faquant_k_matmul_qdq_cache
        assert kc.length == lk and packed.faquant_v_matmul_qdq_cache.length == lk
    assert kc is not cache0  # grown past the capacity
    kb = plain.faquant_k_matmul_qdq_cache.float().cpu().numpy()
    assert np.array_equal(_packed_values(kc), kb)
    if not core:
        ref = _oracle(q[:, :, -1:], k, v, causal=True, levels="123", dtype="bfloat16")  # bf16 output
        assert_close_attention(a.float().cpu().numpy(), ref, "packed decode step", **TIGHT)
