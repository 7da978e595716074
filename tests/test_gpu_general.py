"""GPU parity of the general attention kernel (faq_attention_fwd_general) against the oracle.

The general kernel takes what the MFMA kernel does not: key chunks other than 128 (any
size from 1 to 1024 keys, P quantized in 64-key groups from each chunk's start, the last one
zero-padded, sfa:292-338, 793-806), head_dim other than 128 (up to 256; Q/K/V groups of 64
along head_dim with a zero-padded tail), and fp32 Q/K/V whose matmul is not quantized, which
the reference multiplies as they are (sfa:723-724, 848-850).  It runs the simulator's steps
in fp32 with the device library's exp and tanh, so it differs from the oracle by fp32
rounding.  Bars, about ten times what each case reaches on MI355X: FP32 for fp32 outputs
(reached 1e-8..7e-7 relative Frobenius and max); TIGHT for bf16 outputs (most cases reach 0:
the bf16 rounding absorbs the fp32 differences); FEW_FLIPS where a quantized P code flipped
(key chunks of 1: 5e-6 / 1.7e-4; the softcap case: 3e-6 / 1.3e-4).  The
oracle's recurrence is pinned for these shapes by its own tests (dense closed forms with
chunks of 2..4 keys and 8-dim heads, tests/test_oracle_attention.py).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from oracle import hif4 as OQ
from tests.test_gpu_attention import TIGHT, assert_close_attention, module, to_dev, with_levels

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FP32 = dict(fro_tol=5e-6, max_tol=1e-5)
FEW_FLIPS = dict(fro_tol=5e-5, max_tol=2e-3)


def _inputs(seed, B, Hq, Hkv, Lq, Lk, D, *, q_scale=1.0):
    g = np.random.default_rng(seed)
    q = g.standard_normal((B, Hq, Lq, D)).astype(np.float32) * np.float32(q_scale)
    k = g.standard_normal((B, Hkv, Lk, D)).astype(np.float32)
    v = g.standard_normal((B, Hkv, Lk, D)).astype(np.float32)
    k[..., :4] *= 6.0  # a few outlier channels, as configuration 1 has
    return q, k, v


def _run(dev, q, k, v, dt, *, qk, pv, mode, causal=True, key_chunk=128, query_chunk=256, mask=None,
         sliding_window=None, softcap=None, levels="123", stats=False, diagnostics=False):
    from faquant_amd.simulated_flash_attention import (
        new_pv_normalizer_diagnostics,
        simulated_flash_attention_forward,
    )

    tdt = {"bfloat16": torch.bfloat16, "float16": torch.float16}.get(dt, torch.float32)
    qt, kt, vt = (to_dev(a, dev, tdt) for a in (q, k, v))
    mod = module(qk=qk, pv=pv, mode=mode, causal=causal, key_chunk=key_chunk, query_chunk=query_chunk)
    if diagnostics:
        mod.faquant_pv_normalizer_diagnostics = new_pv_normalizer_diagnostics()
    mt = None if mask is None else torch.from_numpy(mask).to(dev)
    with with_levels(levels):
        out, _ = simulated_flash_attention_forward(mod, qt, kt, vt, mt, sliding_window=sliding_window,
                                                   softcap=softcap)
    assert out.dtype == tdt and out.shape == (q.shape[0], q.shape[2], q.shape[1], q.shape[3])
    cfg = OA.SimConfig(pv_normalizer_mode=mode, query_chunk=query_chunk, key_chunk=key_chunk, qk_quant=qk,
                       pv_quant=pv, is_causal=causal, levels=dict.fromkeys("qkpv", levels))
    ostats = OA.new_stats() if stats else None
    odiag = OA.new_diagnostics() if diagnostics else None
    ref = OA.simulated_flash_attention(q, k, v, cfg, dtype=dt, attention_mask=mask, sliding_window=sliding_window,
                                       softcap=softcap, stats=ostats, diagnostics=odiag)
    extra = {}
    if stats:
        extra["stats"] = (dict(mod.faquant_simulated_attention_stats), ostats)
    if diagnostics:
        extra["diag"] = (mod.faquant_pv_normalizer_diagnostics, odiag)
    return out.float().cpu().numpy(), ref, extra


@pytest.mark.parametrize("qk,pv,mode", [(False, False, "unquantized"), (False, True, "unquantized"),
                                        (True, False, "unquantized"), (False, True, "quantized_same")])
def test_fp32_operands_with_a_matmul_unquantized(dev, qk, pv, mode):
    """fp32 Q/K/V with QK or PV quantization off: the reference multiplies the fp32 values."""
    q, k, v = _inputs(1, 1, 4, 2, 300, 300, 128)
    got, ref, extra = _run(dev, q, k, v, "float32", qk=qk, pv=pv, mode=mode, stats=True)
    assert extra["stats"][0] == extra["stats"][1]
    assert_close_attention(got, ref, f"fp32 qk={qk} pv={pv} {mode}", **FP32)


def test_fp32_unquantized_matches_dense_softmax(dev):
    """With both matmuls unquantized the tiled recurrence is plain causal softmax attention:
    compare with a float64 dense computation of the same fp32 inputs."""
    q, k, v = _inputs(2, 2, 2, 1, 64, 200, 96)
    got, _, _ = _run(dev, q, k, v, "float32", qk=False, pv=False, mode="unquantized", key_chunk=48)
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), np.repeat(k, 2, axis=1).astype(np.float64)) / np.sqrt(96)
    off = 200 - 64
    s = np.where(np.arange(200)[None, :] <= np.arange(64)[:, None] + off, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    dense = np.einsum("bhqk,bhkd->bhqd", p / p.sum(-1, keepdims=True), np.repeat(v, 2, axis=1).astype(np.float64))
    assert_close_attention(got, dense.transpose(0, 2, 1, 3), "dense fp64", **FP32)


@pytest.mark.parametrize("key_chunk", [1, 37, 64, 100, 256, 1024])
def test_key_chunks_other_than_128(dev, key_chunk):
    q, k, v = _inputs(3, 1, 4, 1, 260, 260, 128)
    q, k, v = (OQ.bf16_round(a) for a in (q, k, v))
    got, ref, extra = _run(dev, q, k, v, "bfloat16", qk=True, pv=True, mode="quantized_same", key_chunk=key_chunk,
                           query_chunk=64, stats=True)
    assert extra["stats"][0] == extra["stats"][1]
    assert_close_attention(got, ref, f"key_chunk {key_chunk}", **(FEW_FLIPS if key_chunk == 1 else TIGHT))


@pytest.mark.parametrize("D,levels", [(64, "123"), (96, "12"), (80, "13"), (200, "123"), (256, "123"), (8, "123")])
def test_head_dims_other_than_128(dev, D, levels):
    q, k, v = _inputs(4, 2, 2, 2, 150, 150, D)
    q, k, v = (OQ.bf16_round(a) for a in (q, k, v))
    got, ref, extra = _run(dev, q, k, v, "bfloat16", qk=True, pv=True, mode="quantized_same", levels=levels,
                           stats=True)
    assert extra["stats"][0] == extra["stats"][1]
    assert_close_attention(got, ref, f"head_dim {D} levels {levels}", **TIGHT)


def test_general_masks_window_softcap_and_chunked_prefill(dev):
    """2-D padding mask, sliding window, softcap and Lq < Lk through the general kernel."""
    q, k, v = _inputs(5, 2, 4, 2, 90, 170, 64)
    q, k, v = (OQ.bf16_round(a) for a in (q, k, v))
    mask = np.ones((2, 170), dtype=bool)
    mask[0, :25] = False
    mask[1, 60:75] = False
    got, ref, _ = _run(dev, q, k, v, "bfloat16", qk=True, pv=True, mode="quantized_same", key_chunk=96, mask=mask)
    assert_close_attention(got, ref, "padding mask, chunk 96", **TIGHT)
    got, ref, _ = _run(dev, q, k, v, "bfloat16", qk=True, pv=True, mode="unquantized", key_chunk=96,
                       sliding_window=33)
    assert_close_attention(got, ref, "sliding window, chunk 96", **TIGHT)
    got, ref, _ = _run(dev, q, k, v, "bfloat16", qk=True, pv=True, mode="quantized_same", key_chunk=64,
                       softcap=5.0)
    assert_close_attention(got, ref, "softcap, chunk 64", **FEW_FLIPS)
    got, ref, _ = _run(dev, q, k, v, "float32", qk=False, pv=False, mode="unquantized", causal=False,
                       key_chunk=50, softcap=3.0)
    assert_close_attention(got, ref, "fp32 unquantized non-causal softcap", **FP32)


@pytest.mark.parametrize("D,qk,pv,mode", [(64, False, False, "unquantized"), (96, True, True, "unquantized"),
                                          (72, True, False, "unquantized"), (32, False, True, "quantized_same"),
                                          (112, True, True, "quantized_same")])
def test_narrow_heads_on_the_mfma_kernel(dev, D, qk, pv, mode):
    """head_dim below 128 with key chunks of 128 and bf16-exact operands: zero-padded to 128 on
    the MFMA kernel (padding adds exact zeros to every score), with a padding mask, a window
    and the PV probe, against the oracle.  The MFMA kernel's P is exp2 of log2-scaled scores,
    a few ulp from the reference's exp, so a P-hat code on a rounding boundary can flip (one
    key's weight moves by a code step), as on the 128-dim path: the inputs and the bar are
    those of the MFMA kernel's random-configuration tests (queries x2, the FLIPS bar of
    tests/test_gpu_attention.py).  Unquantized P enters the MFMAs as two bf16 parts (16
    significant bits), as on the 128-dim path."""
    g = np.random.default_rng(12)
    q = OQ.bf16_round(g.standard_normal((2, 4, 150, D)).astype(np.float32) * 2)
    k = OQ.bf16_round(g.standard_normal((2, 2, 190, D)).astype(np.float32))
    v = OQ.bf16_round(g.standard_normal((2, 2, 190, D)).astype(np.float32))
    mask = np.ones((2, 190), dtype=bool)
    mask[1, :30] = False
    got, ref, extra = _run(dev, q, k, v, "bfloat16", qk=qk, pv=pv, mode=mode, mask=mask, stats=True,
                           diagnostics=pv)
    assert extra["stats"][0] == extra["stats"][1]
    assert_close_attention(got, ref, f"narrow D {D} qk={qk} pv={pv} {mode}")
    got, ref, _ = _run(dev, q, k, v, "bfloat16", qk=qk, pv=pv, mode=mode, sliding_window=40)
    assert_close_attention(got, ref, f"narrow D {D} window")
    if pv:
        mine, theirs = extra["diag"]
        assert mine["rows"] == theirs["rows"] and mine["p_values"] == theirs["p_values"]


@pytest.mark.parametrize("Lq,Lk", [(200, 150), (1, 300), (7, 7)])
def test_general_query_key_lengths(dev, Lq, Lk):
    """More query rows than keys (bottom-right causal: the first Lq - Lk rows see no key and
    output zeros), one decode row, and a sequence shorter than one chunk."""
    q, k, v = _inputs(9, 1, 4, 2, Lq, Lk, 64)
    q, k, v = (OQ.bf16_round(a) for a in (q, k, v))
    got, ref, extra = _run(dev, q, k, v, "bfloat16", qk=True, pv=True, mode="quantized_same", key_chunk=64,
                           query_chunk=32, stats=True)
    assert extra["stats"][0] == extra["stats"][1]
    assert_close_attention(got, ref, f"Lq {Lq} Lk {Lk}", **TIGHT)
    if Lq > Lk:
        assert not np.any(got[:, : Lq - Lk])


def test_general_dense_masks(dev):
    """3-D boolean and 4-D additive masks (sfa:430-454) with head_dim 64 and key chunks of 80."""
    q, k, v = _inputs(6, 1, 2, 1, 70, 140, 64)
    g = np.random.default_rng(60)
    bmask = g.random((1, 70, 140)) > 0.3
    bmask[:, :, 0] = True
    got, ref, _ = _run(dev, q, k, v, "float32", qk=True, pv=True, mode="quantized_same", key_chunk=80, mask=bmask)
    assert_close_attention(got, ref, "3-D boolean", **FP32)
    amask = (g.standard_normal((1, 2, 70, 140)) * 2).astype(np.float32)
    amask[..., 5:20] = -np.inf
    got, ref, _ = _run(dev, q, k, v, "float32", qk=False, pv=False, mode="unquantized", key_chunk=80, mask=amask)
    assert_close_attention(got, ref, "4-D additive, unquantized fp32", **FP32)


def test_general_pv_normalizer_probe(dev):
    """The PV-normalizer diagnostics of the general path equal the oracle's to fp32 rounding."""
    q, k, v = _inputs(7, 1, 4, 2, 200, 200, 64)
    q, k, v = (OQ.bf16_round(a) for a in (q, k, v))
    got, ref, extra = _run(dev, q, k, v, "bfloat16", qk=True, pv=True, mode="quantized_same", key_chunk=100,
                           diagnostics=True)
    assert_close_attention(got, ref, "probe run", **TIGHT)
    mine, theirs = extra["diag"]
    for key in ("rows", "p_values", "p_zeroed_values"):
        assert mine[key] == theirs[key], key
    for key in ("mass_ratio_sum", "p_error_sq_sum", "p_reference_sq_sum", "mass_ratio_min", "mass_ratio_max"):
        assert abs(mine[key] - theirs[key]) <= 1e-4 * max(abs(theirs[key]), 1e-30), (key, mine[key], theirs[key])
    assert sum(mine["mass_ratio_histogram"]) == sum(theirs["mass_ratio_histogram"])


def test_general_path_single_key_rows_are_exact(dev):
    """A row that sees one key outputs that key's (quantized) value: P = exp(0) = 1 exactly,
    P-hat(1) and the normalizer give V-hat itself (window 1, both normalizer modes)."""
    q, k, v = _inputs(8, 1, 2, 1, 40, 40, 96)
    for mode in ("quantized_same", "unquantized"):
        got, ref, _ = _run(dev, q, k, v, "float32", qk=True, pv=True, mode=mode, key_chunk=16, sliding_window=1)
        assert np.array_equal(got, ref), mode


@pytest.mark.parametrize("qk,pv,mode", [(True, True, "quantized_same"), (False, False, "unquantized"),
                                        (True, False, "unquantized")])
def test_fp16_operands(dev, qk, pv, mode):
    """fp16 Q/K/V (the reference quantizes them in fp16 and multiplies in fp32; the output keeps
    the query's dtype): the general kernel, against the oracle in fp16."""
    q, k, v = _inputs(10, 1, 4, 2, 130, 130, 128)
    q, k, v = (OQ.fp16_round(a) for a in (q, k, v))
    got, ref, extra = _run(dev, q, k, v, "float16", qk=qk, pv=pv, mode=mode, stats=True)
    assert extra["stats"][0] == extra["stats"][1]
    # fp16 outputs: one-ulp rounding differences (2^-11 relative) where P is not quantized
    # (reached 4.6e-6 / 6.8e-5), none where it is
    assert_close_attention(got, ref, f"fp16 qk={qk} pv={pv} {mode}", **(TIGHT if pv else FEW_FLIPS))


def test_fp16_quantized_operands_in_the_subnormal_range(dev):
    """Quantized fp16 operands run on the MFMA kernel through exact bf16 copies: V rows scaled
    into fp16's subnormal range (HiF4 values there are rounded to fp16 first, as the reference
    rounds its QDQ output to the input dtype) and tiny queries, against the oracle in fp16."""
    q, k, v = _inputs(11, 1, 4, 2, 200, 200, 128)
    v[:, 0] *= np.float32(2.0**-20)
    q[:, 1] *= np.float32(2.0**-12)
    q, k, v = (OQ.fp16_round(a) for a in (q, k, v))
    got, ref, _ = _run(dev, q, k, v, "float16", qk=True, pv=True, mode="quantized_same")
    assert np.any((np.abs(ref) < 2.0**-14) & (ref != 0))  # outputs in fp16's subnormal range
    assert_close_attention(got, ref, "fp16 subnormal operands", **TIGHT)


def test_general_refusals(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q = torch.randn(1, 2, 8, 128, device=dev)
    k = torch.randn(1, 1, 8, 128, device=dev)
    with pytest.raises(NotImplementedError, match="key chunks"):
        simulated_flash_attention_forward(module(key_chunk=2048), q, k, k, None)
    with pytest.raises(ValueError, match="key chunk size"):
        simulated_flash_attention_forward(module(key_chunk=0), q, k, k, None)
    big = torch.randn(1, 1, 8, 320, device=dev)
    with pytest.raises(NotImplementedError, match="head_dim"):
        simulated_flash_attention_forward(module(), big, big, big, None)


def _draw_general(n, seed=2027):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B = int(rng.integers(1, 3))
        hkv = int(rng.integers(1, 3))
        G = int(rng.choice([1, 2, 4]))
        lk = int(rng.integers(1, 400))
        lq = int(rng.integers(1, lk + 1)) if rng.random() < 0.8 else int(rng.integers(lk, lk + 100))
        D = int(rng.choice([16, 32, 64, 72, 96, 128, 160, 256]))
        chunk = int(rng.choice([16, 48, 64, 100, 128, 200, 256, 512]))
        dt = str(rng.choice(["bfloat16", "float32", "float16"]))
        qk, pv = bool(rng.random() < 0.7), bool(rng.random() < 0.7)
        mode = str(rng.choice(["quantized_same", "unquantized"])) if pv else "unquantized"
        causal = bool(rng.random() < 0.7)
        kind = str(rng.choice(["none", "left", "holes"]))
        window = None if rng.random() < 0.7 else int(rng.integers(1, 200))
        softcap = None if rng.random() < 0.8 else 3.0
        levels = str(rng.choice(["123", "12", "13"]))
        cases.append((i, B, hkv * G, hkv, lq, lk, D, chunk, dt, qk, pv, mode, causal, kind, window, softcap, levels))
    return cases


@pytest.mark.parametrize("case", _draw_general(20), ids=lambda c: f"g{c[0]}_D{c[6]}_T{c[7]}_{c[8]}")
def test_general_random_configuration(dev, case):
    """Seeded random shapes, chunks, dtypes, flags, masks and levels through the drop-in on the
    general kernel (and, for quantized fp16 at 128/128, the MFMA kernel), against the oracle,
    with equal stats counters."""
    from tests.test_gpu_masks import make_mask

    i, B, hq, hkv, lq, lk, D, chunk, dt, qk, pv, mode, causal, kind, window, softcap, levels = case
    print(f"[general random] {case}", flush=True)
    q, k, v = _inputs(500 + i, B, hq, hkv, lq, lk, D)
    rnd = {"bfloat16": OQ.bf16_round, "float16": OQ.fp16_round}.get(dt, lambda a: a)
    q, k, v = (rnd(a) for a in (q, k, v))
    mask = None if kind == "none" else make_mask(kind, B, lk, seed=i)
    got, ref, extra = _run(dev, q, k, v, dt, qk=qk, pv=pv, mode=mode, causal=causal, key_chunk=chunk, mask=mask,
                           sliding_window=window, softcap=softcap, levels=levels, stats=True)
    assert extra["stats"][0] == extra["stats"][1]
    # reached: 0 to 1.1e-5 relative Frobenius, 2.4e-4 max (one-ulp bf16/fp16 output flips)
    assert_close_attention(got, ref, str(case), fro_tol=1e-4, max_tol=3e-3)
