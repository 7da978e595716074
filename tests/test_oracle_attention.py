"""Pins the numpy attention oracle.

1. Golden outputs written by the reference simulator with HiF4 Q/K/P/V
   (tests/golden/attention.npz): bf16 outputs within two bf16 ulps, differing
   on at most 0.1% of elements (exp/GEMM rounding flips a P code now and then), fp32
   outputs within 1e-6 of the output scale; stats counters exactly.
2. The reference's own simulator tests, restated on the oracle with the same
   torch-seeded inputs (tests/test_simulated_flash_attention.py, whose module
   fake selects the int format), and the single-tile equality with the
   differentiable core (tests/test_qad_attention.py:84-117).
"""

import numpy as np
import pytest

from oracle import attention as A
from oracle import hadamard as H
from oracle import hif4
from tests.golden.cases import CASES, build_inputs, golden_output

torch = pytest.importorskip("torch")


def cfg_int(*, qk=False, pv=False, query_chunk=3, key_chunk=4, bits=4, group_size=4, mode="unquantized"):
    spec = A.QuantSpec(quant_format="int", bits=bits, group_size=group_size)
    return A.SimConfig(
        query_chunk=query_chunk, key_chunk=key_chunk, qk_quant=qk, pv_quant=pv,
        qk_spec=spec, pv_spec=spec, pv_normalizer_mode=mode,
    )


def randn(*shape, scale=1.0):
    return (torch.randn(*shape) * scale).numpy()


def dense_causal(q, k, v):
    reps = q.shape[1] // k.shape[1]
    k = np.repeat(k, reps, axis=1).astype(np.float64)
    v = np.repeat(v, reps, axis=1).astype(np.float64)
    s = q.astype(np.float64) @ np.swapaxes(k, -1, -2) * q.shape[-1] ** -0.5
    qp = np.arange(q.shape[-2]) + k.shape[-2] - q.shape[-2]
    allowed = np.arange(k.shape[-2])[None, :] <= qp[:, None]
    s = np.where(allowed, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        p = np.exp(s - np.where(np.isfinite(m), m, 0))
        p = np.nan_to_num(p / p.sum(axis=-1, keepdims=True))
    return np.swapaxes(p @ v, 1, 2)


def dense_padded(q, k, v, mask):
    out = np.zeros((q.shape[0], q.shape[-2], q.shape[1], q.shape[-1]))
    for b in range(q.shape[0]):
        idx = np.nonzero(mask[b])[0]
        out[b, idx] = dense_causal(q[b : b + 1, :, idx], k[b : b + 1, :, idx], v[b : b + 1, :, idx])[0]
    return out


# ---------------------------------------------------------------- golden parity

@pytest.mark.parametrize("case", list(CASES))
def test_matches_reference_golden_outputs(golden_attention, case):
    builder, mk, _, levels, rot = CASES[case]
    q, k, v, dt = build_inputs(builder)
    rnd = hif4.bf16_round if dt == "bfloat16" else None
    if rot is not None:
        q = H.qk_rotation(q, block_size=rot, out_round=rnd)
        k = H.qk_rotation(k, block_size=rot, out_round=rnd)
    cfg = A.SimConfig(
        qk_quant=mk["qk"], pv_quant=mk["pv"], pv_normalizer_mode=mk["mode"],
        levels=dict.fromkeys("qkpv", levels), is_causal=mk.get("causal", True),
    )
    stats = A.new_stats()
    out = A.simulated_flash_attention(q, k, v, cfg, dtype=dt, stats=stats)
    ref = golden_output(golden_attention, case)
    if case == "c1_unq":
        out = out[:, :, :4]
    keys = [str(s) for s in golden_attention[f"{case}__stats_keys"]]
    assert {kk: stats[kk] for kk in keys} == dict(zip(keys, golden_attention[f"{case}__stats"].tolist()))
    if dt == "bfloat16":
        ulp = np.ldexp(np.float32(1.0), np.frexp(np.abs(ref))[1] - 8).astype(np.float32)
        diff = np.abs(out - ref)
        assert np.all(diff <= 2 * ulp + 1e-30), float((diff / ulp).max())
        assert np.mean(diff > 0) < 1e-3
    else:
        np.testing.assert_allclose(out, ref, rtol=0, atol=1e-6 * np.abs(ref).max())


# ------------------------------------------------ reference simulator tests

def test_streaming_matches_dense_causal_gqa_with_block_tails():
    torch.manual_seed(1)
    q, k, v = randn(2, 4, 7, 8), randn(2, 2, 11, 8), randn(2, 2, 11, 8)
    out = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=3, key_chunk=4, group_size=8), scaling=8**-0.5)
    np.testing.assert_allclose(out, dense_causal(q, k, v), atol=2e-6, rtol=2e-6)


def test_skipping_fully_future_tiles_is_bitwise_equal():
    torch.manual_seed(19)
    q, k, v = randn(1, 4, 11, 8), randn(1, 2, 11, 8), randn(1, 2, 11, 8)
    opt = cfg_int(qk=True, pv=True, query_chunk=3, key_chunk=2)
    ref = cfg_int(qk=True, pv=True, query_chunk=3, key_chunk=2)
    ref.skip_fully_masked_tiles = False
    so, sr = A.new_stats(), A.new_stats()
    a = A.simulated_flash_attention(q, k, v, opt, stats=so)
    b = A.simulated_flash_attention(q, k, v, ref, stats=sr)
    np.testing.assert_array_equal(a, b)
    assert so["qk_tiles"] < sr["qk_tiles"] and so["pv_tiles"] < sr["pv_tiles"]
    mask = np.ones((1, 11), bool)
    np.testing.assert_array_equal(
        A.simulated_flash_attention(q, k, v, opt, attention_mask=mask),
        A.simulated_flash_attention(q, k, v, ref, attention_mask=mask),
    )


def test_bottom_right_causal_zeroes_queries_without_any_keys():
    torch.manual_seed(2)
    q, k, v = randn(1, 2, 7, 4), randn(1, 1, 3, 4), randn(1, 1, 3, 4)
    out = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=2, key_chunk=2), softcap=0)
    assert np.count_nonzero(out[:, :4]) == 0
    np.testing.assert_allclose(out, dense_causal(q, k, v), atol=2e-6, rtol=2e-6)


def test_two_dimensional_padding_matches_unpadded_batches():
    torch.manual_seed(3)
    q, k, v = randn(2, 4, 7, 4), randn(2, 2, 7, 4), randn(2, 2, 7, 4)
    mask = np.array([[0, 0, 1, 1, 1, 1, 1], [1, 1, 1, 1, 0, 0, 0]], bool)
    out = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=3, key_chunk=4), attention_mask=mask)
    np.testing.assert_allclose(out, dense_padded(q, k, v, mask), atol=2e-6, rtol=2e-6)
    assert np.count_nonzero(out[0, :2]) == 0 and np.count_nonzero(out[1, 4:]) == 0


def test_four_dimensional_additive_masks_keep_fully_masked_rows_zero():
    torch.manual_seed(4)
    q, k, v = randn(1, 2, 5, 4), randn(1, 1, 5, 4), randn(1, 1, 5, 4)
    mask = np.full((1, 1, 5, 5), np.finfo(np.float32).min, np.float32)
    mask[..., 1:, 0] = 0
    out = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=2, key_chunk=3), attention_mask=mask)
    assert np.count_nonzero(out[:, 0]) == 0 and np.isfinite(out).all()
    torch.manual_seed(9)
    q, k, v = randn(1, 2, 3, 4), randn(1, 1, 3, 4), randn(1, 1, 3, 4)
    m16 = np.full((1, 1, 3, 3), np.finfo(np.float16).min, np.float16)
    out = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=2, key_chunk=2), attention_mask=m16)
    assert np.count_nonzero(out) == 0 and np.isfinite(out).all()


def test_decode_with_padding_and_sliding_window():
    torch.manual_seed(8)
    q, k, v = randn(2, 4, 1, 4), randn(2, 2, 7, 4), randn(2, 2, 7, 4)
    mask = np.array([[0, 0, 1, 1, 1, 1, 1], [0, 1, 1, 1, 1, 1, 1]], bool)
    out = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=1, key_chunk=3), attention_mask=mask, sliding_window=3)
    rk, rv = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    for b in range(2):
        idx = np.nonzero(mask[b])[0][-3:]
        s = q[b].astype(np.float64) @ np.swapaxes(rk[b][:, idx], -1, -2) * 0.5
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        np.testing.assert_allclose(out[b, 0], (p @ rv[b][:, idx])[:, 0], atol=2e-6, rtol=2e-6)


def test_noncausal_sliding_window_masks_both_sides():
    torch.manual_seed(14)
    q, k, v = randn(1, 2, 5, 4), randn(1, 2, 5, 4), randn(1, 2, 5, 4)
    out = A.simulated_flash_attention(
        q, k, v, cfg_int(query_chunk=2, key_chunk=3), is_causal=False, sliding_window=2
    )
    s = q.astype(np.float64) @ np.swapaxes(k, -1, -2) * 0.5
    pos = np.arange(5)
    s = np.where(np.abs(pos[None, :] - pos[:, None]) < 2, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(out, np.swapaxes(p @ v, 1, 2), atol=2e-6, rtol=2e-6)


def test_multi_token_decode_with_left_padding():
    torch.manual_seed(11)
    q, k, v = randn(2, 4, 3, 4), randn(2, 2, 7, 4), randn(2, 2, 7, 4)
    mask = np.array([[0, 0, 1, 1, 1, 1, 1], [0, 1, 1, 1, 1, 1, 1]], bool)
    out = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=2, key_chunk=3), attention_mask=mask)
    rk, rv = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    for b in range(2):
        idx = np.nonzero(mask[b])[0]
        s = q[b].astype(np.float64) @ np.swapaxes(rk[b][:, idx], -1, -2) * 0.5
        qp = np.arange(3) + idx.size - 3
        s = np.where(np.arange(idx.size)[None, :] > qp[:, None], -np.inf, s)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        np.testing.assert_allclose(out[b], np.swapaxes(p @ rv[b][:, idx], 0, 1), atol=2e-6, rtol=2e-6)


def test_qk_pv_quantization_modes_are_independent_and_counted():
    torch.manual_seed(5)
    q, k, v = randn(1, 4, 5, 4, scale=3), randn(1, 2, 7, 4, scale=2), randn(1, 2, 7, 4, scale=4)
    outs = {}
    for name, qk, pv in (("none", False, False), ("qk", True, False), ("pv", False, True), ("both", True, True)):
        st = A.new_stats()
        outs[name] = A.simulated_flash_attention(q, k, v, cfg_int(qk=qk, pv=pv, bits=2), stats=st)
        assert st["calls"] == 1 and st["qk_tiles"] == st["pv_tiles"] == 4
        assert st["qk_quantized_tiles"] == (4 if qk else 0) and st["pv_quantized_tiles"] == (4 if pv else 0)
        assert st["q_quant_calls"] == (2 if qk else 0) and st["k_quant_calls"] == (4 if qk else 0)
        assert st["p_quant_calls"] == (4 if pv else 0) and st["v_quant_calls"] == (4 if pv else 0)
        for op, en in (("q", qk), ("k", qk), ("p", pv), ("v", pv)):
            assert (st[f"{op}_quantized_values"] > 0) is en
            assert st[f"{op}_quant_padding_values"] == (20 if op == "p" and en else 0)
    assert not np.array_equal(outs["none"], outs["qk"]) and not np.array_equal(outs["none"], outs["pv"])
    assert not np.array_equal(outs["qk"], outs["both"])


def test_single_tile_quantization_matches_operand_level_reference():
    torch.manual_seed(12)
    q, k, v = randn(1, 2, 2, 4, scale=3), randn(1, 2, 3, 4, scale=2), randn(1, 2, 3, 4, scale=4)
    fq = lambda t: hif4.fake_quantize(t, bits=2, group_size=4)  # noqa: E731
    for qk, pv in ((False, False), (True, False), (False, True), (True, True)):
        out = A.simulated_flash_attention(
            q, k, v, cfg_int(qk=qk, pv=pv, query_chunk=4, key_chunk=4, bits=2), is_causal=False
        )
        qo, ko = (fq(q), fq(k)) if qk else (q, k)
        s = (np.matmul(qo, np.swapaxes(ko, -1, -2)) * np.float32(0.5)).astype(np.float32)
        p = np.exp(s - s.max(-1, keepdims=True)).astype(np.float32)
        den = p.sum(-1, keepdims=True)
        po = fq(np.concatenate([p, np.zeros((*p.shape[:-1], 1), np.float32)], -1))[..., :3] if pv else p
        vo = fq(v) if pv else v
        np.testing.assert_allclose(out, np.swapaxes((po @ vo) / den, 1, 2), atol=2e-6, rtol=2e-6)


def test_normalizer_modes_without_quantization_are_identical():
    torch.manual_seed(21)
    q, k, v = randn(1, 4, 6, 8), randn(1, 2, 9, 8), randn(1, 2, 9, 8)
    exp = dense_causal(q, k, v)
    outs = {}
    for mode in A.PV_NORMALIZER_MODES:
        outs[mode] = A.simulated_flash_attention(q, k, v, cfg_int(query_chunk=2, key_chunk=4, group_size=8, mode=mode))
        np.testing.assert_allclose(outs[mode], exp, atol=2e-6, rtol=2e-6)
    np.testing.assert_array_equal(outs["unquantized"], outs["quantized_same"])


def test_constant_scores_make_modes_identical_and_unit_values_exact():
    q, k = np.zeros((1, 2, 6, 4), np.float32), np.zeros((1, 1, 12, 4), np.float32)
    torch.manual_seed(0)
    v = randn(1, 1, 12, 4)
    outs = {m: A.simulated_flash_attention(q, k, v, cfg_int(pv=True, query_chunk=3, key_chunk=4, mode=m))
            for m in A.PV_NORMALIZER_MODES}
    np.testing.assert_array_equal(outs["unquantized"], outs["quantized_same"])
    torch.manual_seed(22)
    q, k = randn(1, 4, 5, 4, scale=2), randn(1, 2, 5, 4, scale=2)
    ones = np.ones((1, 2, 5, 4), np.float32)
    same = A.simulated_flash_attention(q, k, ones, cfg_int(pv=True, query_chunk=2, key_chunk=4, bits=2, mode="quantized_same"))
    np.testing.assert_allclose(same, np.ones_like(same), atol=1e-6, rtol=1e-6)
    mism = A.simulated_flash_attention(q, k, ones, cfg_int(pv=True, query_chunk=2, key_chunk=4, bits=2))
    assert float(np.abs(mism - 1.0).max()) > 1e-3


def test_normalizers_are_stable_across_tile_shapes():
    torch.manual_seed(23)
    q, k, v = randn(1, 4, 8, 4), randn(1, 2, 16, 4), randn(1, 2, 16, 4)
    for mode in A.PV_NORMALIZER_MODES:
        base = None
        for qc, kc in ((2, 4), (4, 8), (8, 16)):
            out = A.simulated_flash_attention(q, k, v, cfg_int(qk=True, pv=True, query_chunk=qc, key_chunk=kc, mode=mode))
            if base is None:
                base = out
            else:
                np.testing.assert_allclose(out, base, atol=2e-6, rtol=2e-6)


def test_quantized_same_matches_dense_gqa_with_masked_short_tail():
    torch.manual_seed(24)
    q, k, v = randn(1, 4, 3, 4, scale=2), randn(1, 2, 7, 4, scale=2), randn(1, 2, 7, 4, scale=2)
    out = A.simulated_flash_attention(q, k, v, cfg_int(pv=True, query_chunk=4, key_chunk=8, bits=3, mode="quantized_same"))
    rk, rv = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    s = (np.matmul(q, np.swapaxes(rk, -1, -2)) * np.float32(0.5)).astype(np.float32)
    allowed = np.arange(7)[None, :] <= (np.arange(3) + 4)[:, None]
    s = np.where(allowed, s, -np.inf)
    p = np.where(allowed, np.exp(s - s.max(-1, keepdims=True)), 0).astype(np.float32)
    pq = hif4.fake_quantize(np.concatenate([p, np.zeros((*p.shape[:-1], 1), np.float32)], -1), bits=3, group_size=4)[..., :7]
    vq = hif4.fake_quantize(rv, bits=3, group_size=4)
    np.testing.assert_allclose(out, np.swapaxes((pq @ vq) / pq.sum(-1, keepdims=True), 1, 2), atol=2e-6, rtol=2e-6)


def test_diagnostics_dense_mass_ratio_and_mode_independence():
    torch.manual_seed(12)
    q, k, v = randn(1, 2, 2, 4, scale=3), randn(1, 2, 3, 4, scale=2), randn(1, 2, 3, 4, scale=4)
    d = A.new_diagnostics()
    A.simulated_flash_attention(q, k, v, cfg_int(pv=True, query_chunk=4, key_chunk=4, bits=2), is_causal=False, diagnostics=d)
    s = (np.matmul(q, np.swapaxes(k, -1, -2)) * np.float32(0.5)).astype(np.float32)
    p = np.exp(s - s.max(-1, keepdims=True)).astype(np.float32)
    pq = hif4.fake_quantize(np.concatenate([p, np.zeros((*p.shape[:-1], 1), np.float32)], -1), bits=2, group_size=4)[..., :3]
    ratios = pq.sum(-1) / p.sum(-1)
    summ = A.summarize_diagnostics(d)
    assert summ["rows"] == ratios.size
    assert abs(summ["mass_ratio_mean"] - float(ratios.mean())) < 1e-6
    assert summ["p_zero_collapse_rate"] > 0.0
    torch.manual_seed(25)
    q, k, v = randn(1, 4, 6, 4, scale=2), randn(1, 2, 9, 4, scale=2), randn(1, 2, 9, 4, scale=2)
    summaries = {}
    for mode in A.PV_NORMALIZER_MODES:
        d = A.new_diagnostics()
        A.simulated_flash_attention(q, k, v, cfg_int(pv=True, query_chunk=2, key_chunk=4, bits=2, mode=mode), diagnostics=d)
        summaries[mode] = A.summarize_diagnostics(d)
    a, b = summaries["unquantized"], summaries["quantized_same"]
    assert a["mass_ratio_histogram"] == b["mass_ratio_histogram"] and a["rows"] == b["rows"]
    assert a["mean_relative_scale_error"] < -1e-3 and a["mass_ratio_fraction_below_one"] > 0.5


@pytest.mark.parametrize(
    "qk,pv,mode",
    [(False, False, "unquantized"), (True, False, "unquantized"), (True, True, "unquantized"), (True, True, "quantized_same")],
)
def test_hif4_single_tile_equals_tiled_when_one_tile_covers_every_key(qk, pv, mode):
    """tests/test_qad_attention.py:84-117 with HiF4 (levels 123), D=64."""
    torch.manual_seed(7)
    q, k, v = randn(2, 4, 96, 64), randn(2, 2, 96, 64), randn(2, 2, 96, 64)
    cfg = A.SimConfig(query_chunk=512, key_chunk=96, qk_quant=qk, pv_quant=pv, pv_normalizer_mode=mode)
    tiled = A.simulated_flash_attention(q, k, v, cfg)
    single = A.single_tile_attention(q, k, v, cfg)
    np.testing.assert_allclose(single, tiled, atol=1e-5, rtol=1e-5)


def test_validation_errors():
    q = np.zeros((1, 2, 3, 4), np.float32)
    k = np.zeros((1, 1, 3, 4), np.float32)
    with pytest.raises(ValueError, match="matching K/V"):
        A.simulated_flash_attention(q, k, np.zeros((1, 1, 4, 4), np.float32), cfg_int())
    with pytest.raises(ValueError, match="divisible"):
        A.simulated_flash_attention(np.zeros((1, 3, 3, 4), np.float32), np.zeros((1, 2, 3, 4), np.float32),
                                    np.zeros((1, 2, 3, 4), np.float32), cfg_int())
    with pytest.raises(ValueError, match="sliding_window"):
        A.simulated_flash_attention(q, k, k, cfg_int(), sliding_window=0)
