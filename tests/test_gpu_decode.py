"""Chunked prefill and decode through the drop-in: bottom-right causal attention with
q_len < k_len, and the decode K/V QDQ cache of the reference (sfa:243-289).

The reference's own test (test_simulated_flash_attention.py:267-304) grows a cache one
position at a time and requires the output to be bitwise equal to a fresh module's and
the cache to hold exactly `length` positions; the same checks run here at head_dim 128
and key tiles of 128.  Chunked prefill (eval_longbench.py:521-537) must equal one pass
bitwise, since every query row runs the same key-tile recurrence wherever it sits.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import TIGHT, _oracle, assert_close_attention, module, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _qkv(seed, hq, hkv, lq, lk):
    g = OI.rng(seed)
    q = OQ.bf16_round(g.standard_normal((1, hq, lq, 128), dtype=np.float32) * 2)
    k = OQ.bf16_round(g.standard_normal((1, hkv, lk, 128), dtype=np.float32))
    v = OQ.bf16_round(g.standard_normal((1, hkv, lk, 128), dtype=np.float32))
    return q, k, v


@pytest.mark.parametrize("chunk", [256, 300])
def test_chunked_prefill_equals_one_pass(dev, chunk):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(31, 8, 2, 700, 700))
    full, _ = simulated_flash_attention_forward(module(), q, k, v, None)
    mod = module()
    for start in range(0, 700, chunk):
        stop = min(start + chunk, 700)
        print(f"[chunk] {chunk} rows {start}:{stop}", flush=True)
        part, _ = simulated_flash_attention_forward(mod, q[:, :, start:stop], k[:, :, :stop], v[:, :, :stop], None)
        assert torch.equal(part, full[:, start:stop])


@pytest.mark.parametrize("lengths", [(300, 301, 302, 303), (382, 383, 384, 385, 386)])
def test_decode_kv_qdq_cache_is_bitwise_equal_to_full_requantization(dev, lengths):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    _, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(32, 4, 2, 1, max(lengths)))
    g = OI.rng(33)
    cached = module()
    # prefill of the first length - 1 positions fills the cache
    q0 = to_dev(OQ.bf16_round(g.standard_normal((1, 4, lengths[0] - 1, 128), dtype=np.float32)), dev, torch.bfloat16)
    simulated_flash_attention_forward(cached, q0, k[:, :, : lengths[0] - 1], v[:, :, : lengths[0] - 1], None)
    for length in lengths:
        print(f"[decode] length {length}", flush=True)
        kbuf = cached.faquant_k_matmul_qdq_cache.untyped_storage().data_ptr()
        query = to_dev(OQ.bf16_round(g.standard_normal((1, 4, 1, 128), dtype=np.float32)), dev, torch.bfloat16)
        actual, _ = simulated_flash_attention_forward(cached, query, k[:, :, :length], v[:, :, :length], None)
        fresh = module()
        reference, _ = simulated_flash_attention_forward(fresh, query, k[:, :, :length], v[:, :, :length], None)
        assert torch.equal(actual, reference)
        assert cached.faquant_k_matmul_qdq_cache.shape[-2] == length
        assert cached.faquant_v_matmul_qdq_cache.shape[-2] == length
        assert torch.equal(cached.faquant_k_matmul_qdq_cache, fresh.faquant_k_matmul_qdq_cache)
        assert torch.equal(cached.faquant_v_matmul_qdq_cache, fresh.faquant_v_matmul_qdq_cache)
        if length <= 384:
            # appended in place: the capacity-padded buffer was not reallocated
            assert cached.faquant_k_matmul_qdq_cache.untyped_storage().data_ptr() == kbuf


def test_decode_steps_equal_prefill_rows_and_match_oracle(dev):
    """Each decode step equals the same row of a one-pass prefill up to the fp32 order of
    the final sums; the prefill matches the oracle within the stated tolerance.
    fp32 inputs keep the output in fp32 (the drop-in returns the query dtype)."""
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = _qkv(34, 8, 2, 1000, 1000)
    qt, kt, vt = (to_dev(a, dev, torch.float32) for a in (q, k, v))
    full, _ = simulated_flash_attention_forward(module(), qt, kt, vt, None)
    assert_close_attention(full.float().cpu().numpy(), _oracle(q, k, v), "prefill 1000 keys", **TIGHT)
    mod = module()
    simulated_flash_attention_forward(mod, qt[:, :, :997], kt[:, :, :997], vt[:, :, :997], None)
    for length in (998, 999, 1000):
        out, _ = simulated_flash_attention_forward(mod, qt[:, :, length - 1 : length], kt[:, :, :length],
                                                   vt[:, :, :length], None)
        # decode runs split over key ranges: the same P-hat codes, O and l summed in another order
        ref = full[:, length - 1 : length]
        assert torch.allclose(out, ref, rtol=2e-6, atol=2e-6 * ref.abs().max().item())


def test_cache_is_not_reused_after_reset_or_mismatch(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(35, 4, 2, 1, 260))
    mod = module()
    simulated_flash_attention_forward(mod, q.expand(1, 4, 258, 128).contiguous(), k[:, :, :258], v[:, :, :258], None)
    # a caller that drops the cache (eval_longbench.py:541-542) forces a full quantization
    mod.faquant_k_matmul_qdq_cache = None
    mod.faquant_v_matmul_qdq_cache = None
    other = k.clone()
    other[:, :, :258] = -other[:, :, :258]  # different history: reuse would be wrong
    a, _ = simulated_flash_attention_forward(mod, q, other[:, :, :259], v[:, :, :259], None)
    b, _ = simulated_flash_attention_forward(module(), q, other[:, :, :259], v[:, :, :259], None)
    assert torch.equal(a, b)
    # a prefill chunk (q_len > 1) never appends (sfa:268-276)
    c, _ = simulated_flash_attention_forward(mod, q.expand(1, 4, 2, 128).contiguous(), k[:, :, :260], v[:, :, :260], None)
    d, _ = simulated_flash_attention_forward(module(), q.expand(1, 4, 2, 128).contiguous(), k[:, :, :260], v[:, :, :260], None)
    assert torch.equal(c, d)
    # quantization off: no cache (sfa:264-266)
    off = module(qk=False, pv=False)
    simulated_flash_attention_forward(off, q, k, v, None)
    assert off.faquant_k_matmul_qdq_cache is None and off.faquant_v_matmul_qdq_cache is None


def test_attention_core_decode_uses_the_cache(dev):
    from faquant_amd.qwen3 import attention_core

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in OI.qwen(36, 8, 2, 300))
    g = OI.rng(37)
    scale = to_dev(g.uniform(0.5, 2.0, size=(128,)), dev)
    offset = to_dev(g.standard_normal((2, 1, 128)) * 0.3, dev)

    def mk():
        m = module()
        m.faquant_qk_smooth_scale = scale
        m.faquant_qk_key_offset = offset
        m.faquant_qk_rotation = True
        m.faquant_qk_rotation_block_size = 64
        return m

    cached = mk()
    attention_core(cached, q[:, :, :298], k[:, :, :298], v[:, :, :298])
    for length in (299, 300):
        got = attention_core(cached, q[:, :, length - 1 : length], k[:, :, :length], v[:, :, :length])
        ref = attention_core(mk(), q[:, :, length - 1 : length], k[:, :, :length], v[:, :, :length])
        assert torch.equal(got, ref)
        assert cached.faquant_k_matmul_qdq_cache.shape[-2] == length


SPLIT_CASES = [
    # (B, Hq, Hkv, Lq, Lk, causal, mode, quant_p, p_levels, nsplit)
    (1, 32, 8, 1, 5000, True, "quantized_same", True, "123", None),   # Qwen3-8B decode step
    (2, 8, 2, 3, 1000, True, "quantized_same", True, "123", 6),
    (1, 4, 4, 1, 777, False, "quantized_same", True, "12", 3),       # non-causal, ragged
    # non-causal GQA, 2 position blocks per head group: 16 items in the head-major order,
    # 16 workgroups per range (one round), then 8 per range (two rounds)
    (2, 32, 4, 64, 3000, False, "quantized_same", True, "123", 4),
    (2, 32, 4, 64, 3000, False, "unquantized", True, "12", 32),
    (1, 4, 1, 5, 900, True, "unquantized", True, "123", 4),
    (1, 4, 1, 2, 640, True, "quantized_same", False, "123", 5),
    (1, 2, 1, 1, 300, True, "quantized_same", True, "13", 16),       # more ranges than tiles
    (1, 2, 1, 1, 40000, True, "quantized_same", True, "123", 300),   # the scan's carry over 256 splits
    (1, 4, 2, 2, 140000, True, "unquantized", True, "12", 1000),     # four scan chunks, 1094 tiles
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"_{c[6]}_{c[8]}")
def test_split_key_path_equals_one_pass(dev, case):
    """The split-key path gives every P-hat code of the one-pass recurrence (each range
    starts from the running maximum of the tiles before it); only the fp32 order of the
    final O and l sums differs.  Also checked against the oracle."""
    from faquant_amd import _ops

    B, Hq, Hkv, Lq, Lk, causal, mode, qp, lv, nsplit = case
    g = OI.rng(Lk + Lq)
    q = OQ.bf16_round(g.standard_normal((B, Hq, Lq, 128), dtype=np.float32) * 2)
    k = OQ.bf16_round(g.standard_normal((B, Hkv, Lk, 128), dtype=np.float32))
    v = OQ.bf16_round(g.standard_normal((B, Hkv, Lk, 128), dtype=np.float32))
    qh, _ = _ops.operand_prep(to_dev(q, dev, torch.bfloat16), levels=lv)
    kh, _ = _ops.operand_prep(to_dev(k, dev, torch.bfloat16), levels=lv)
    vt = _ops.operand_prep_vt(to_dev(v, dev, torch.bfloat16), levels=lv if qp else None)
    kw = dict(causal=causal, scale=128**-0.5, quant_p=qp, p_levels=lv, norm_same=mode == "quantized_same")
    outs, dens = [], []
    for split in (1, nsplit):
        out = torch.empty((B, Lq, Hq, 128), device=dev, dtype=torch.float32)
        den = torch.empty((B, Hq, Lq), device=dev, dtype=torch.float32)
        _ops.attention_fwd(qh, kh, vt, Lk, out=out.transpose(1, 2), row_den=den, split=split, **kw)
        outs.append(out.cpu().numpy())
        dens.append(den.cpu().numpy())
    if nsplit is None:
        assert _ops._split_count(B, Hq, Hkv, Lq, Lk) > 1  # the automatic choice splits a decode step
    print(f"[split] {case}", flush=True)
    np.testing.assert_allclose(outs[1], outs[0], rtol=1e-5, atol=1e-6 * np.abs(outs[0]).max())
    # l is a sum over up to ~10^5 keys (fp32 P in unquantized mode) taken in another order
    np.testing.assert_allclose(dens[1], dens[0], rtol=3e-6)
    ref = _oracle(q, k, v, causal=causal, levels=lv, mode=mode, qk=True, pv=qp)
    # the split path's row blocks see random keys x3: codes flip (reached 1.4e-5 / 1.3e-4)
    assert_close_attention(outs[1], ref, f"split {case}", fro_tol=2e-4, max_tol=2e-3)
