"""The Qwen3 attention core (qwen3.py:90-166) and per-operand HiF4 levels on the GPU.

- ``faquant_attention_input_quant``: the excursion's Q/K/V go through the core quantizer
  and then through the simulator's own operand QDQ (qwen3.py:132-136; HiF4 QDQ is not
  idempotent, so both count), against the oracle running the same two QDQs;
- ``sliding_window`` and ``cache_position`` reach the kernel through attention_core as they
  reach the reference's attention interface (qwen3.py:154-165, sfa:511-520);
- the PV-normalizer probe through attention_core equals the drop-in's;
- mixed per-operand levels (FAQUANT_HIF4_ATTN_OPERAND_LEVELS, hif4.py:29-43) through the
  drop-in and attention_core against oracle.attention.SimConfig(levels=...).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from oracle import hadamard as OH
from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import assert_close_attention, module, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

HIF4 = {"quant_format": "hif4", "bits": 4, "group_size": 64, "symmetric": True, "clip_ratio": 1.0}


def _qwen_module(block=64):
    m = module()
    m.faquant_qk_rotation = True
    m.faquant_qk_rotation_block_size = block
    return m


def operand_levels(table):
    """Temporarily set the attention operands' HiF4 levels (the env-derived table)."""
    from faquant_amd import hif4 as H

    class _Ctx:
        def __enter__(self):
            self.saved = dict(H.HIF4_ATTN_OPERAND_SCALE_LEVELS)
            H.HIF4_ATTN_OPERAND_SCALE_LEVELS.update(table)

        def __exit__(self, *exc):
            H.HIF4_ATTN_OPERAND_SCALE_LEVELS.clear()
            H.HIF4_ATTN_OPERAND_SCALE_LEVELS.update(self.saved)

    return _Ctx()


def test_input_quant_runs_both_qdqs(dev):
    from faquant_amd.qwen3 import attention_core

    q, k, v = OI.qwen(51, 8, 2, 300)
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    mod = _qwen_module()
    mod.faquant_attention_input_quant = True
    mod.faquant_core_quant_kwargs = dict(HIF4)
    got = attention_core(mod, qt, kt, vt).float().cpu().numpy()
    qr = OQ.bf16_round(OH.block_hadamard_transform(q, 64))
    kr = OQ.bf16_round(OH.block_hadamard_transform(k, 64))
    iq = lambda a: OQ.fake_quantize(a, quant_format="hif4", group_size=64, dtype="bfloat16")  # noqa: E731
    cfg = OA.SimConfig(pv_normalizer_mode="quantized_same")
    ref = OA.simulated_flash_attention(iq(qr), iq(kr), iq(v), cfg, dtype="bfloat16")
    assert_close_attention(got, ref, "input quant")
    single = OA.simulated_flash_attention(qr, kr, v, cfg, dtype="bfloat16")
    assert np.linalg.norm(ref - single) / np.linalg.norm(single) > 1e-3  # the second QDQ is visible
    # non-HiF4 core formats are refused, not computed differently
    mod.faquant_core_quant_kwargs = dict(HIF4, quant_format="int")
    with pytest.raises(NotImplementedError):
        attention_core(mod, qt, kt, vt)


def test_sliding_window_through_attention_core(dev):
    from faquant_amd.qwen3 import attention_core, post_rope_qk_transform
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = OI.qwen(52, 8, 2, 400)
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    for window in (1, 100, 300):
        fused = attention_core(_qwen_module(), qt, kt, vt, sliding_window=window)
        qr, kr = post_rope_qk_transform(qt, kt, rotation=True, rotation_block_size=64)
        two, _ = simulated_flash_attention_forward(module(), qr, kr, vt, None, sliding_window=window)
        assert torch.equal(fused, two), window
        qo = OQ.bf16_round(OH.block_hadamard_transform(q, 64))
        ko = OQ.bf16_round(OH.block_hadamard_transform(k, 64))
        ref = OA.simulated_flash_attention(qo, ko, v, OA.SimConfig(pv_normalizer_mode="quantized_same"),
                                           sliding_window=window, dtype="bfloat16")
        assert_close_attention(fused.float().cpu().numpy(), ref, f"window {window}")


def test_cache_position_trims_a_static_cache(dev):
    from faquant_amd.qwen3 import attention_core

    q, k, v = OI.qwen(53, 8, 2, 300)
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    q_new = qt[:, :, 150:200].contiguous()  # a chunk at positions 150..199 of a 300-slot buffer
    got = attention_core(_qwen_module(), q_new, kt, vt, cache_position=torch.arange(150, 200, device=dev))
    want = attention_core(_qwen_module(), q_new, kt[:, :, :200].contiguous(), vt[:, :, :200].contiguous())
    assert torch.equal(got, want)
    untrimmed = attention_core(_qwen_module(), q_new, kt, vt)
    assert not torch.equal(got, untrimmed)  # the unwritten slots would otherwise be attended


def test_probe_through_attention_core(dev):
    from faquant_amd.qwen3 import attention_core, post_rope_qk_transform
    from faquant_amd.simulated_flash_attention import (
        new_pv_normalizer_diagnostics,
        simulated_flash_attention_forward,
        summarize_pv_normalizer_diagnostics,
    )

    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in OI.qwen(54, 8, 2, 500))
    a = _qwen_module()
    a.faquant_pv_normalizer_diagnostics = new_pv_normalizer_diagnostics()
    out_a = attention_core(a, qt, kt, vt)
    b = module()
    b.faquant_pv_normalizer_diagnostics = new_pv_normalizer_diagnostics()
    qr, kr = post_rope_qk_transform(qt, kt, rotation=True, rotation_block_size=64)
    out_b, _ = simulated_flash_attention_forward(b, qr, kr, vt, None)
    assert torch.equal(out_a, out_b)
    sa = summarize_pv_normalizer_diagnostics(a.faquant_pv_normalizer_diagnostics)
    assert sa == summarize_pv_normalizer_diagnostics(b.faquant_pv_normalizer_diagnostics)
    assert sa["rows"] == 8 * 500
    assert torch.equal(out_a, attention_core(_qwen_module(), qt, kt, vt))  # the probe changes nothing


MIXES = [
    {"q": "12", "k": "123", "p": "13", "v": "12"},
    {"q": "13", "k": "12", "p": "123", "v": "13"},
    {"q": "123", "k": "123", "p": "12", "v": "123"},
]


@pytest.mark.parametrize("mix", MIXES, ids=lambda m: "_".join(f"{k}{v}" for k, v in m.items()))
def test_mixed_operand_levels_match_oracle(dev, mix):
    from faquant_amd.qwen3 import attention_core
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = OI.qwen(55, 8, 2, 333, student_t_keys=True)
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    cfg = OA.SimConfig(pv_normalizer_mode="quantized_same", levels=dict(mix))
    ref = OA.simulated_flash_attention(q, k, v, cfg, dtype="bfloat16")
    with operand_levels(mix):
        out, _ = simulated_flash_attention_forward(module(), qt, kt, vt, None)
        core = attention_core(module(), qt, kt, vt)
    assert_close_attention(out.float().cpu().numpy(), ref, f"mix {mix}")
    assert torch.equal(out, core)
    # a mix is not the uniform setting: the result moves
    uniform = OA.simulated_flash_attention(q, k, v, OA.SimConfig(pv_normalizer_mode="quantized_same"),
                                           dtype="bfloat16")
    assert np.abs(ref - uniform).max() > 0
