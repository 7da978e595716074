"""The PV-normalizer probe (sfa:36-185, 835-869) through the drop-in.

The probe is the kernel's diagnostic instantiation.  It computes the same outputs and
additionally returns per-row sums (sum P-hat, sum P, #(P-hat = 0 < P), sum (P-hat - P)^2,
sum P^2).  The checks mirror the reference's own probe tests
(test_simulated_flash_attention.py:496-600, 780-815):
- the probe leaves outputs and stats untouched;
- it is idle without PV quantization;
- its summary does not depend on the normalizer mode;
- constant scores give one exact ratio across many key tiles.
The summary also matches the oracle's probe within the attention tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from tests.test_gpu_attention import module, to_dev
from tests.test_gpu_masks import _qkv, make_mask

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _probed(mode="quantized_same", pv=True, causal=True):
    from faquant_amd.simulated_flash_attention import new_pv_normalizer_diagnostics

    m = module(mode=mode, pv=pv, causal=causal)
    m.faquant_pv_normalizer_diagnostics = new_pv_normalizer_diagnostics()
    return m


def test_probe_leaves_outputs_and_stats_untouched(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(13, 1, 8, 2, 700, 700))
    probed, plain = _probed(), module()
    a, _ = simulated_flash_attention_forward(probed, q, k, v, None)
    b, _ = simulated_flash_attention_forward(plain, q, k, v, None)
    assert torch.equal(a, b)
    assert probed.faquant_simulated_attention_stats == plain.faquant_simulated_attention_stats
    assert probed.faquant_pv_normalizer_diagnostics["rows"] == 8 * 700


def test_probe_is_idle_without_pv_quantization(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward, summarize_pv_normalizer_diagnostics

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(14, 1, 4, 1, 300, 300))
    m = _probed(pv=False)
    simulated_flash_attention_forward(m, q, k, v, None)
    summary = summarize_pv_normalizer_diagnostics(m.faquant_pv_normalizer_diagnostics)
    assert summary["rows"] == 0.0 and "mass_ratio_mean" not in summary


def test_probe_summary_is_mode_independent(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward, summarize_pv_normalizer_diagnostics

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in _qkv(21, 1, 8, 2, 500, 500))
    summaries = {}
    for mode in ("unquantized", "quantized_same"):
        m = _probed(mode=mode)
        simulated_flash_attention_forward(m, q, k, v, None)
        summaries[mode] = summarize_pv_normalizer_diagnostics(m.faquant_pv_normalizer_diagnostics)
    a, b = summaries["unquantized"], summaries["quantized_same"]
    assert a == b
    assert sum(a["mass_ratio_histogram"]) == a["rows"]
    assert abs(a["mean_relative_scale_error"]) > 1e-4  # the probe measured a real mismatch


def test_probe_constant_scores_give_one_exact_ratio(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward, summarize_pv_normalizer_diagnostics

    q = torch.zeros(1, 2, 600, 128, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 600, 128, device=dev, dtype=torch.bfloat16)
    v = torch.randn(1, 1, 600, 128, device=dev).to(torch.bfloat16)
    m = _probed()
    simulated_flash_attention_forward(m, q, k, v, None)
    s = summarize_pv_normalizer_diagnostics(m.faquant_pv_normalizer_diagnostics)
    # every P is 1; HiF4 123 of a constant group is 0.9375 (scale 0.15625, code 6 at 2^2)
    assert s["rows"] == 1200 and s["mass_ratio_min"] == s["mass_ratio_max"] == 0.9375
    assert s["p_zero_collapse_rate"] == 0.0


@pytest.mark.parametrize("mode", ["quantized_same", "unquantized"])
@pytest.mark.parametrize("masked", [False, True])
def test_probe_matches_the_oracle(dev, mode, masked):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward, summarize_pv_normalizer_diagnostics

    B = 2 if masked else 1
    q, k, v = _qkv(31, B, 8, 2, 400, 400)
    mask = make_mask("left", B, 400, seed=31) if masked else None
    m = _probed(mode=mode)
    simulated_flash_attention_forward(m, *(to_dev(a, dev, torch.bfloat16) for a in (q, k, v)),
                                      None if mask is None else torch.from_numpy(mask).to(dev))
    got = summarize_pv_normalizer_diagnostics(m.faquant_pv_normalizer_diagnostics)
    d = OA.new_diagnostics()
    OA.simulated_flash_attention(q, k, v, OA.SimConfig(pv_normalizer_mode=mode), attention_mask=mask,
                                 dtype="bfloat16", diagnostics=d)
    ref = OA.summarize_diagnostics(d)
    print(f"[probe] {mode} masked={masked} got={got} ref={ref}", flush=True)
    assert got["rows"] == ref["rows"] and got["p_values"] == ref["p_values"]
    for key in ("mass_ratio_mean", "mass_ratio_min", "mass_ratio_max", "p_relative_l2"):
        assert got[key] == pytest.approx(ref[key], rel=2e-3), key
    assert got["mass_ratio_std"] == pytest.approx(ref["mass_ratio_std"], rel=2e-2)
    # P-hat codes may differ at rounding boundaries (exp2 vs exp): a handful of values
    assert abs(got["p_zero_collapse_rate"] - ref["p_zero_collapse_rate"]) * got["p_values"] <= 16
    assert np.abs(np.subtract(got["mass_ratio_histogram"], ref["mass_ratio_histogram"])).sum() <= 4
