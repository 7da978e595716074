"""Seeded random configurations through the drop-in, against the oracle.

Each case draws a shape and a feature mix the fixed tests combine less often: batch 1-3,
GQA ratios 1/2/4/8, Lq below and above Lk (bottom-right alignment, queries without keys),
causal or not, 2-D padding masks (left, right, holes), sliding windows, the logit softcap
and both PV normalizer modes.  The output must meet the attention tolerance against the
oracle and the stats counters must be equal.  The draws are fixed by the seed.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from tests.test_gpu_attention import assert_close_attention, module, to_dev
from tests.test_gpu_masks import _qkv, make_mask

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _draw(n, seed=2026):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B = int(rng.integers(1, 4))
        hkv = int(rng.integers(1, 3))
        G = int(rng.choice([1, 2, 4, 8]))
        lk = int(rng.integers(1, 500))
        lq = int(rng.integers(1, lk + 1)) if rng.random() < 0.8 else int(rng.integers(lk, lk + 200))
        causal = bool(rng.random() < 0.7)
        kind = str(rng.choice(["none", "left", "right", "holes"]))
        window = None if rng.random() < 0.6 else int(rng.integers(1, 300))
        mode = str(rng.choice(["quantized_same", "unquantized"]))
        softcap = None if rng.random() < 0.75 else 2.0
        cases.append((i, B, hkv * G, hkv, lq, lk, causal, kind, window, mode, softcap))
    return cases


@pytest.mark.parametrize("case", _draw(24), ids=lambda c: f"c{c[0]}_B{c[1]}_h{c[2]}x{c[3]}_{c[4]}x{c[5]}")
def test_random_configuration_matches_oracle(dev, case):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    i, B, hq, hkv, lq, lk, causal, kind, window, mode, softcap = case
    print(f"[random] {case}", flush=True)
    q, k, v = _qkv(i + 100, B, hq, hkv, lq, lk)
    mask = None if kind == "none" else make_mask(kind, B, lk, seed=i)
    mod = module(mode=mode, causal=causal)
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    out, _ = simulated_flash_attention_forward(mod, qt, kt, vt, None if mask is None else torch.from_numpy(mask).to(dev),
                                               sliding_window=window, softcap=softcap)
    stats = OA.new_stats()
    ref = OA.simulated_flash_attention(q, k, v, OA.SimConfig(pv_normalizer_mode=mode, is_causal=causal),
                                       attention_mask=mask, sliding_window=window, softcap=softcap, dtype="bfloat16",
                                       stats=stats)
    assert_close_attention(out.float().cpu().numpy(), ref, str(case))
    assert mod.faquant_simulated_attention_stats == stats
