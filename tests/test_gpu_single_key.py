"""Rows that see exactly one key, bitwise against the oracle.

The reference scales the scores, takes the row maximum and then exp(scores - maximum)
(sfa:725-727, 788-797), so the only key of a row gets P = exp(0) = 1 exactly and the row's
output is fixed by the quantizers alone: V^ under quantized_same (P^ V^ / P^), HiF4(1) V^
under the unquantized normalizer, V with quantization off.  The kernel forms its exponent
argument as RN(RN(s c1) - m) outside quantized_same (P = 1 exactly, as the reference) and as
one fma inside it (where a single key's output is V^ whatever P is), so every case here must
equal the oracle bit for bit: a sliding window of 1 through the one-pass kernel (with and
without a 2-D padding mask), and one cached key through the decode kernel.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA
from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import module, to_dev
from tests.test_gpu_masks import make_mask

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

MODES = [("quantized_same", True), ("unquantized", True), ("quantized_same", False)]


def _qkv(seed, B, hq, hkv, lq, lk):
    g = OI.rng(seed)
    q = OQ.bf16_round(g.standard_normal((B, hq, lq, 128), dtype=np.float32) * 3)
    k = OQ.bf16_round(g.standard_normal((B, hkv, lk, 128), dtype=np.float32) * 3)
    v = OQ.bf16_round(g.standard_normal((B, hkv, lk, 128), dtype=np.float32))
    return q, k, v


@pytest.mark.parametrize("mode,quant", MODES, ids=lambda x: str(x))
@pytest.mark.parametrize("masked", [False, True])
def test_window_one_rows_are_bitwise_the_oracle(dev, mode, quant, masked):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    B, hq, hkv, L = 2, 4, 2, 300
    print(f"[single-key] window 1 mode={mode} quant={quant} masked={masked}", flush=True)
    q, k, v = _qkv(71, B, hq, hkv, L, L)
    mask = make_mask("holes", B, L, seed=5) if masked else None
    mod = module(mode=mode, qk=quant, pv=quant)
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    out, _ = simulated_flash_attention_forward(mod, qt, kt, vt, None if mask is None else torch.from_numpy(mask).to(dev),
                                               sliding_window=1)
    cfg = OA.SimConfig(pv_normalizer_mode=mode, qk_quant=quant, pv_quant=quant, is_causal=True)
    ref = OA.simulated_flash_attention(q, k, v, cfg, attention_mask=mask, sliding_window=1, dtype="bfloat16")
    got = out.float().cpu().numpy()
    diff = int(np.sum(got != ref))
    print(f"[single-key] {diff} of {got.size} outputs differ", flush=True)
    assert diff == 0


@pytest.mark.parametrize("mode,quant", MODES, ids=lambda x: str(x))
def test_decode_over_one_cached_key_is_bitwise_the_oracle(dev, mode, quant):
    from faquant_amd import _ops

    B, hq, hkv = 2, 8, 2
    print(f"[single-key] decode Lk=1 mode={mode} quant={quant}", flush=True)
    q, k, v = _qkv(72, B, hq, hkv, 1, 1)
    lv = "123" if quant else None
    qt, kt, vt = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    qh, _ = _ops.operand_prep(qt, levels=lv)
    kh, _ = _ops.operand_prep(kt, levels=lv)
    vh, _ = _ops.operand_prep(vt, levels=lv)
    out = torch.empty((B, 1, hq, 128), device=dev, dtype=torch.bfloat16)
    _ops.attention_decode(qh, 1, k=kh, v=vh, causal=True, scale=128 ** -0.5, quant_p=quant, p_levels="123",
                          norm_same=mode == "quantized_same", out=out.transpose(1, 2))
    cfg = OA.SimConfig(pv_normalizer_mode=mode, qk_quant=quant, pv_quant=quant, is_causal=True)
    ref = OA.simulated_flash_attention(q, k, v, cfg, dtype="bfloat16")
    got = out.float().cpu().numpy()
    diff = int(np.sum(got != ref))
    print(f"[single-key] {diff} of {got.size} outputs differ", flush=True)
    assert diff == 0
