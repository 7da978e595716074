"""The o_proj-input HiF4 QDQ fused into the attention epilogue (qwen3.py:167-171).

The reference quantizes the attention output after its cast to the query dtype, along
the hidden axis Hq * 128 in groups of 64 (each group is half of one head's row).  The
fused epilogue must equal that composition bitwise: the kernel's own plain output (cast to
the output dtype), then the oracle's fake_quantize_hif4 (the reference's hif4.py:377-390,
pinned by its known-answer vector and goldens) over [B, L, Hq * 128], and also the HIP row
quantizer on the same values.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import module, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _operands(dev, hq, hkv, lq, lk, seed):
    from faquant_amd import _ops

    g = OI.rng(seed)
    q = to_dev(OQ.bf16_round(g.standard_normal((1, hq, lq, 128), dtype=np.float32) * 2), dev, torch.bfloat16)
    k = to_dev(OQ.bf16_round(g.standard_normal((1, hkv, lk, 128), dtype=np.float32)), dev, torch.bfloat16)
    v = to_dev(OQ.bf16_round(g.standard_normal((1, hkv, lk, 128), dtype=np.float32) * 3), dev, torch.bfloat16)
    qh, _ = _ops.operand_prep(q, levels="123")
    kh, _ = _ops.operand_prep(k, levels="123")
    vt = _ops.operand_prep_vt(v, levels="123")
    return qh, kh, vt


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("levels", ["123", "12", "13"])
@pytest.mark.parametrize("shape", [(8, 2, 300, 300), (4, 4, 200, 70)], ids=["gqa", "rows_without_keys"])
def test_fused_output_qdq_equals_attention_then_row_quantizer(dev, out_dtype, levels, shape):
    from faquant_amd import _ops

    hq, hkv, lq, lk = shape
    qh, kh, vt = _operands(dev, hq, hkv, lq, lk, seed=41 + lq)
    kw = dict(causal=True, scale=128**-0.5, quant_p=True, p_levels="123", norm_same=True)
    plain = torch.empty((1, lq, hq, 128), device=dev, dtype=out_dtype)
    _ops.attention_fwd(qh, kh, vt, lk, out=plain.transpose(1, 2), **kw)
    fused = torch.empty_like(plain)
    _ops.attention_fwd(qh, kh, vt, lk, out=fused.transpose(1, 2), out_levels=levels, **kw)
    rows = plain.reshape(1, lq, hq * 128)
    dt = "bfloat16" if out_dtype == torch.bfloat16 else "float32"
    oracle = OQ.fake_quantize_hif4(rows.float().cpu().numpy(), levels, dtype=dt).reshape(plain.shape)
    print(f"[epilogue] {shape} {levels} {out_dtype}", flush=True)
    got = fused.float().cpu().numpy()
    assert np.array_equal(got, oracle)
    # and the HIP row quantizer on the same values
    assert torch.equal(fused, _ops.qdq_rows(rows, levels).view(plain.shape))
    assert not torch.equal(fused, plain)


def test_attention_core_output_quant_equals_reference_composition(dev):
    from faquant_amd.qwen3 import attention_core
    from faquant_amd.quantization import fake_quantize

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in OI.qwen(42, 8, 2, 300))
    kwargs = {"quant_format": "hif4", "bits": 4, "group_size": 64, "symmetric": True, "clip_ratio": 1.0}

    def mk(out_quant):
        m = module()
        m.faquant_qk_rotation = True
        m.faquant_qk_rotation_block_size = 64
        m.faquant_attention_output_quant = out_quant
        m.faquant_core_quant_kwargs = kwargs
        return m

    fused = attention_core(mk(True), q, k, v)
    plain = attention_core(mk(False), q, k, v)
    expected = fake_quantize(plain.reshape(1, 300, -1), **kwargs).view(plain.shape)
    assert torch.equal(fused, expected)
    # o_proj quantizing its own input switches the boundary QDQ off (qwen3.py:168-170)
    m = mk(True)
    m.o_proj = type("P", (), {"faquant_quantizes_input": True})()
    assert torch.equal(attention_core(m, q, k, v), plain)
