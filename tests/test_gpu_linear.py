"""HiF4 W4A4 Linear: the fused activation prologue and the Linear drop-ins.

The activation path of FakeQuantLinear.forward (quantization.py:204-276) is
x * dtype(input_scale) in the input dtype, the per-block fp32 Hadamard
(rotation.py:117-135, true division by sqrt(n)) cast back to the input dtype, then
fake_quantize (HiF4, ACT levels) in that dtype.  The oracle restates each step
(pinned against the reference's codec and Hadamard goldens), so the fused kernel is
compared with it bit for bit; the Linear drop-ins are compared with the reference's
composition of those steps and F.linear.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hadamard as OH
from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _round(x, dtype):
    return OQ.bf16_round(x) if dtype == torch.bfloat16 else np.asarray(x, np.float32)


def _oracle_act(x, dtype, *, scale=None, hadamard=0, levels="123"):
    name = "bfloat16" if dtype == torch.bfloat16 else "float32"
    v = np.asarray(x, np.float32)
    if scale is not None:
        v = _round(v * _round(scale, dtype), dtype)
    if hadamard:
        v = _round(OH.block_hadamard_transform(v, hadamard), dtype)
    return OQ.fake_quantize_hif4(v, levels, dtype=name) if levels else v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("hadamard", [0, 64, 128, 512])
@pytest.mark.parametrize("levels", ["123", "12", "13"])
def test_act_prologue_matches_oracle_bitwise(dev, dtype, hadamard, levels):
    from faquant_amd import _ops

    g = OI.rng(hadamard + int(levels))
    x = _round(g.standard_normal((37, 1024), dtype=np.float32) * np.exp(g.standard_normal((1, 1024))), dtype)
    x[3, 100:140] = 0.0  # zero groups
    scale = g.uniform(0.25, 4.0, size=(1024,)).astype(np.float32)
    for sc in (None, scale):
        got = _ops.act_qdq_rows(to_dev(x, dev, dtype), levels=levels, hadamard=hadamard,
                                col_scale=None if sc is None else to_dev(sc, dev))
        ref = _oracle_act(x, dtype, scale=sc, hadamard=hadamard, levels=levels)
        print(f"[act] {dtype} hadamard={hadamard} levels={levels} scale={sc is not None}", flush=True)
        assert np.array_equal(got.float().cpu().numpy(), ref)


def test_act_prologue_partial_group_and_leading_shape(dev):
    from faquant_amd import _ops

    g = OI.rng(7)
    x = OQ.bf16_round(g.standard_normal((2, 3, 200), dtype=np.float32))
    got = _ops.act_qdq_rows(to_dev(x, dev, torch.bfloat16), levels="123")
    assert got.shape == (2, 3, 200)
    assert np.array_equal(got.float().cpu().numpy(), OQ.fake_quantize_hif4(x, "123", dtype="bfloat16"))


@pytest.mark.parametrize("block", [None, 64])
def test_fake_quant_linear_equals_reference_composition(dev, block):
    from faquant_amd import _ops
    from faquant_amd.hif4 import HIF4_ACT_SCALE_LEVELS, HIF4_SCALE_LEVELS
    from faquant_amd.quantization import FakeQuantLinear, fake_quantize

    g = OI.rng(8)
    lin = torch.nn.Linear(256, 192, bias=True).to(dev, torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_dev(g.standard_normal((192, 256)) * 0.05, dev, torch.bfloat16))
    scale = to_dev(g.uniform(0.5, 2.0, size=(256,)), dev)
    mod = FakeQuantLinear(lin, quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64,
                          symmetric=True, clip_ratio=1.0, online_hadamard=block is not None,
                          online_hadamard_block_size=block, input_scale=scale)
    w_ref = OQ.fake_quantize_hif4(lin.weight.detach().float().cpu().numpy(), HIF4_SCALE_LEVELS, dtype="bfloat16")
    assert np.array_equal(mod.weight.float().cpu().numpy(), w_ref)
    x = to_dev(g.standard_normal((4, 33, 256)), dev, torch.bfloat16)
    # the reference's steps (quantization.py:204-276) with this library's standalone ops
    ref_x = x * scale.to(torch.bfloat16)
    if block is not None:
        ref_x = _ops.hadamard_rows(ref_x.float(), block, out_dtype=torch.bfloat16)
    ref_x = fake_quantize(ref_x, quant_format="hif4", bits=4, group_size=64)
    expected = torch.nn.functional.linear(ref_x, mod.weight, mod.bias)
    got = mod(x)
    assert torch.equal(got, expected)
    assert HIF4_ACT_SCALE_LEVELS in ("123", "12", "13")


def test_fake_quant_linear_unsupported_options_raise(dev):
    from faquant_amd.quantization import FakeQuantLinear

    lin = torch.nn.Linear(64, 64).to(dev)
    common = dict(quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64, symmetric=True,
                  clip_ratio=1.0)
    with pytest.raises(NotImplementedError):
        FakeQuantLinear(lin, **common, activation_min=-1.0)
    with pytest.raises(NotImplementedError):
        FakeQuantLinear(lin, **common, online_hadamard=True)
    with pytest.raises(ValueError):
        FakeQuantLinear(lin, **{**common, "weight_group_size": 32})


def test_hif4_linear_equals_quantize_then_linear(dev):
    from faquant_amd.hif4 import fake_quantize_hif4
    from faquant_amd.wan22_hif4 import HiF4Linear, faquant_qdq

    g = OI.rng(9)
    lin = torch.nn.Linear(320, 128, bias=True).to(dev, torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_dev(g.standard_normal((128, 320)) * 0.05, dev, torch.bfloat16))
    qdq = faquant_qdq("123")
    mod = HiF4Linear(lin, weight_qdq=qdq, input_qdq=qdq, device=dev, chunk_elements=320 * 64)
    w = fake_quantize_hif4(lin.weight.detach().float(), levels="123").to(torch.bfloat16)
    assert torch.equal(mod.weight, w)
    np.testing.assert_array_equal(mod.weight.float().cpu().numpy(),
                                  OQ.fake_quantize_hif4(lin.weight.detach().float().cpu().numpy(), "123"))
    seen = []
    mod.collector = lambda m, rows, start: seen.append((rows.clone(), start))
    x = to_dev(g.standard_normal((3, 50, 320)), dev, torch.float32)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = mod(x)
        want = torch.nn.functional.linear(fake_quantize_hif4(x.reshape(-1, 320), levels="123"), mod.weight, mod.bias)
    assert got.shape == (3, 50, 128)
    assert torch.equal(got.reshape(-1, 128), want)
    # the collector sees every quantized input row once, bit-exact with the oracle's QDQ
    assert len(seen) == 1 and seen[0][1] == 0
    np.testing.assert_array_equal(seen[0][0].cpu().numpy(), OQ.fake_quantize_hif4(x.reshape(-1, 320).cpu().numpy(), "123"))
    # and the product is the fp32 product of the HiF4 operands within bf16 GEMM rounding
    ref = seen[0][0].double() @ mod.weight.double().T + mod.bias.double()
    assert float((got.reshape(-1, 128).double() - ref).abs().max() / ref.abs().max()) < 1e-2
    with pytest.raises(RuntimeError, match="exactly representable"):
        HiF4Linear(lin, weight_qdq=lambda w: w * 1.001, input_qdq=qdq, device=dev)
    with pytest.raises(ValueError, match="HiF4 weight of shape"):
        HiF4Linear(lin, weight_qdq=qdq, input_qdq=qdq, device=dev, weight=torch.zeros(3, 3))
