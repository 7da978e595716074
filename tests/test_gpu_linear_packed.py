"""The packed-weight HiF4 Linear (faq_hif4_linear_packed, ``linear_packed``, FakeQuantLinear
with ``packed_weight=True``).

FakeQuantLinear.forward (quantization.py:199-277) is F.linear on the activation QDQ and the
weight QDQ.  Here the weight stays packed (4.5 bits per weight) and the kernel decodes it
in registers, so:
- the packed weight decodes to the oracle's weight QDQ (fake_quantize_hif4, hif4.py:377-390)
  bitwise, for levels 123 / 12 / 13, bf16 and fp32 weights, zero rows and a NaN group;
- y equals the exact product of the same operands (float64) within fp32 summation error,
  for 1..8 rows, ragged N, 1..96 blocks of K (one and several passes of 32), bias or none,
  fp32 and bf16 outputs; bf16 outputs differ from F.linear's by at most one bf16 ulp;
- repeated calls give the same bits (fixed summation order); more than 8 rows are refused;
- FakeQuantLinear(packed_weight=True) decodes to its own ``weight`` and takes the packed
  contraction for at most ``packed_max_rows`` rows, F.linear beyond.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import to_dev
from tests.test_gpu_decode_kernel import unpack_rows

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _weight(g, N, K, scale=0.05):
    w = g.standard_normal((N, K)) * scale * np.exp(g.standard_normal((N, 1)) * 0.5)
    w[g.integers(0, N, 7), g.integers(0, K, 7)] *= 40.0  # outliers
    return w


def _decoded(pw):
    N, K = pw.shape
    rows = pw.rows
    vals = unpack_rows(rows.codes[0, 0].cpu().numpy(), rows.meta[0, 0].cpu().numpy())
    return vals.reshape(N, K)


@pytest.mark.filterwarnings("ignore::RuntimeWarning")  # the NaN group's oracle exponents
@pytest.mark.parametrize("levels", ["123", "12", "13"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_packed_weight_decodes_to_the_weight_qdq(dev, levels, dtype):
    from faquant_amd import _ops

    g = OI.rng(int(levels) + (7 if dtype == torch.float32 else 0))
    w = _weight(g, 96, 384)
    w[5] = 0.0
    w[9, 64:128] = np.nan  # a NaN group: its 64 values decode to NaN
    wt = to_dev(w, dev, dtype)
    pw = _ops.PackedHiF4Weight(wt, levels)
    print(f"[lin pack] levels {levels} {dtype}", flush=True)
    want = OQ.fake_quantize_hif4(wt.float().cpu().numpy(), levels, dtype="bfloat16" if dtype == torch.bfloat16 else "float32")
    got = _decoded(pw)
    assert np.array_equal(got, want, equal_nan=True)
    assert np.isnan(got[9, 64:128]).all() and not np.isnan(got[9, :64]).any()
    assert pw.nbytes() == 96 * 384 * 9 // 16  # 4.5 bits per weight


def _within_one_bf16_ulp(a: "torch.Tensor", b: "torch.Tensor") -> bool:
    """|a - b| <= one bf16 ulp of max(|a|, |b|) (bf16: 8 significant bits)."""
    af, bf = a.float(), b.float()
    big = torch.maximum(af.abs(), bf.abs())
    ulp = torch.where(big > 0, torch.exp2(torch.floor(torch.log2(big)) - 7), torch.zeros_like(big))
    return bool(((af - bf).abs() <= ulp).all())


def _exact(x, w, b):
    return x.astype(np.float64) @ w.astype(np.float64).T + (0.0 if b is None else b.astype(np.float64))


def _check_close(y, exact, x, w, b, what):
    """fp32 sums: |y - exact| within 1e-5 of the sum of |x w| terms (the typical error is far
    below; a dropped or repeated block is off by about 1/nkb of it)."""
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T + (0.0 if b is None else np.abs(b))
    err = np.abs(y.astype(np.float64) - exact)
    assert np.all(err <= 1e-5 * mag + 1e-30), (what, float((err / (mag + 1e-30)).max()))


CASES = [
    # M, N, K, bias, out dtype
    (1, 4096, 4096, None, "bf16"),        # a Qwen3-8B q_proj decode step (two features per wave)
    (3, 1000, 384, "bf16", "fp32"),       # ragged N; 3 of 64 lane pairs' blocks per row
    (8, 256, 1280, "fp32", "bf16"),       # eight rows of x
    (5, 4100, 512, None, "fp32"),         # N not a multiple of the features per wave
    (2, 96, 128, "bf16", "bf16"),         # one block of K per row
    (4, 12288, 4096, None, "bf16"),       # gate/up_proj: four features per wave
    (1, 4096, 12288, "fp32", "fp32"),     # down_proj: three passes of 32 blocks per row
    (7, 40, 4224, "bf16", "bf16"),        # 33 blocks: the second pass holds one block
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "M{}N{}K{}_{}_{}".format(*c))
def test_linear_packed_matches_the_exact_product(dev, case):
    from faquant_amd import _ops

    M, N, K, bias, out = case
    g = OI.rng(M * 7 + N + K)
    w = OQ.bf16_round(_weight(g, N, K))
    x = OQ.bf16_round(g.standard_normal((M, K)) * 2.0)
    b = None if bias is None else OQ.bf16_round(g.standard_normal(N))
    wq = OQ.fake_quantize_hif4(w, "123", dtype="bfloat16")
    pw = _ops.PackedHiF4Weight(to_dev(w, dev, torch.bfloat16), "123")
    bt = None if b is None else to_dev(b, dev, torch.bfloat16 if bias == "bf16" else torch.float32)
    odt = torch.bfloat16 if out == "bf16" else torch.float32
    print(f"[lin] {case}", flush=True)
    xt = to_dev(x, dev, torch.bfloat16)
    y = _ops.linear_packed(xt, pw, bt, out_dtype=odt)
    assert y.shape == (M, N) and y.dtype == odt
    exact = _exact(x, wq, b)
    yf = y.float().cpu().numpy()
    if out == "fp32":
        _check_close(yf, exact, x, wq, b, case)
    else:
        # one rounding of the fp32 sum to bf16: within a bf16 ulp of the exact value
        ulp = np.abs(exact).astype(np.float32).view(np.uint32) & 0x7F800000
        ulp = (ulp.view(np.float32).astype(np.float64)) * 2.0 ** -7
        mag = np.abs(x.astype(np.float64)) @ np.abs(wq.astype(np.float64)).T
        assert np.all(np.abs(yf - exact) <= ulp + 1e-5 * mag + 1e-30), case
        # against F.linear on the same bf16 operands: at most one bf16 ulp apart
        ref = torch.nn.functional.linear(xt, to_dev(wq, dev, torch.bfloat16), bt.to(torch.bfloat16) if bt is not None else None)
        assert _within_one_bf16_ulp(y, ref), case
    # the same bits on a second call
    y2 = _ops.linear_packed(xt, pw, bt, out_dtype=odt)
    assert torch.equal(y.view(torch.int16) if odt == torch.bfloat16 else y.view(torch.int32),
                       y2.view(torch.int16) if odt == torch.bfloat16 else y2.view(torch.int32))


@pytest.mark.parametrize("M", [1, 3, 8])
def test_features_per_wave_do_not_change_the_bits(dev, M, monkeypatch):
    """One, two or four output features per wave (FAQ_LIN_RPW test hook): each feature's sum
    runs in the same order whichever wave owns it, so the outputs are equal bitwise."""
    from faquant_amd import _ops

    g = OI.rng(40 + M)
    N, K = 1030, 1664
    w = OQ.bf16_round(_weight(g, N, K))
    pw = _ops.PackedHiF4Weight(to_dev(w, dev, torch.bfloat16), "123")
    x = to_dev(OQ.bf16_round(g.standard_normal((M, K))), dev, torch.bfloat16)
    b = to_dev(g.standard_normal(N), dev, torch.float32)
    outs = []
    for rpw in ("1", "2", "4"):
        monkeypatch.setenv("FAQ_LIN_RPW", rpw)
        print(f"[lin rpw] M={M} rpw={rpw}", flush=True)
        outs.append(_ops.linear_packed(x, pw, b, out_dtype=torch.float32))
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    assert torch.equal(outs[0].view(torch.int32), outs[2].view(torch.int32))


def test_linear_packed_row_limit(dev):
    from faquant_amd import _ops

    pw = _ops.PackedHiF4Weight(torch.zeros((64, 256), device=dev, dtype=torch.bfloat16), "123")
    assert _ops.linear_packed(torch.zeros((0, 256), device=dev, dtype=torch.bfloat16), pw).shape == (0, 64)
    with pytest.raises(NotImplementedError, match="at most 8 rows"):
        _ops.linear_packed(torch.zeros((9, 256), device=dev, dtype=torch.bfloat16), pw)


def test_linear_packed_leading_shape_strides_and_nan(dev):
    from faquant_amd import _ops

    g = OI.rng(3)
    N, K = 512, 1024
    w = OQ.bf16_round(_weight(g, N, K))
    w[7, 128:192] = np.nan
    pw = _ops.PackedHiF4Weight(to_dev(w, dev, torch.bfloat16), "123")
    x = to_dev(OQ.bf16_round(g.standard_normal((2, 3, K))), dev, torch.bfloat16)
    y = _ops.linear_packed(x, pw)
    assert y.shape == (2, 3, N)
    assert torch.isnan(y[..., 7]).all() and not torch.isnan(y[..., :7]).any()
    # a strided view of rows gives the rows' results
    xs = torch.empty((6, K + 64), device=dev, dtype=torch.bfloat16)
    xs[:, :K] = x.reshape(6, K)
    ys = _ops.linear_packed(xs[:, :K], pw)
    assert torch.equal(ys.view(torch.int16), y.reshape(6, N).view(torch.int16))
    # a view that starts 2 bytes past 16-byte alignment is copied, not refused
    flat = torch.empty(6 * K + 1, device=dev, dtype=torch.bfloat16)
    flat[1:].copy_(x.reshape(-1))
    yo = _ops.linear_packed(flat[1:].view(6, K), pw)
    assert torch.equal(yo.view(torch.int16), y.reshape(6, N).view(torch.int16))


def test_fake_quant_linear_packed_weight(dev):
    from faquant_amd import _ops
    from faquant_amd.hif4 import HIF4_SCALE_LEVELS
    from faquant_amd.quantization import FakeQuantLinear

    g = OI.rng(11)
    lin = torch.nn.Linear(512, 384, bias=True).to(dev, torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_dev(_weight(g, 384, 512), dev, torch.bfloat16))
    common = dict(quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64, symmetric=True,
                  clip_ratio=1.0, online_hadamard=True, online_hadamard_block_size=128)
    plain = FakeQuantLinear(lin, **common)
    packed = FakeQuantLinear(lin, **common, packed_weight=True, packed_max_rows=8)
    assert torch.equal(packed.weight, plain.weight)
    assert np.array_equal(_decoded(packed._packed), packed.weight.float().cpu().numpy())
    assert packed._packed.levels == HIF4_SCALE_LEVELS
    for rows in (1, 8, 9):
        x = to_dev(g.standard_normal((rows, 512)), dev, torch.bfloat16)
        y_plain, y_packed = plain(x), packed(x)
        print(f"[lin module] rows {rows}", flush=True)
        if rows <= 8:
            assert _within_one_bf16_ulp(y_plain, y_packed)  # packed contraction: another fp32 order
            xq = _ops.act_qdq_rows(x, levels="123", hadamard=128)
            assert torch.equal(y_packed, _ops.linear_packed(xq, packed._packed, packed.bias))
        else:
            assert torch.equal(y_plain, y_packed)  # beyond packed_max_rows: F.linear
    with pytest.raises(ValueError, match="quantize_weight"):
        FakeQuantLinear(lin, **common, packed_weight=True, quantize_weight=False)
