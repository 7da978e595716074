"""Pins the numpy HiF4 oracle before it is trusted as the checker of the HIP kernels.

Pins used (each chosen so that a plausible slip fails at least one):
  * the reference's own known-answer vector (tests/test_quantization.py:51-74);
  * golden vectors written by the reference for levels 123/12/13 (tests/golden);
  * an exhaustive E6M2 closed form over every positive finite bf16 block maximum;
  * block locality and tail padding (tests/test_quantization.py:77-85);
  * packed encode/decode round trip and the level-exponent definitions.
"""

import numpy as np
import pytest

from oracle import hif4

KAT = [
    -17.5, -17.5, -15.0, -15.0, -15.0, -15.0, -15.0, -12.5,
    -12.5, -12.5, -12.5, -12.5, -10.0, -10.0, -10.0, -10.0,
    -8.75, -8.75, -7.5, -7.5, -6.25, -6.25, -6.25, -5.0,
    -4.375, -4.375, -3.75, -3.125, -2.5, -1.875, -1.875, -1.25,
    -0.625, -0.0, 0.625, 1.25, 1.25, 1.875, 2.5, 3.125,
    3.75, 3.75, 5.0, 5.0, 6.25, 6.25, 6.25, 7.5,
    7.5, 8.75, 8.75, 8.75, 10.0, 10.0, 10.0, 12.5,
    12.5, 12.5, 12.5, 12.5, 15.0, 15.0, 15.0, 15.0,
    15.0, 17.5, 17.5, 17.5, 17.5, 17.5,
]


def kat_input():
    """The reference test's input: torch.linspace(-17.25, 18.75, 70) in float32."""
    torch = pytest.importorskip("torch")
    return torch.linspace(-17.25, 18.75, 70, dtype=torch.float32).numpy()


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_known_answer_vector(dtype):
    x = kat_input()
    if dtype == "bfloat16":
        x = hif4.bf16_round(x)
    expected = np.array(KAT, dtype=np.float32)
    if dtype == "bfloat16":
        expected[2] = -17.5
    got = hif4.fake_quantize(x, quant_format="hif4", bits=4, group_size=64, dtype=dtype)
    np.testing.assert_array_equal(got, expected)
    # the sign of zero follows torch.sign(x) * 0: index 33 is a small negative -> -0.0
    assert np.signbit(got[33])


@pytest.mark.parametrize("levels", ["123", "12", "13"])
def test_matches_reference_golden_vectors(golden_codec, levels):
    g = golden_codec
    np.testing.assert_array_equal(
        hif4.fake_quantize_hif4(g["x"], levels).view(np.uint32), g[f"y_{levels}"].view(np.uint32)
    )
    np.testing.assert_array_equal(
        hif4.fake_quantize_hif4(g["x_bf16"], levels, "bfloat16").view(np.uint32),
        g[f"yb_{levels}"].view(np.uint32),
    )
    for w in (70, 100):
        np.testing.assert_array_equal(
            hif4.fake_quantize_hif4(g[f"tail{w}"], levels).view(np.uint32),
            g[f"ytail{w}_{levels}"].view(np.uint32),
        )
    p = hif4.fit_compact(g["x"].reshape(-1, 64), levels)
    np.testing.assert_array_equal(p["scale"].reshape(-1), g[f"scale_{levels}"])
    np.testing.assert_array_equal(p["reciprocal"].reshape(-1), g[f"rec_{levels}"])
    np.testing.assert_array_equal(p["lv2"].reshape(-1, 8), g[f"lv2_{levels}"])
    np.testing.assert_array_equal(p["lv3"].reshape(-1, 16), g[f"lv3_{levels}"])


def _e6m2_closed_form(maximum: np.ndarray, divisor: float):
    """Independent statement: s0 = bf16(max * bf16(1/div)) clamped; E6M2 = nearest of
    {2^e (1 + m/4)} with ties to even m, computed with exact rationals in float64."""
    r = float(hif4.bf16_round(np.array([np.float32(1.0) / np.float32(divisor)]))[0])
    s0 = hif4.bf16_round((maximum.astype(np.float32) * np.float32(r)).astype(np.float32)).astype(np.float64)
    s0 = np.clip(s0, 2.0**-48, 49152.0)
    e = np.floor(np.log2(s0))
    t = s0 / 2.0**e * 4.0  # in [4, 8), exact in float64
    lo = np.floor(t)
    frac = t - lo
    up = (frac > 0.5) | ((frac == 0.5) & (lo % 2 == 1))
    q = (lo + up) * 2.0 ** (e - 2)
    rec = hif4.bf16_round((1.0 / q).astype(np.float32))  # 1/q is exact enough: q has 3 bits
    return q.astype(np.float32), rec


@pytest.mark.parametrize("levels,divisor", [("123", 7.0), ("12", 3.5)])
def test_e6m2_scale_exhaustive_over_bf16_maxima(levels, divisor):
    bits = np.arange(0x0000, 0x7F80, dtype=np.uint32) << 16  # every positive finite bf16
    maxima = bits.view(np.float32)
    s, rec = hif4.e6m2_scale(maxima, levels)
    s2, rec2 = _e6m2_closed_form(maxima, divisor)
    np.testing.assert_array_equal(s, s2)
    # 1/q in float64 rounded to float32 equals the correctly rounded fp32 division
    np.testing.assert_array_equal(rec, rec2)
    # every scale is an 8-bit E6M2 value: e in [-48, 15], two mantissa bits
    sb = s.view(np.uint32)
    assert np.all(sb & 0x1FFFFF == 0)
    e = ((sb >> 23) & 0xFF).astype(np.int64) - 127
    assert e.min() >= -48 and e.max() <= 15


def test_e6m2_reciprocal_table():
    """rec = bf16(fp32(1 / (1 + m/4))) * 2^-e: the four-entry table the HIP kernels use."""
    table = [1.0, 0.80078125, 0.66796875, 0.5703125]
    for m in range(4):
        s = np.float32(1.0 + m / 4.0)
        assert hif4.bf16_round(np.array([np.float32(1.0) / s]))[0] == np.float32(table[m])


def test_blocks_are_local_and_tail_is_padded():
    g = np.random.Generator(np.random.PCG64(3))
    x = g.standard_normal((2, 70), dtype=np.float32)
    expected = hif4.fake_quantize_hif4(x)
    changed = x.copy()
    changed[:, 64:] *= 1000
    actual = hif4.fake_quantize_hif4(changed)
    np.testing.assert_array_equal(actual[:, :64], expected[:, :64])
    assert np.isfinite(actual).all()
    # zero padding: quantizing [x, 0...] to 128 equals quantizing x then padding
    padded = np.concatenate([x, np.zeros((2, 58), np.float32)], axis=-1)
    np.testing.assert_array_equal(hif4.fake_quantize_hif4(padded)[:, :70], expected)


def test_special_blocks():
    z = np.zeros((1, 64), np.float32)
    np.testing.assert_array_equal(hif4.fake_quantize_hif4(z), z)
    p = hif4.fit_compact(z)
    assert p["scale"].item() == 2.0**-48
    # all-equal block: max/7 -> bf16 -> E6M2, value v reproduced exactly when v = 7 s
    v = np.full((1, 64), 7.0, np.float32)
    y = hif4.fake_quantize_hif4(v)
    assert np.all(y == 7.0)
    # a huge block saturates at the 49152 scale clamp: 1.75 * 49152 * 4
    h = np.full((1, 64), 1e30, np.float32)
    assert np.all(hif4.fake_quantize_hif4(h) == np.float32(1.75 * 49152 * 4))


@pytest.mark.parametrize("levels", ["123", "12", "13"])
def test_encode_decode_round_trip(golden_codec, levels):
    x = golden_codec["x"]
    packed = hif4.encode(x, levels)
    assert packed["codes"].max() <= 15
    np.testing.assert_array_equal(hif4.decode(packed).view(np.uint32), hif4.fake_quantize_hif4(x, levels).view(np.uint32))
    if levels == "12":
        assert np.all(packed["lv3_bits"] == 0)
    if levels == "13":
        assert np.all(packed["lv2_bits"] == 0)


def test_relative_error_matches_published_gaussian_figures():
    """QWEN3_32B.md:124-126 reports HiF4 relative squared error on Gaussian data of
    0.00689 / 0.00894 / 0.00702 for levels 123 / 12 / 13 (sample size unstated)."""
    g = np.random.Generator(np.random.PCG64(5))
    x = g.standard_normal((4096, 128), dtype=np.float32)
    for levels, published in (("123", 0.00689), ("12", 0.00894), ("13", 0.00702)):
        y = hif4.fake_quantize_hif4(x, levels)
        rse = float(((y - x) ** 2).sum() / (x**2).sum())
        assert abs(rse - published) / published < 0.03, (levels, rse)


def test_int_format_matches_reference_semantics():
    # tests/test_quantization.py:16-25: group-local int4
    x = np.array([[0.0, 1.0, -2.0, 3.0, 100.0, -50.0, 1.0, 2.0]], np.float32)
    q = hif4.fake_quantize(x, bits=4, group_size=4)
    ch = x.copy()
    ch[0, 4] = 1000
    np.testing.assert_array_equal(hif4.fake_quantize(ch, bits=4, group_size=4)[:, :4], q[:, :4])
    with pytest.raises(ValueError, match="divisible"):
        hif4.fake_quantize(np.zeros((2, 7), np.float32), group_size=4)


def test_dispatcher_errors():
    x = np.zeros((1, 64), np.float32)
    with pytest.raises(ValueError, match="bits=4"):
        hif4.fake_quantize(x, quant_format="hif4", bits=8, group_size=64)
    with pytest.raises(ValueError, match="group_size=64"):
        hif4.fake_quantize(x, quant_format="hif4", group_size=32)
    with pytest.raises(ValueError, match="asymmetric"):
        hif4.fake_quantize(x, quant_format="hif4", group_size=64, symmetric=False)
    with pytest.raises(ValueError, match="clipping"):
        hif4.fake_quantize(x, quant_format="hif4", group_size=64, clip_ratio=0.9)


def test_int_format_known_answers():
    """Closed-form values of the int branch (quantization.py:74-94): scales that are powers
    of two keep every step exact, so the expected outputs follow from the rule alone --
    round half to even (torch.round), the signed range [-2^(b-1), 2^(b-1) - 1], the clip
    ratio applied to the maximum before the scale, the asymmetric zero point and range, the
    eps floor of the scale, and bits >= 16 as the identity."""
    q = lambda x, **kw: hif4.fake_quantize(np.array([x], np.float32), **kw)[0]  # noqa: E731
    # symmetric int4, max 7: scale 1, ties to even, -7 in range
    np.testing.assert_array_equal(q([0.5, 1.5, 2.5, -7.0], bits=4, group_size=4), [0.0, 2.0, 2.0, -7.0])
    # clip ratio 0.5 of max 14: scale 1, 14 clamps to 7 and -10 to -8 (qmin = -8)
    np.testing.assert_array_equal(q([14.0, -10.0, 1.5, 0.25], bits=4, group_size=4, clip_ratio=0.5),
                                  [7.0, -8.0, 2.0, 0.0])
    # symmetric int8 with max 127 * 2^-3: scale 2^-3
    np.testing.assert_array_equal(q([127 / 8, -1.0, 0.0625, 0.1875], bits=8, group_size=4),
                                  [127 / 8, -1.0, 0.0, 0.25])
    # asymmetric int2 over [-1, 2]: scale 1, zero point 1, codes 0..3
    np.testing.assert_array_equal(q([-1.0, 0.0, 1.0, 2.0], bits=2, group_size=4, symmetric=False), [-1.0, 0.0, 1.0, 2.0])
    # asymmetric int2, all non-negative (the range is widened to include 0): scale 1, zero 0
    np.testing.assert_array_equal(q([3.0, 0.5, 1.5, 3.0], bits=2, group_size=4, symmetric=False), [3.0, 0.0, 2.0, 3.0])
    # an all-zero group: the scale floors at fp32 eps and the group stays zero
    np.testing.assert_array_equal(q([0.0, 0.0, 0.0, 0.0], bits=4, group_size=4), [0.0, 0.0, 0.0, 0.0])
    # groups are independent; group_size -1 is the whole row
    np.testing.assert_array_equal(q([7.0, 1.0, 0.5, 3.5], bits=4, group_size=2), [7.0, 1.0, 0.5, 3.5])
    np.testing.assert_array_equal(q([7.0, 1.0, 0.5, 3.5], bits=4, group_size=-1), [7.0, 1.0, 0.0, 4.0])
    # bits >= 16: unchanged
    np.testing.assert_array_equal(q([0.1, -0.3, 7.7, 1e-9], bits=16, group_size=4), np.float32([0.1, -0.3, 7.7, 1e-9]))
