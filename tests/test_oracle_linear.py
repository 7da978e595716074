"""Pins the numpy oracle of the quantized Linear's activation path (oracle/linear.py):
bit-exact against the reference's FakeQuantLinear on its fixtures, then closed forms."""

import numpy as np
import pytest

from oracle import hadamard as OH
from oracle import hif4 as OQ
from oracle import linear as OL
from tests.linear_cases import generalized_vectors, golden_cases

CASES = golden_cases()


@pytest.mark.parametrize("name", sorted(CASES))
def test_matches_reference_fake_quant_linear(name):
    c = CASES[name]
    got = OL.fake_quant_linear_input(c["x"], c["dtype"], levels=c["levels"], **c["kw"])
    np.testing.assert_array_equal(got, c["y"])


def test_fixtures_cover_every_step():
    keys = set()
    for c in CASES.values():
        keys |= {k for k, v in c["kw"].items() if v is not None and not (np.isscalar(v) and v == 0)}
        if c["kw"].get("rot_signs") is not None:
            keys.add("rot_block" if c["kw"]["rot_block"] else "rot_no_block")
    assert {"input_scale", "rot_signs", "rot_block", "rot_no_block", "act_min", "act_max", "compand", "hadamard",
            "hadamard_generalized"} <= keys
    assert {c["dtype"] for c in CASES.values()} == {"bfloat16", "float16", "float32"}


def _rng_rows(rows, cols, seed=5):
    g = np.random.default_rng(seed)
    return (g.standard_normal((rows, cols)) * g.uniform(0.1, 3, (rows, 1))).astype(np.float32)


def test_rotation_is_orthogonal_in_fp32():
    x = _rng_rows(6, 512)
    g = np.random.default_rng(1)
    signs = g.choice(np.array([-1, 1], np.int8), 512)
    perm = g.permutation(512)
    for block in (None, 64, 512):
        y = OL.fake_quant_linear_input(x, "float32", levels=None, rot_signs=signs, rot_perm=perm, rot_block=block)
        np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=2e-6)
    # without a block the rotation is a signed permutation: exact
    y = OL.fake_quant_linear_input(x, "float32", levels=None, rot_signs=signs, rot_perm=perm, rot_block=None)
    np.testing.assert_array_equal(y, (x * signs)[:, perm])
    # the block Hadamard applied twice is the identity up to rounding
    z = OL.fake_quant_linear_input(y, "float32", levels=None, rot_signs=np.ones(512, np.int8),
                                   rot_perm=np.arange(512), rot_block=64)
    z = OH.block_hadamard_transform(z, 64)
    np.testing.assert_allclose(z, y, atol=1e-5 * np.abs(y).max())


def test_identity_rotation_and_no_quantizer_keep_the_input():
    x = OQ.bf16_round(_rng_rows(3, 256))
    y = OL.fake_quant_linear_input(x, "bfloat16", levels=None, rot_signs=np.ones(256, np.int8),
                                   rot_perm=np.arange(256), rot_block=None)
    np.testing.assert_array_equal(y, x)


def test_clamp_keeps_nan_and_rounds_bounds_to_the_dtype():
    x = np.array([[np.nan, -5.0, 0.30078125, 0.298828125, 7.0] + [0.0] * 59], np.float32)
    y = OL.fake_quant_linear_input(x, "bfloat16", levels=None, act_min=0.3001, act_max=2.0)
    assert np.isnan(y[0, 0])
    # bf16(0.3001) = 0.30078125; values below it are lifted to it
    np.testing.assert_array_equal(y[0, 1:5], np.array([0.30078125, 0.30078125, 0.30078125, 2.0], np.float32))
    # min above max gives max, as torch.clamp does
    y = OL.fake_quant_linear_input(x, "float32", levels=None, act_min=3.0, act_max=1.0)
    np.testing.assert_array_equal(y[0, 1:], np.ones(63, np.float32))


def test_companding_round_trip_without_quantizer():
    # scale by 2^k and divide back: exact in every dtype
    x = OQ.bf16_round(_rng_rows(2, 128))
    c = np.exp2(np.random.default_rng(3).integers(-3, 4, 128)).astype(np.float32)
    y = OL.fake_quant_linear_input(x, "bfloat16", levels=None, compand=c)
    np.testing.assert_array_equal(y, x)


@pytest.mark.parametrize("n", sorted(generalized_vectors()))
def test_generalized_hadamard_matches_reference(n):
    x, y = generalized_vectors()[n]
    np.testing.assert_array_equal(OH.generalized_hadamard_transform(x), y)


def test_generalized_hadamard_closed_form():
    """(H12 kron H_b) x / sqrt(12 b) in float64, orthogonal: H12 H12^T = 12 I."""
    h12 = OH.hadamard12().astype(np.float64)
    np.testing.assert_array_equal(h12 @ h12.T, 12 * np.eye(12))
    g = np.random.default_rng(4)
    for b in (1, 2, 16, 64):
        n = 12 * b
        x = g.standard_normal((3, n)).astype(np.float32)
        dense = np.kron(h12, OH.sylvester_matrix(b)) / np.sqrt(n)
        want = x.astype(np.float64) @ dense.T
        got = OH.generalized_hadamard_transform(x)
        np.testing.assert_allclose(got, want, rtol=0, atol=2e-6 * np.abs(want).max())
        np.testing.assert_allclose(np.linalg.norm(got, axis=1), np.linalg.norm(x, axis=1), rtol=2e-6)
    with pytest.raises(ValueError, match="unsupported generalized Hadamard dimension"):
        OH.generalized_hadamard_transform(np.zeros((1, 36), np.float32))
