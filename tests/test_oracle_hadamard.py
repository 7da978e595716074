"""Pins the numpy Hadamard oracle: golden vectors (bit-exact), closed forms, invariants."""

import numpy as np
import pytest

from oracle import hadamard
from oracle import hadamard as OH
from oracle import hif4 as OQ
from oracle.hif4 import bf16_round
from tests.conftest import load_golden


def test_matches_reference_golden_vectors(golden_hadamard):
    g = golden_hadamard
    x = g["x"]
    np.testing.assert_array_equal(hadamard.hadamard_transform(x), g["h128"])
    np.testing.assert_array_equal(hadamard.hadamard_transform(x.reshape(-1, 64)).reshape(64, 128), g["h64"])
    np.testing.assert_array_equal(hadamard.block_hadamard_transform(x, 64), g["blk64"])


def test_qwen_prologue_matches_reference(golden_hadamard):
    g = golden_hadamard
    np.testing.assert_array_equal(hadamard.qk_rotation(g["qwen_q"], out_round=bf16_round), g["qwen_q_h128"])
    np.testing.assert_array_equal(hadamard.qk_rotation(g["qwen_k"], out_round=bf16_round), g["qwen_k_h128"])
    np.testing.assert_array_equal(
        hadamard.qk_rotation(g["qwen_q"], block_size=64, out_round=bf16_round), g["qwen_q_blk64"]
    )
    np.testing.assert_array_equal(
        hadamard.qk_rotation(
            g["qwen_k"], smooth_scale=g["smooth_scale"], smooth_is_key=True, key_offset=g["key_offset"],
            out_round=bf16_round,
        ),
        g["qwen_k_offset_smooth_h128"],
    )
    np.testing.assert_array_equal(
        hadamard.qk_rotation(g["qwen_q"], smooth_scale=g["smooth_scale"], out_round=bf16_round),
        g["qwen_q_smooth_h128"],
    )


@pytest.mark.parametrize("n", [2, 8, 64, 128])
def test_sylvester_closed_form(n):
    """x @ H_n / sqrt(n) in float64 (the construction of tests/test_hisq_rotation.py:29-43)."""
    g = np.random.Generator(np.random.PCG64(n))
    x = g.standard_normal((16, n), dtype=np.float32)
    dense = (x.astype(np.float64) @ hadamard.sylvester_matrix(n)) / np.sqrt(n)
    np.testing.assert_allclose(hadamard.hadamard_transform(x), dense, rtol=0, atol=2e-6 * np.sqrt(n))


def test_orthogonal_and_self_inverse():
    g = np.random.Generator(np.random.PCG64(0))
    x = g.standard_normal((3, 16), dtype=np.float32)
    r = hadamard.hadamard_transform(x)
    np.testing.assert_allclose(hadamard.hadamard_transform(r), x, atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(x, axis=-1), atol=1e-5, rtol=1e-6)


def test_64_point_is_exact_dyadic():
    """n=64 divides by exactly 8: on small integers the transform is exact."""
    g = np.random.Generator(np.random.PCG64(1))
    x = g.integers(-8, 8, size=(8, 64)).astype(np.float32)
    exact = (x.astype(np.float64) @ hadamard.sylvester_matrix(64)) / 8.0
    np.testing.assert_array_equal(hadamard.hadamard_transform(x), exact.astype(np.float32))


def test_block_equals_full_for_one_block():
    g = np.random.Generator(np.random.PCG64(2))
    x = g.standard_normal((5, 128), dtype=np.float32)
    np.testing.assert_array_equal(hadamard.block_hadamard_transform(x, 128), hadamard.hadamard_transform(x))


def test_rejects_non_power_of_two():
    with pytest.raises(ValueError, match="power of two"):
        hadamard.hadamard_transform(np.zeros((1, 12), np.float32))
    with pytest.raises(ValueError, match="divisible"):
        hadamard.block_hadamard_transform(np.zeros((1, 96), np.float32), 64)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("n", [8, 64, 128, 512])
def test_stage_rounded_transform_matches_reference_goldens(dt, n):
    """hadamard_transform on a bf16 / fp16 tensor (rotation.py:14-29 in that dtype): every
    stage rounded, bitwise equal to the reference's output."""
    g = load_golden("hadamard_native.npz")
    rnd = OQ.bf16_round if dt == "bf16" else OQ.fp16_round
    got = OH.hadamard_transform(g[f"x_{dt}_{n}"], stage_round=rnd)
    assert np.array_equal(got.view(np.uint32), g[f"h_{dt}_{n}"].view(np.uint32))
    # and the per-stage rounding matters: one rounding at the end differs somewhere
    once = rnd(OH.hadamard_transform(g[f"x_{dt}_{n}"]))
    assert not np.array_equal(once, g[f"h_{dt}_{n}"])


def _from_bits(u, dt):
    if dt == "bf16":
        return (u.astype(np.uint32) << 16).view(np.float32)
    return u.view(np.float16).astype(np.float32)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
def test_in_dtype_transforms_match_reference_goldens(dt):
    """hadamard_transform above 512 and generalized_hadamard_transform (12 * 2^k) on bf16 /
    fp16 tensors, which the reference runs in the tensor's dtype (rotation.py:14-69: every
    butterfly stage and the 12 x 12 matmul rounded to it, then the division): the oracle's
    stage-rounded forms equal the reference's vectors bit for bit, and the fp32 forms do not
    (the vectors tell the two apart)."""
    from tests.conftest import load_golden

    g = load_golden("hadamard_native.npz")
    rnd = OQ.bf16_round if dt == "bf16" else OQ.fp16_round
    for kind in ("p", "g"):
        keys = sorted(k for k in g if k.startswith(f"{kind}x_{dt}_"))
        assert keys
        for k in keys:
            n = k.rsplit("_", 1)[1]
            x = _from_bits(g[k], dt)
            want = _from_bits(g[f"{kind}h_{dt}_{n}"], dt)
            fn = OH.hadamard_transform if kind == "p" else OH.generalized_hadamard_transform
            got = fn(x, stage_round=rnd)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), k
            assert not np.array_equal(rnd(fn(x)).view(np.uint32), want.view(np.uint32)), k
