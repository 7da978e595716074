"""The companding quotient of the quantized Linear's activation path (quantization.py:268,
x / compand_scale in the activation dtype) as a product with the column's fp32 reciprocal.

The activation kernel computes T(fp32(x * r)) with r = fp32(1 / c) once per column, in place
of T(fp32(x / c)), for bf16 columns whose scale is a normal number and fp16 columns with
|c| < 8 (the reference's scales are exp(clamp(log_scale, -2.079, 2.079)) in (0.125, 8)); every
other column, and fp32 activations, divide.  tests/compand_div_check.c proves the identity
over every pair of 16-bit values (2^32 pairs per dtype, a few seconds on 8 cores) and fails
on any mismatch where the kernel takes the product; here it runs exhaustively, its fp16
rounding is compared with numpy's cast, and numpy restates the identity on its own (the
product form holds on a sample of the rule's domain and fails for fp16 scales of 14, so the
C check is not vacuous)."""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import numpy as np
import pytest

from oracle import hif4 as OQ

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path_factory.mktemp("cdiv") / "compand_div_check")
    flags = ["-O2", "-ffp-contract=off"]
    probe = subprocess.run(["gcc", "-fopenmp", "-x", "c", "-", "-o", os.devnull], input="int main(){return 0;}",
                           capture_output=True, text=True)
    if probe.returncode == 0:
        flags.append("-fopenmp")
    subprocess.run(["gcc", *flags, os.path.join(HERE, "compand_div_check.c"), "-o", exe, "-lm"], check=True)
    return exe


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_product_quotient_is_exact_where_the_kernel_takes_it(checker, dtype):
    out = subprocess.run([checker, dtype, "exhaustive"], capture_output=True, text=True, timeout=900)
    print(out.stdout.strip())
    assert out.returncode == 0, out.stdout
    m = re.search(r"mismatches (\d+) over (\d+) scales; (\d+) scales take the product, mismatches there (\d+)",
                  out.stdout)
    assert m is not None
    total, _, taken, there = (int(g) for g in m.groups())
    assert there == 0
    # most scales take the product, and the check does find the pairs where it differs
    assert taken > (60000 if dtype == "bf16" else 36000)
    assert total > 0


def test_fp16_rounding_of_the_checker_is_numpys(checker):
    g = np.random.default_rng(3)
    x = np.concatenate([
        g.standard_normal(1 << 18).astype(np.float32) * np.float32(2.0) ** g.integers(-30, 18, 1 << 18).astype(np.float32),
        np.float32([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, np.inf, -np.inf, 2.0 ** -14, 2.0 ** -24,
                    2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]),
    ]).astype(np.float32)
    got = subprocess.run([checker, "conv16"], input=x.tobytes(), capture_output=True, timeout=60).stdout
    got = np.frombuffer(got, np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert got.shape == want.shape
    assert np.array_equal(got, want)


def _q(x, c, rnd):
    with np.errstate(all="ignore"):
        return rnd(x / c), rnd(x * (np.float32(1.0) / c))


def _same(a, b):
    return np.array_equal(a, b) or bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


def test_numpy_restatement_agrees():
    g = np.random.default_rng(4)
    bf16_x = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    bf16_c = OQ.bf16_round(np.exp(g.uniform(-2.079, 2.079, 96)).astype(np.float32))
    for c in bf16_c:
        a, b = _q(bf16_x, np.float32(c), OQ.bf16_round)
        assert _same(a, b), c
    f16_x = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    f16_c = np.exp(g.uniform(-2.079, 2.079, 96)).astype(np.float16).astype(np.float32)
    to16 = lambda v: v.astype(np.float16).astype(np.float32)  # noqa: E731
    for c in f16_c:
        a, b = _q(f16_x, np.float32(c), to16)
        assert _same(a, b), c
    # outside the rule: fp16 scale 14 has pairs where the product form differs
    a, b = _q(f16_x, np.float32(14.0), to16)
    assert not _same(a, b)
