"""The logit softcap (sfa:725-727) needs tanh inside the attention kernel, which uses
its own branch-free form (a polynomial below 0.625, 1 - 2 / (exp(2x) + 1) above).
tests/tanh_check.c restates it on the host, with the hardware exp2 / reciprocal moved by
one ulp either way, and bounds its error against tanh in double by 3 ulp (sampled here;
run the checker with stride 1 for every fp32 value in [0, 12])."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_kernel_tanh_is_within_three_ulp(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path / "tanh_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", os.path.join(HERE, "tanh_check.c"), "-o", exe, "-lm"],
                   check=True)
    out = subprocess.run([exe, "997"], capture_output=True, text=True, timeout=300)
    print(out.stdout.strip())
    assert out.returncode == 0, out.stdout
