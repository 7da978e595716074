"""HiF4 level selection from the environment (hif4.py:13-43), read at import.

Each case imports ``faquant_amd.hif4`` in a fresh interpreter with the variables set and
checks the resulting tables: the scale / act / attention fallback chain, the per-operand
override list, and the ValueError for invalid values.  No GPU is needed (the library is
loaded lazily).
"""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

from tests.conftest import PKG_ROOT, REPO

PROBE = (
    "import json, faquant_amd.hif4 as H; print(json.dumps([H.HIF4_SCALE_LEVELS, H.HIF4_ACT_SCALE_LEVELS, "
    "H.HIF4_ATTN_SCALE_LEVELS, H.HIF4_ATTN_OPERAND_SCALE_LEVELS]))"
)


def _import_with(env_extra: dict) -> subprocess.CompletedProcess:
    env = {k: v for k, v in os.environ.items() if not k.startswith("FAQUANT_HIF4_")}
    env.update(env_extra)
    env["PYTHONPATH"] = os.pathsep.join([PKG_ROOT, REPO])
    return subprocess.run([sys.executable, "-c", PROBE], env=env, capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize(
    "env,expect",
    [
        ({}, ["123", "123", "123", dict.fromkeys("qkpv", "123")]),
        ({"FAQUANT_HIF4_SCALE_LEVELS": "12"}, ["12", "12", "12", dict.fromkeys("qkpv", "12")]),
        ({"FAQUANT_HIF4_ACT_SCALE_LEVELS": "13"}, ["123", "13", "13", dict.fromkeys("qkpv", "13")]),
        ({"FAQUANT_HIF4_SCALE_LEVELS": "12", "FAQUANT_HIF4_ATTN_SCALE_LEVELS": "123"},
         ["12", "12", "123", dict.fromkeys("qkpv", "123")]),
        ({"FAQUANT_HIF4_ATTN_SCALE_LEVELS": "12", "FAQUANT_HIF4_ATTN_OPERAND_LEVELS": "p=123,v=13"},
         ["123", "123", "12", {"q": "12", "k": "12", "p": "123", "v": "13"}]),
        ({"FAQUANT_HIF4_ATTN_OPERAND_LEVELS": "q=12,,k=13"},  # empty entries are skipped
         ["123", "123", "123", {"q": "12", "k": "13", "p": "123", "v": "123"}]),
    ],
)
def test_level_tables(env, expect):
    r = _import_with(env)
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout.strip().splitlines()[-1]) == expect


@pytest.mark.parametrize(
    "env,message",
    [
        ({"FAQUANT_HIF4_SCALE_LEVELS": "23"}, "FAQUANT_HIF4_SCALE_LEVELS must be 123, 12 or 13"),
        ({"FAQUANT_HIF4_ACT_SCALE_LEVELS": "1"}, "FAQUANT_HIF4_ACT_SCALE_LEVELS must be 123, 12 or 13"),
        ({"FAQUANT_HIF4_ATTN_SCALE_LEVELS": ""}, "FAQUANT_HIF4_ATTN_SCALE_LEVELS must be 123, 12 or 13"),
        ({"FAQUANT_HIF4_ATTN_OPERAND_LEVELS": "o=12"}, "entries must be q|k|p|v=123|12|13"),
        ({"FAQUANT_HIF4_ATTN_OPERAND_LEVELS": "p=14"}, "entries must be q|k|p|v=123|12|13"),
    ],
)
def test_invalid_levels_raise_value_error(env, message):
    r = _import_with(env)
    assert r.returncode != 0
    assert "ValueError" in r.stderr and message in r.stderr
