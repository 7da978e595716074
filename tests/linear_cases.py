"""Cases of the quantized Linear's activation path: the reference-written fixtures of
tests/golden/linear_act.npz turned into the oracle's arguments."""

from __future__ import annotations

import numpy as np
import torch

from tests.conftest import load_golden

GOLDEN = "linear_act.npz"


def compand_scale(log_scale: np.ndarray, cols: int, dtype: str) -> np.ndarray:
    """``log_scale`` expanded to ``cols`` features, clamped to [-2.079, 2.079], exp'd and cast
    to ``dtype`` with torch on the CPU, as the reference computes it (quantization.py:222-234);
    float32 values of ``dtype``.  The last bit of torch's CPU exp depends on the host's vector
    unit, so tests that compare with a fixture use the scale stored in it."""
    ls = torch.from_numpy(np.asarray(log_scale, np.float32))
    if ls.numel() != cols:
        ls = ls.repeat_interleave(cols // ls.numel())
    return ls.clamp(-2.079, 2.079).exp().to(getattr(torch, dtype)).float().numpy()


def golden_cases() -> dict[str, dict]:
    """case -> {"x", "y", "dtype", "levels", "kw"}; "kw" are the oracle's keyword arguments
    (``oracle.linear.fake_quant_linear_input``)."""
    g = load_golden(GOLDEN)
    names = sorted({k.split("__")[0] for k in g if "__" in k and not k.startswith("gen")})
    out = {}
    for name in names:
        def get(key, default=None):
            return g.get(f"{name}__{key}", default)

        dtype = str(get("dtype"))
        x = get("x")
        kw: dict = {}
        if get("input_scale") is not None:
            kw["input_scale"] = get("input_scale")
        if get("input_rotation_signs") is not None:
            kw["rot_signs"] = get("input_rotation_signs")
            kw["rot_perm"] = get("input_rotation_permutation")
            kw["rot_block"] = int(get("input_rotation_block_size")) or None
        if get("activation_min") is not None:
            kw["act_min"] = float(get("activation_min"))
        if get("activation_max") is not None:
            kw["act_max"] = float(get("activation_max"))
        if get("activation_compand_log_scale") is not None:
            # the scale the reference multiplied by (exp's last bit depends on the CPU)
            kw["compand"] = get("compand_scale")
        online = int(get("online"))
        kw["hadamard"] = max(online, 0)
        if online < 0:
            kw["hadamard_generalized"] = True
        out[name] = {"x": x, "y": get("y"), "dtype": dtype, "levels": str(g["levels"]), "kw": kw}
    return out


def generalized_vectors() -> dict[int, tuple]:
    """n -> (x, y) of the reference's generalized_hadamard_transform on fp32 rows."""
    g = load_golden(GOLDEN)
    sizes = sorted({int(k[3:].split("__")[0]) for k in g if k.startswith("gen")})
    return {n: (g[f"gen{n}__x"], g[f"gen{n}__y"]) for n in sizes}
