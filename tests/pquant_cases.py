"""Inputs for the P-quantizer parity tests: 64-value groups of non-negative P values placed
on and around the rounding thresholds of the reference's code rule.

The reference codes a value as floor(fp32(fp32(|x| qm) 4) + 0.5) (hif4.py:266-270): two
roundings, with ties rounding up and u = 0.5 - 2^-25 giving code 1.  A single rounding of
the exact product with ties to even differs from it at u = n + 0.5 and where the exact
product lies within half an ulp below n + 0.5.  ``tie_groups`` builds groups whose 4-value
groups have chosen maxima (so every micro exponent k occurs) and whose other values are the
floats nearest to (n + 0.5) / (4 qm) and a few ulps either side, for random n in 0..7.
"""

from __future__ import annotations

import numpy as np

from oracle import hif4 as OQ

F32 = np.float32


def tie_groups(levels: str, seed: int, ngroups: int = 400) -> np.ndarray:
    rng = np.random.default_rng(seed)
    out = []
    for gi in range(ngroups):
        e = int(rng.integers(-20, 3))
        m1 = F32(np.ldexp(1.0 + rng.integers(0, 256) / 256.0, e))
        if gi % 3 == 0:
            m1 = F32(np.ldexp(1.0, e))  # scales whose reciprocal is a power of two: exact ties
        g = np.zeros(64, F32)
        g[0] = m1
        for j in range(1, 16):  # each 4-group's maximum sits at its first element
            g[4 * j] = F32(m1 * rng.choice([1.0, 0.6, 0.3, 0.2, 0.1, 0.05]))
        meta = OQ.fit_compact(g[None], levels)
        rec = meta["reciprocal"].reshape(())
        k = meta["lv2"].reshape(8).repeat(2).astype(F32) + meta["lv3"].reshape(16).astype(F32)
        K = np.exp2(k).astype(F32)
        for j in range(16):
            qm4 = F32(F32(rec / K[j]) * F32(4.0))
            m3 = g[4 * j]
            for t in range(1, 4):
                n = int(rng.integers(0, 8))
                p = F32((n + 0.5) / float(qm4))
                d = int(rng.integers(-3, 4))
                for _ in range(abs(d)):
                    p = np.nextafter(p, F32(np.inf) if d > 0 else F32(0.0))
                if p > m3:  # keep the 4-group's maximum (and so its micro exponent)
                    p = F32(m3 * rng.random())
                g[4 * j + t] = p
        out.append(g)
    return np.stack(out)


def softmax_groups(seed: int, ngroups: int = 2000, spread: float = 3.0) -> np.ndarray:
    """exp(s - max s) of Gaussian scores: the value distribution P has in attention."""
    rng = np.random.default_rng(seed)
    s = (rng.standard_normal((ngroups, 64)) * spread).astype(F32)
    return np.exp((s - s.max(axis=1, keepdims=True)).astype(F32)).astype(F32)


def single_rounding_codes(p: np.ndarray, levels: str) -> np.ndarray:
    """Dequantized values under rint-to-even of the exact product p 4 rec / K (one rounding):
    the rule the reference does NOT use; the tests check the tie groups separate the two."""
    p = np.asarray(p, F32).reshape(-1, 64)
    meta = OQ.fit_compact(p, levels)
    rec = meta["reciprocal"].reshape(-1, 1).astype(np.float64)
    s = meta["scale"].reshape(-1, 1).astype(np.float64)
    k = (np.repeat(meta["lv2"].reshape(-1, 8), 8, axis=1) + np.repeat(meta["lv3"].reshape(-1, 16), 4, axis=1))
    K = np.exp2(k.astype(np.float64))
    c = np.minimum(np.rint(p.astype(np.float64) * 4.0 * rec / K), 7.0)
    return (c * K * s / 4.0).astype(F32)
