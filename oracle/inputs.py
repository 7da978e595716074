"""Seeded synthetic inputs for the benchmark configurations (numpy PCG64, version-stable).

Distributions follow the configuration list of the north-star metric:
  1  fp32 Q/K/V ~ N(0,1), four fixed outlier channels scaled x10.
  2  Qwen3-8B: bf16 N(0,1) Q/K/V, RoPE (theta 1e6, rotate-half) applied to Q/K.
  3  Qwen3-32B: bf16 Gaussian Q/V, Student-t (df=3) K channels, RoPE.
  4  Wan2.2 480p: bf16 N(0,1).
  5  Wan2.2 720p: bf16 N(0,1) scaled per head by U[0.5, 4].
Values are drawn in float32 and rounded once to bf16 (round to nearest even).
"""

from __future__ import annotations

import numpy as np

from .hif4 import bf16_round

SALT = 0x5EED_F4A7
_F32 = np.float32


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SALT + seed))


def rope(x: np.ndarray, positions: np.ndarray, theta: float = 1.0e6) -> np.ndarray:
    """HF rotate-half RoPE over the last axis, float32 math (cos/sin in float32)."""
    d = x.shape[-1]
    inv = (1.0 / (theta ** (np.arange(0, d, 2, dtype=np.float64) / d))).astype(_F32)
    ang = positions.astype(_F32)[:, None] * inv[None, :]
    emb = np.concatenate([ang, ang], axis=-1)
    cos, sin = np.cos(emb).astype(_F32), np.sin(emb).astype(_F32)
    half = d // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return (x * cos + rot * sin).astype(_F32)


def outlier_channels(d: int, count: int = 4, seed: int = 1) -> np.ndarray:
    return np.sort(rng(seed).choice(d, size=count, replace=False))


def config1(seed: int = 1, heads: int = 8, length: int = 512, dim: int = 128):
    """CPU plumbing case: fp32 [1, H, L, D] Q/K/V with 4 outlier channels x10."""
    g = rng(seed)
    ch = outlier_channels(dim, 4, seed)
    out = []
    for _ in range(3):
        t = g.standard_normal((1, heads, length, dim), dtype=_F32)
        t[..., ch] *= _F32(10.0)
        out.append(t)
    return tuple(out)


def qwen(seed: int, hq: int, hkv: int, length: int, dim: int = 128, student_t_keys: bool = False):
    """bf16-valued [1, H, L, D] Q/K/V with RoPE on Q/K (Qwen3 layout before transpose)."""
    g = rng(seed)
    q = g.standard_normal((1, hq, length, dim), dtype=_F32)
    if student_t_keys:
        k = g.standard_t(3.0, size=(1, hkv, length, dim)).astype(_F32)
    else:
        k = g.standard_normal((1, hkv, length, dim), dtype=_F32)
    v = g.standard_normal((1, hkv, length, dim), dtype=_F32)
    pos = np.arange(length)
    q = rope(bf16_round(q), pos)
    k = rope(bf16_round(k), pos)
    return bf16_round(q), bf16_round(k), bf16_round(v)


def wan(seed: int, heads: int, length: int, dim: int = 128, head_scale: bool = False):
    """bf16-valued Wan layout [1, L, H, D] Q/K/V."""
    g = rng(seed)
    out = []
    scale = g.uniform(0.5, 4.0, size=(heads,)).astype(_F32) if head_scale else None
    for _ in range(3):
        t = g.standard_normal((1, length, heads, dim), dtype=_F32)
        if scale is not None:
            t = t * scale[None, None, :, None]
        out.append(bf16_round(t))
    return tuple(out)
