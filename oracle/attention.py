"""numpy restatement of the reference's tiled HiF4 flash-attention simulator (test oracle).

Follows ``src/faquant/simulated_flash_attention.py`` ("sfa"):
  * argument validation                        sfa:479-529
  * normalizer mode and causal flag            sfa:530-559
  * all-valid 2-D mask normalization           sfa:561-586
  * ``_two_dimensional_mask``                  sfa:341-368
  * ``_streaming_mask``                        sfa:371-427
  * ``_apply_four_dimensional_mask``           sfa:430-454
  * K/V QDQ before GQA repeat, Q QDQ           sfa:588-619 (``_fake_quantize_tail`` 292-338)
  * ``_repeat_kv``                             sfa:231-240
  * tiled online softmax, fully-future skip    sfa:623-884
  * query-tile schedule and output layout      sfa:886-909
  * stats counters                             sfa:18-33, 187-211, 901-908
  * PV-normalizer diagnostics                  sfa:36-185, 835-869
and ``quantized_eager_attention_forward`` (qad_attention.py:112-226), the
single-tile closed form used as an independent cross-check.

All state is float32 as in the reference.  Matmuls are float32 GEMMs, whose
summation order differs from torch's, so the output agrees with the reference
to float32 rounding, not bit for bit; quantized operands and tile-local P
quantization follow the reference exactly given the same scores.

Parity pins (tests/test_oracle_attention.py): the dense closed forms and
invariants of tests/test_simulated_flash_attention.py and
tests/test_qad_attention.py:84-117, and golden outputs written by the
reference for HiF4 Q/K/P/V at the configured shapes (tests/golden).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import hif4

_F32 = np.float32
PV_NORMALIZER_MODES = ("unquantized", "quantized_same")
PV_MASS_RATIO_BIN_EDGES = (0.5, 0.7, 0.8, 0.9, 0.95, 0.99, 1.0, 1.01, 1.05, 1.1, 1.3)
OPERANDS = ("q", "k", "p", "v")


def new_stats() -> dict[str, int]:
    stats = {"calls": 0, "qk_tiles": 0, "pv_tiles": 0, "qk_quantized_tiles": 0, "pv_quantized_tiles": 0}
    for op in OPERANDS:
        stats[f"{op}_quant_calls"] = 0
        stats[f"{op}_quantized_values"] = 0
        stats[f"{op}_quant_blocks"] = 0
        stats[f"{op}_quant_padding_values"] = 0
    return stats


def new_diagnostics() -> dict[str, object]:
    d: dict[str, object] = dict.fromkeys(
        (
            "rows",
            "mass_ratio_sum",
            "mass_ratio_sq_sum",
            "p_values",
            "p_zeroed_values",
            "p_error_sq_sum",
            "p_reference_sq_sum",
        ),
        0.0,
    )
    d["mass_ratio_min"] = float("inf")
    d["mass_ratio_max"] = float("-inf")
    d["mass_ratio_histogram"] = [0.0] * (len(PV_MASS_RATIO_BIN_EDGES) + 1)
    return d


def _record(stats, op, width, numel, group_size, repeats):
    g = width if group_size == -1 else group_size
    groups = math.ceil(width / g)
    vectors = numel // width
    stats[f"{op}_quant_calls"] += repeats
    stats[f"{op}_quantized_values"] += numel * repeats
    stats[f"{op}_quant_blocks"] += vectors * groups * repeats
    stats[f"{op}_quant_padding_values"] += vectors * (groups * g - width) * repeats


@dataclass
class QuantSpec:
    """``faquant_*_matmul_quant_kwargs`` of the reference module."""

    quant_format: str = "hif4"
    bits: int = 4
    group_size: int = 64
    symmetric: bool = True
    clip_ratio: float = 1.0

    def kwargs(self) -> dict:
        return dict(
            quant_format=self.quant_format,
            bits=self.bits,
            group_size=self.group_size,
            symmetric=self.symmetric,
            clip_ratio=self.clip_ratio,
        )


@dataclass
class SimConfig:
    """The module attributes ``simulated_flash_attention_forward`` reads (sfa:530-559)."""

    query_chunk: int = 256
    key_chunk: int = 128
    qk_quant: bool = True
    pv_quant: bool = True
    qk_spec: QuantSpec = field(default_factory=QuantSpec)
    pv_spec: QuantSpec = field(default_factory=QuantSpec)
    levels: dict = field(default_factory=lambda: dict.fromkeys(OPERANDS, "123"))
    pv_normalizer_mode: str = "unquantized"
    skip_fully_masked_tiles: bool = True
    is_causal: bool = True


def fake_quantize_tail(t: np.ndarray, spec: QuantSpec, levels: str, dtype: str) -> np.ndarray:
    """``_fake_quantize_tail`` (sfa:292-338): pad a short last group, QDQ, slice."""
    kw = spec.kwargs()
    g = spec.group_size
    if g == -1 or t.shape[-1] % g == 0:
        return hif4.fake_quantize(t, hif4_levels=levels, dtype=dtype, **kw)
    pad = g - t.shape[-1] % g
    padded = np.concatenate([t, np.zeros((*t.shape[:-1], pad), dtype=_F32)], axis=-1)
    return hif4.fake_quantize(padded, hif4_levels=levels, dtype=dtype, **kw)[..., : t.shape[-1]]


def repeat_kv(x: np.ndarray, repeats: int) -> np.ndarray:
    """Contiguous GQA mapping: query head h reads KV head h // repeats (sfa:231-240)."""
    return x if repeats == 1 else np.repeat(x, repeats, axis=1)


def _two_dimensional_mask(mask, query_length, key_length):
    if mask.shape[-1] < key_length:
        raise ValueError("2-D attention mask is shorter than the simulated key sequence")
    key_valid = mask[:, -key_length:].astype(bool)
    if query_length > key_valid.shape[-1]:
        missing = query_length - key_valid.shape[-1]
        query_valid = np.concatenate([np.zeros((key_valid.shape[0], missing), bool), key_valid], axis=-1)
    else:
        query_valid = key_valid[:, -query_length:]
    return query_valid, key_valid


def streaming_mask(
    *, batch, q0, q1, k0, k1, query_length, key_length, is_causal, sliding_window, query_valid, key_valid
) -> np.ndarray:
    """Boolean allowed mask [B, 1, q1-q0, k1-k0] (sfa:371-427)."""
    qp = np.arange(q0, q1)
    kp = np.arange(k0, k1)
    allowed = np.ones((batch, 1, q1 - q0, k1 - k0), dtype=bool)
    if query_valid is None or key_valid is None:
        anchors = qp + key_length - query_length
        if is_causal:
            allowed &= kp[None, :] <= anchors[:, None]
        if sliding_window is not None:
            allowed &= kp[None, :] > anchors[:, None] - sliding_window
            if not is_causal:
                allowed &= kp[None, :] < anchors[:, None] + sliding_window
        return allowed
    key_ranks = np.cumsum(key_valid.astype(np.int64), axis=-1) - 1
    query_ranks = np.cumsum(query_valid.astype(np.int64), axis=-1) - 1
    key_counts = key_valid.sum(axis=-1, keepdims=True)
    query_counts = query_valid.sum(axis=-1, keepdims=True)
    anchors = query_ranks[:, q0:q1] + key_counts - query_counts
    tk = key_ranks[:, k0:k1]
    allowed &= query_valid[:, None, q0:q1, None]
    allowed &= key_valid[:, None, None, k0:k1]
    if is_causal:
        allowed &= tk[:, None, None, :] <= anchors[:, None, :, None]
    if sliding_window is not None:
        allowed &= tk[:, None, None, :] > anchors[:, None, :, None] - sliding_window
        if not is_causal:
            allowed &= tk[:, None, None, :] < anchors[:, None, :, None] + sliding_window
    return allowed


def _four_dimensional_mask(scores, mask, q0, q1, k0, k1, query_length):
    mq = mask.shape[-2]
    if mq == 1:
        qs = slice(0, 1)
    elif mq >= query_length:
        off = mq - query_length
        qs = slice(off + q0, off + q1)
    else:
        raise ValueError("4-D attention mask is shorter than the query sequence")
    m = mask[..., qs, k0:k1]
    if m.dtype == bool or not np.issubdtype(m.dtype, np.floating):
        return np.where(m.astype(bool), scores, -np.inf).astype(_F32)
    finfo_min = np.finfo(m.dtype).min
    invalid = np.isneginf(m) | (m <= finfo_min / 2)
    return np.where(invalid, -np.inf, scores + m.astype(_F32)).astype(_F32)


def simulated_flash_attention(
    query: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    cfg: SimConfig,
    *,
    attention_mask: np.ndarray | None = None,
    scaling: float | None = None,
    sliding_window: int | None = None,
    softcap: float | None = None,
    is_causal: bool | None = None,
    dtype: str = "float32",
    stats: dict | None = None,
    diagnostics: dict | None = None,
) -> np.ndarray:
    """Restatement of ``simulated_flash_attention_forward``; returns [B, Lq, Hq, D] float32.

    ``query``/``key``/``value`` are float32 arrays holding ``dtype`` values
    ("float32", "bfloat16" or "float16"); the output is rounded to ``dtype`` (sfa:871-884,
    ``.to(query.dtype)``).
    """
    query = np.asarray(query, dtype=_F32)
    key = np.asarray(key, dtype=_F32)
    value = np.asarray(value, dtype=_F32)
    if softcap is not None and softcap < 0:
        raise ValueError("softcap must be non-negative")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError("sliding_window must be positive")
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("simulated FlashAttention expects rank-4 Q/K/V tensors")
    if key.shape != value.shape:
        raise ValueError("simulated FlashAttention requires matching K/V shapes")
    if query.shape[0] != key.shape[0] or query.shape[-1] != key.shape[-1]:
        raise ValueError("simulated FlashAttention received incompatible Q/K shapes")
    if attention_mask is not None and attention_mask.shape[-1] < key.shape[-2]:
        key = key[:, :, : attention_mask.shape[-1]]
        value = value[:, :, : attention_mask.shape[-1]]
    B, Hq, Lq, D = query.shape
    _, Hkv, Lk, _ = key.shape
    if Hq % Hkv:
        raise ValueError("query heads must be divisible by key/value heads")
    if min(query.shape) == 0 or Lk == 0:
        raise ValueError("simulated FlashAttention does not support zero dimensions")
    if cfg.pv_normalizer_mode not in PV_NORMALIZER_MODES:
        raise ValueError(f"unsupported pv_normalizer_mode {cfg.pv_normalizer_mode!r}")
    reps = Hq // Hkv
    scale = _F32(scaling if scaling is not None else D**-0.5)
    causal = cfg.is_causal if is_causal is None else bool(is_causal)
    same = cfg.pv_normalizer_mode == "quantized_same"
    stats = new_stats() if stats is None else stats
    collect = cfg.pv_quant and diagnostics is not None

    query_valid = key_valid = None
    mask = attention_mask
    if mask is not None and mask.ndim == 2:
        all_valid = cfg.skip_fully_masked_tiles and B == 1 and Lq > 1 and bool(np.all(mask[:, -Lk:]))
        if all_valid:
            mask = None
        else:
            query_valid, key_valid = _two_dimensional_mask(mask, Lq, Lk)
    elif mask is not None and mask.ndim not in (3, 4):
        raise ValueError("attention mask must be rank 2, 3, or 4")
    if mask is not None and mask.ndim == 3:
        mask = mask[:, None]

    lv = cfg.levels
    k_op = fake_quantize_tail(key, cfg.qk_spec, lv["k"], dtype) if cfg.qk_quant else key
    v_op = fake_quantize_tail(value, cfg.pv_spec, lv["v"], dtype) if cfg.pv_quant else value
    key_r = repeat_kv(key, reps)
    k_op = repeat_kv(k_op, reps)
    v_op = repeat_kv(v_op, reps)
    value_r = repeat_kv(value, reps)
    q_op = fake_quantize_tail(query, cfg.qk_spec, lv["q"], dtype) if cfg.qk_quant else query
    output = np.zeros((B, Hq, Lq, D), dtype=_F32)
    counts = {"qk": 0, "pv": 0}

    def process(q0: int, rows: int, tiles: int) -> None:
        q1 = q0 + rows * tiles
        qt = q_op[:, :, q0:q1].reshape(B, Hq, tiles, rows, D).transpose(2, 0, 1, 3, 4)
        if cfg.qk_quant:
            _record(stats, "q", D, B * Hq * rows * D, cfg.qk_spec.group_size, tiles)
        shape = (tiles, B, Hq, rows, 1)
        m = np.full(shape, -np.inf, dtype=_F32)
        den = np.zeros(shape, dtype=_F32)
        shadow = np.zeros(shape, dtype=_F32) if collect else None
        acc = np.zeros((tiles, B, Hq, rows, D), dtype=_F32)
        for k0 in range(0, Lk, cfg.key_chunk):
            k1 = min(k0 + cfg.key_chunk, Lk)
            first = 0
            if cfg.skip_fully_masked_tiles and mask is None and causal and sliding_window is None:
                off = Lk - Lq
                first = max(0, min(tiles, (k0 - off - q0) // rows))
            active = tiles - first
            if active == 0:
                continue
            aq0 = q0 + first * rows
            kw = k1 - k0
            if cfg.qk_quant:
                _record(stats, "k", D, B * Hq * kw * D, cfg.qk_spec.group_size, active)
            s = np.matmul(qt[first:], np.swapaxes(k_op[None, :, :, k0:k1], -1, -2)).astype(_F32)
            s = (s * scale).astype(_F32)
            if softcap:
                s = (np.tanh((s / _F32(softcap)).astype(_F32)) * _F32(softcap)).astype(_F32)
            if mask is not None and mask.ndim == 4:
                flat = s.transpose(1, 2, 0, 3, 4).reshape(B, Hq, active * rows, kw)
                flat = _four_dimensional_mask(flat, mask, aq0, q1, k0, k1, Lq)
                s = flat.reshape(B, Hq, active, rows, kw).transpose(2, 0, 1, 3, 4)
            else:
                allowed = streaming_mask(
                    batch=B, q0=aq0, q1=q1, k0=k0, k1=k1, query_length=Lq, key_length=Lk,
                    is_causal=causal, sliding_window=sliding_window,
                    query_valid=query_valid, key_valid=key_valid,
                )
                allowed = allowed.reshape(B, 1, active, rows, kw).transpose(2, 0, 1, 3, 4)
                s = np.where(allowed, s, -np.inf).astype(_F32)
            am = m[first:]
            bmax = s.max(axis=-1, keepdims=True)
            new = np.maximum(am, bmax)
            with np.errstate(invalid="ignore", over="ignore"):
                prev = np.where(np.isfinite(am), np.exp((am - new).astype(_F32)), _F32(0)).astype(_F32)
                p = np.where(np.isfinite(s), np.exp((s - new).astype(_F32)), _F32(0)).astype(_F32)
            if cfg.pv_quant:
                p_op = fake_quantize_tail(p, cfg.pv_spec, lv["p"], "float32")
                vt = v_op[:, :, k0:k1]
                _record(stats, "p", kw, B * Hq * rows * kw, cfg.pv_spec.group_size, active)
                _record(stats, "v", D, B * Hq * kw * D, cfg.pv_spec.group_size, active)
            else:
                p_op = p
                vt = value_r[:, :, k0:k1]
            src = p_op if same else p
            d_new = (prev * den[first:] + src.sum(axis=-1, keepdims=True, dtype=_F32)).astype(_F32)
            if collect:
                sh_src = p if same else p_op
                shadow[first:] = (prev * shadow[first:] + sh_src.sum(axis=-1, keepdims=True, dtype=_F32)).astype(_F32)
                ref = p.astype(np.float64)
                err = p_op.astype(np.float64) - ref
                diagnostics["p_values"] += float(ref.size)
                diagnostics["p_zeroed_values"] += float(np.count_nonzero((p_op == 0) & (p > 0)))
                diagnostics["p_error_sq_sum"] += float((err * err).sum())
                diagnostics["p_reference_sq_sum"] += float((ref * ref).sum())
            acc[first:] = (prev * acc[first:] + np.matmul(p_op, vt[None])).astype(_F32)
            den[first:] = d_new
            m[first:] = new
            counts["qk"] += active
            counts["pv"] += active
        if collect:
            qd, ud = (den, shadow) if same else (shadow, den)
            valid = ud > 0
            if np.any(valid):
                ratio = (qd[valid].astype(np.float64) / ud[valid].astype(np.float64)).ravel()
                diagnostics["rows"] += float(ratio.size)
                diagnostics["mass_ratio_sum"] += float(ratio.sum())
                diagnostics["mass_ratio_sq_sum"] += float((ratio * ratio).sum())
                diagnostics["mass_ratio_min"] = min(diagnostics["mass_ratio_min"], float(ratio.min()))
                diagnostics["mass_ratio_max"] = max(diagnostics["mass_ratio_max"], float(ratio.max()))
                idx = np.searchsorted(np.array(PV_MASS_RATIO_BIN_EDGES), ratio, side="left")
                hist = diagnostics["mass_ratio_histogram"]
                for i, c in enumerate(np.bincount(idx, minlength=len(PV_MASS_RATIO_BIN_EDGES) + 1)):
                    hist[i] += float(c)
        with np.errstate(invalid="ignore", divide="ignore"):
            norm = np.where(den > 0, acc / np.maximum(den, np.finfo(np.float32).tiny), _F32(0)).astype(_F32)
        out = norm.transpose(1, 2, 0, 3, 4).reshape(B, Hq, tiles * rows, D)
        if dtype == "bfloat16":
            out = hif4.bf16_round(out)
        elif dtype == "float16":
            out = hif4.fp16_round(out)
        output[:, :, q0:q1] = out

    full = Lq // cfg.query_chunk
    if full:
        process(0, cfg.query_chunk, full)
    tail = full * cfg.query_chunk
    if tail < Lq:
        process(tail, Lq - tail, 1)
    stats["calls"] += 1
    stats["qk_tiles"] += counts["qk"]
    stats["pv_tiles"] += counts["pv"]
    if cfg.qk_quant:
        stats["qk_quantized_tiles"] += counts["qk"]
    if cfg.pv_quant:
        stats["pv_quantized_tiles"] += counts["pv"]
    return np.ascontiguousarray(output.transpose(0, 2, 1, 3))


def summarize_diagnostics(d: dict) -> dict:
    """``summarize_pv_normalizer_diagnostics`` (sfa:95-130)."""
    rows = float(d["rows"])
    values = float(d["p_values"])
    ref = float(d["p_reference_sq_sum"])
    out: dict[str, object] = {"rows": rows, "p_values": values}
    if rows > 0:
        hist = list(d["mass_ratio_histogram"])
        below = PV_MASS_RATIO_BIN_EDGES.index(1.0) + 1
        mean = float(d["mass_ratio_sum"]) / rows
        var = max(float(d["mass_ratio_sq_sum"]) / rows - mean * mean, 0.0)
        out.update(
            mass_ratio_mean=mean,
            mass_ratio_std=math.sqrt(var),
            mass_ratio_min=float(d["mass_ratio_min"]),
            mass_ratio_max=float(d["mass_ratio_max"]),
            mass_ratio_bin_edges=list(PV_MASS_RATIO_BIN_EDGES),
            mass_ratio_histogram=hist,
            mass_ratio_fraction_below_one=sum(hist[:below]) / rows,
            mean_relative_scale_error=mean - 1.0,
        )
    if values > 0:
        out["p_zero_collapse_rate"] = float(d["p_zeroed_values"]) / values
    if ref > 0:
        out["p_relative_l2"] = math.sqrt(float(d["p_error_sq_sum"]) / ref)
    return out


def single_tile_attention(
    query, key, value, cfg: SimConfig, *, scaling=None, is_causal=True, dtype="float32"
) -> np.ndarray:
    """Single-tile closed form (qad_attention.py:112-226) with bottom-right causal mask."""
    query = np.asarray(query, _F32)
    key = np.asarray(key, _F32)
    value = np.asarray(value, _F32)
    B, Hq, Lq, D = query.shape
    reps = Hq // key.shape[1]
    Lk = key.shape[2]
    lv = cfg.levels
    k_op = fake_quantize_tail(key, cfg.qk_spec, lv["k"], dtype) if cfg.qk_quant else key
    v_op = fake_quantize_tail(value, cfg.pv_spec, lv["v"], dtype) if cfg.pv_quant else value
    k_op = repeat_kv(k_op, reps)
    v_op = repeat_kv(v_op, reps)
    q_op = fake_quantize_tail(query, cfg.qk_spec, lv["q"], dtype) if cfg.qk_quant else query
    scale = _F32(scaling if scaling is not None else D**-0.5)
    s = (np.matmul(q_op, np.swapaxes(k_op, -1, -2)).astype(_F32) * scale).astype(_F32)
    if is_causal:
        qp = np.arange(Lk - Lq, Lk)
        allowed = np.arange(Lk)[None, :] <= qp[:, None]
        s = np.where(allowed, s, -np.inf).astype(_F32)
    rmax = s.max(axis=-1, keepdims=True)
    rmax = np.where(np.isfinite(rmax), rmax, _F32(0))
    with np.errstate(invalid="ignore"):
        p = np.exp((s - rmax).astype(_F32)).astype(_F32)
    p_op = fake_quantize_tail(p, cfg.pv_spec, lv["p"], "float32") if cfg.pv_quant else p
    src = p_op if cfg.pv_normalizer_mode == "quantized_same" else p
    den = src.sum(axis=-1, keepdims=True, dtype=_F32)
    acc = np.matmul(p_op, v_op).astype(_F32)
    with np.errstate(invalid="ignore", divide="ignore"):
        out = np.where(den > 0, acc / np.maximum(den, np.finfo(np.float32).tiny), _F32(0)).astype(_F32)
    if dtype == "bfloat16":
        out = hif4.bf16_round(out)
    return np.ascontiguousarray(out.transpose(0, 2, 1, 3))
