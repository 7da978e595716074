"""HiF4 QK/PV flash attention on the MI355X: drop-in for faquant.simulated_flash_attention.

``simulated_flash_attention_forward`` keeps the reference signature, module
attributes, validation messages, stats counters and output layout
(src/faquant/simulated_flash_attention.py:457-909), and computes the same
recurrence in two HIP launches: an operand prologue (HiF4 QDQ of Q, K and V;
V is written transposed for the PV MFMA operand) and the attention kernel.

Supported on the GPU: head_dim 128, key tiles of 128 (the reference default),
the HiF4 format with groups of 64 (or no quantization), causal (bottom-right)
or full attention, 2-D attention masks (padding, in the reference's rank form),
3-D/4-D masks (boolean or additive), sliding windows, the logit softcap, the
PV-normalizer probe, bf16 or fp32 inputs (fp32 with the matching QK / PV
quantization enabled: the kernel multiplies bf16 operands, and HiF4 values are exact in
bf16).  Everything else the reference accepts (int/MXFP8 formats, unquantized fp32
matmuls) raises NotImplementedError: there is no fallback path.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib, _ops
from .config import PV_NORMALIZER_MODES
from .hif4 import HIF4_ATTN_OPERAND_SCALE_LEVELS, HIF4_BLOCK_SIZE

SIMULATED_ATTENTION_IMPLEMENTATION = "faquant_simulated"

_QUANTIZED_OPERANDS = ("q", "k", "p", "v")

PV_MASS_RATIO_BIN_EDGES = (0.5, 0.7, 0.8, 0.9, 0.95, 0.99, 1.0, 1.01, 1.05, 1.1, 1.3)


def new_simulated_attention_stats() -> dict[str, int]:
    """Zeroed counters of one attention runtime (sfa:18-33)."""
    stats = {"calls": 0, "qk_tiles": 0, "pv_tiles": 0, "qk_quantized_tiles": 0, "pv_quantized_tiles": 0}
    for operand in _QUANTIZED_OPERANDS:
        for field in ("quant_calls", "quantized_values", "quant_blocks", "quant_padding_values"):
            stats[f"{operand}_{field}"] = 0
    return stats


_PV_DIAGNOSTIC_KEYS = ("rows", "mass_ratio_sum", "mass_ratio_sq_sum", "mass_ratio_min", "mass_ratio_max",
                       "p_values", "p_zeroed_values", "p_error_sq_sum", "p_reference_sq_sum")


def new_pv_normalizer_diagnostics() -> dict:
    """Zeroed accumulators of the PV-normalizer probe (sfa:74-92): attach the dict to a
    module as ``faquant_pv_normalizer_diagnostics``; the attention output is unchanged."""
    d: dict = dict.fromkeys(_PV_DIAGNOSTIC_KEYS, 0.0)
    d["mass_ratio_min"] = float("inf")
    d["mass_ratio_max"] = float("-inf")
    d["mass_ratio_histogram"] = [0.0] * (len(PV_MASS_RATIO_BIN_EDGES) + 1)
    return d


def summarize_pv_normalizer_diagnostics(diagnostics: dict) -> dict:
    """Per-run scalars of the probe (sfa:95-130): mass-ratio moments, extremes and
    histogram, the P zero-collapse rate and the relative L2 error of P-hat."""
    rows = float(diagnostics["rows"])
    values = float(diagnostics["p_values"])
    energy = float(diagnostics["p_reference_sq_sum"])
    summary: dict = {"rows": rows, "p_values": values}
    if rows > 0:
        hist = list(diagnostics["mass_ratio_histogram"])
        mean = float(diagnostics["mass_ratio_sum"]) / rows
        var = max(float(diagnostics["mass_ratio_sq_sum"]) / rows - mean * mean, 0.0)
        summary.update(
            mass_ratio_mean=mean,
            mass_ratio_std=math.sqrt(var),
            mass_ratio_min=float(diagnostics["mass_ratio_min"]),
            mass_ratio_max=float(diagnostics["mass_ratio_max"]),
            mass_ratio_bin_edges=list(PV_MASS_RATIO_BIN_EDGES),
            mass_ratio_histogram=hist,
            mass_ratio_fraction_below_one=sum(hist[: PV_MASS_RATIO_BIN_EDGES.index(1.0) + 1]) / rows,
            mean_relative_scale_error=mean - 1.0,
        )
    if values > 0:
        summary["p_zero_collapse_rate"] = float(diagnostics["p_zeroed_values"]) / values
    if energy > 0:
        summary["p_relative_l2"] = math.sqrt(float(diagnostics["p_error_sq_sum"]) / energy)
    return summary


def _record_probe(diagnostics: dict, probe: torch.Tensor, p_values: int) -> None:
    """Fold the kernel's per-row probe sums into the accumulators (sfa:130-185, 835-869):
    the elementwise P-hat error terms, and sum(P-hat) / sum(P) of every row whose
    unquantized denominator is positive."""
    t = probe.double()
    diagnostics["p_values"] += float(p_values)
    sums = t[..., 2:].sum(dim=tuple(range(t.dim() - 1))).tolist()
    diagnostics["p_zeroed_values"] += sums[0]
    diagnostics["p_error_sq_sum"] += sums[1]
    diagnostics["p_reference_sq_sum"] += sums[2]
    quantized, unquantized = t[..., 0], t[..., 1]
    valid = unquantized > 0
    if not bool(valid.any()):
        return
    ratio = (quantized[valid] / unquantized[valid]).flatten()
    diagnostics["rows"] += float(ratio.numel())
    diagnostics["mass_ratio_sum"] += float(ratio.sum())
    diagnostics["mass_ratio_sq_sum"] += float(ratio.square().sum())
    diagnostics["mass_ratio_min"] = min(diagnostics["mass_ratio_min"], float(ratio.min()))
    diagnostics["mass_ratio_max"] = max(diagnostics["mass_ratio_max"], float(ratio.max()))
    edges = torch.tensor(PV_MASS_RATIO_BIN_EDGES, device=ratio.device, dtype=ratio.dtype)
    counts = torch.bincount(torch.bucketize(ratio, edges), minlength=len(PV_MASS_RATIO_BIN_EDGES) + 1)
    hist = diagnostics["mass_ratio_histogram"]
    for i, c in enumerate(counts.tolist()):
        hist[i] += float(c)


def register_simulated_attention_backend() -> None:
    """Register this attention with the transformers attention/mask registries (sfa:214-228)."""
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, flash_attention_mask
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    ALL_ATTENTION_FUNCTIONS.register(SIMULATED_ATTENTION_IMPLEMENTATION, simulated_flash_attention_forward)
    ALL_MASK_ATTENTION_FUNCTIONS.register(SIMULATED_ATTENTION_IMPLEMENTATION, flash_attention_mask)


def _record(stats: dict, operand: str, width: int, numel: int, group_size: int, repeats: int) -> None:
    """Logical and padded geometry of one operand QDQ (sfa:187-211)."""
    g = width if group_size == -1 else group_size
    groups = math.ceil(width / g)
    vectors = numel // width
    stats[f"{operand}_quant_calls"] += repeats
    stats[f"{operand}_quantized_values"] += numel * repeats
    stats[f"{operand}_quant_blocks"] += vectors * groups * repeats
    stats[f"{operand}_quant_padding_values"] += vectors * (groups * g - width) * repeats


def key_ranges(
    module,
    attention_mask: Optional[torch.Tensor],
    *,
    batch: int,
    query_length: int,
    key_length: int,
    causal: bool,
    sliding_window: Optional[int],
    device: torch.device,
):
    """Per-row key ranges for a 2-D attention mask and / or a sliding window, and whether
    a mask stays in force.  sfa:561-586: an all-valid mask of a single multi-token prompt
    is the mask-free bottom-right case (tile skipping stays on); every other 2-D mask
    keeps the rank form of sfa:406-427 (unpadded FlashAttention alignment), which the
    kernel runs as key ranges plus valid-key bits."""
    key_mask = None
    if attention_mask is not None:
        if attention_mask.ndim != 2:
            raise ValueError("key ranges come from a 2-D attention mask")
        skip = bool(getattr(module, "faquant_skip_fully_masked_tiles", True))
        all_valid_prefill = (
            skip and batch == 1 and query_length > 1 and bool(torch.all(attention_mask[:, -key_length:]).item())
        )
        if not all_valid_prefill:
            if attention_mask.shape[-1] < key_length:
                raise ValueError("2-D attention mask is shorter than the simulated key sequence")
            key_mask = attention_mask[:, -key_length:]
    if key_mask is None and sliding_window is None:
        return None, False
    ranges = _ops.attention_key_ranges(key_mask, batch, query_length, key_length, causal=causal,
                                       window=sliding_window, device=device)
    return ranges, key_mask is not None


def count_tiles(
    stats: dict,
    *,
    batch: int,
    query_heads: int,
    query_length: int,
    key_length: int,
    head_dim: int,
    query_chunk: int,
    key_chunk: int,
    causal: bool,
    skip_fully_masked: bool,
    qk_quant: bool,
    pv_quant: bool,
    qk_group: int,
    pv_group: int,
) -> None:
    """The simulator's counters in closed form: its query-tile / key-tile schedule
    (sfa:623-697, 886-908) replayed without computing anything."""
    passes = []
    full = query_length // query_chunk
    if full:
        passes.append((0, query_chunk, full))
    tail = full * query_chunk
    if tail < query_length:
        passes.append((tail, query_length - tail, 1))
    tiles_done = 0
    for q0, rows, tiles in passes:
        if qk_quant:
            _record(stats, "q", head_dim, batch * query_heads * rows * head_dim, qk_group, tiles)
        for k0 in range(0, key_length, key_chunk):
            kw = min(k0 + key_chunk, key_length) - k0
            first = 0
            if skip_fully_masked and causal:
                first = max(0, min(tiles, (k0 - (key_length - query_length) - q0) // rows))
            active = tiles - first
            if active == 0:
                continue
            if qk_quant:
                _record(stats, "k", head_dim, batch * query_heads * kw * head_dim, qk_group, active)
            if pv_quant:
                _record(stats, "p", kw, batch * query_heads * rows * kw, pv_group, active)
                _record(stats, "v", head_dim, batch * query_heads * kw * head_dim, pv_group, active)
            tiles_done += active
    stats["calls"] += 1
    stats["qk_tiles"] += tiles_done
    stats["pv_tiles"] += tiles_done
    if qk_quant:
        stats["qk_quantized_tiles"] += tiles_done
    if pv_quant:
        stats["pv_quantized_tiles"] += tiles_done


def _hif4_group(kwargs: dict, what: str) -> int:
    """Validate matmul quant kwargs for the HIP path; return the group size."""
    fmt = kwargs.get("quant_format", "int")
    if fmt != "hif4":
        raise NotImplementedError(f"{what} quantization with quant_format={fmt!r} is not implemented on the MI355X")
    if kwargs.get("bits", 4) != 4:
        raise ValueError("HiF4 requires bits=4")
    group = kwargs.get("group_size", -1)
    if group not in (-1, HIF4_BLOCK_SIZE):
        raise ValueError("HiF4 requires group_size=64 (or -1 for direct use)")
    if not kwargs.get("symmetric", True):
        raise ValueError("HiF4 does not support asymmetric quantization")
    if kwargs.get("clip_ratio", 1.0) != 1.0:
        raise ValueError("HiF4 direct-cast does not support clipping")
    return HIF4_BLOCK_SIZE if group == -1 else group


_KV_STATE = "_faquant_amd_kv_cache_state"
_KV_GROWTH = 1024  # keys of headroom added when a decode cache buffer grows


def _cache_capacity(length: int) -> int:
    return _ops._pad_keys(length)


def _append_allowed(module, name: str, state, tensor: torch.Tensor, query_length: int) -> bool:
    """The reference's append condition (sfa:268-276): decode step, the cache this
    module holds is ours and still attached, same device/dtype/leading shape/head_dim,
    and exactly one new position."""
    return (
        query_length == 1
        and state is not None
        and getattr(module, name, None) is state["view"]
        and state["device"] == tensor.device
        and state["dtype"] == tensor.dtype
        and state["lead"] == tuple(tensor.shape[:-2])
        and state["length"] + 1 == tensor.shape[-2]
    )


def _key_operand(module, key: torch.Tensor, *, enabled: bool, query_length: int, levels: str, **prep) -> torch.Tensor:
    """bf16 K operand [B, Hkv, Lk, 128]; with K quantization it doubles as the decode QDQ
    cache ``faquant_k_matmul_qdq_cache`` (sfa:243-289): a decode step quantizes only the
    appended position into a capacity-padded buffer.  K QDQ (and the optional Q/K
    prologue ``prep`` of operand_prep) is token-local, so this is bitwise equal to
    quantizing the whole cache again."""
    name = "faquant_k_matmul_qdq_cache"
    states = getattr(module, _KV_STATE, None) or {}
    if not enabled:
        setattr(module, name, None)
        states.pop("k", None)
        setattr(module, _KV_STATE, states)
        return _ops.operand_prep(key, levels=None, **prep)[0]
    B, H, L, D = key.shape
    st = states.get("k")
    if _append_allowed(module, name, st, key, query_length):
        buf = st["buf"]
        if L > buf.shape[2]:
            grown = torch.empty((B, H, _cache_capacity(L + _KV_GROWTH), D), device=key.device, dtype=torch.bfloat16)
            grown[:, :, : L - 1].copy_(buf[:, :, : L - 1])
            buf = grown
        _ops.operand_prep(key[:, :, L - 1 :], levels=levels, out=buf[:, :, L - 1 : L], **prep)
    else:
        buf = torch.empty((B, H, _cache_capacity(L), D), device=key.device, dtype=torch.bfloat16)
        _ops.operand_prep(key, levels=levels, out=buf[:, :, :L], **prep)
    view = buf[:, :, :L]
    states["k"] = dict(buf=buf, view=view, length=L, device=key.device, dtype=key.dtype, lead=(B, H))
    setattr(module, _KV_STATE, states)
    setattr(module, name, view)
    return view


def _value_operand(module, value: torch.Tensor, *, enabled: bool, query_length: int, levels: str) -> torch.Tensor:
    """bf16 V operand [B, Hkv, Lk, 128] in natural rows; with V quantization it doubles as
    the decode QDQ cache ``faquant_v_matmul_qdq_cache`` (sfa:243-289), a capacity-padded
    buffer where a decode step quantizes only the appended position.  The prefill kernels
    take a transposed copy (transposed_values)."""
    name = "faquant_v_matmul_qdq_cache"
    states = getattr(module, _KV_STATE, None) or {}
    if not enabled:
        setattr(module, name, None)
        states.pop("v", None)
        setattr(module, _KV_STATE, states)
        return value
    B, H, L, D = value.shape
    st = states.get("v")
    if _append_allowed(module, name, st, value, query_length):
        buf = st["buf"]
        if L > buf.shape[2]:
            grown = torch.empty((B, H, _cache_capacity(L + _KV_GROWTH), D), device=value.device, dtype=torch.bfloat16)
            grown[:, :, : L - 1].copy_(buf[:, :, : L - 1])
            buf = grown
        _ops.operand_prep(value[:, :, L - 1 :], levels=levels, out=buf[:, :, L - 1 : L])
    else:
        buf = torch.empty((B, H, _cache_capacity(L), D), device=value.device, dtype=torch.bfloat16)
        _ops.operand_prep(value, levels=levels, out=buf[:, :, :L])
    view = buf[:, :, :L]
    states["v"] = dict(buf=buf, view=view, length=L, device=value.device, dtype=value.dtype, lead=(B, H))
    setattr(module, _KV_STATE, states)
    setattr(module, name, view)
    return view


def transposed_values(v: torch.Tensor) -> torch.Tensor:
    """V^T [B, H, 128, Lpad] (zero padded) of bf16 V values, the prefill kernels' operand (an
    exact copy: HiF4 values are bf16, and unquantized V must be bf16)."""
    return _ops.operand_prep_vt(v, levels=None)


def _packed_cache_enabled(module, qk_quant: bool, pv_quant: bool) -> bool:
    """Packed HiF4 decode caches: the module attribute ``faquant_kv_cache_packed`` (an
    extension of this build), with K and V quantization both on."""
    return bool(getattr(module, "faquant_kv_cache_packed", False)) and qk_quant and pv_quant


def _packed_operands(module, key: torch.Tensor, value: torch.Tensor, *, query_length: int, levels, prep: dict):
    """The decode K/V caches of sfa:243-289 held packed (4.5 bits per value, PackedHiF4KV):
    ``faquant_k_matmul_qdq_cache`` / ``faquant_v_matmul_qdq_cache`` are PackedHiF4KV objects
    whose rows decode to the bf16 QDQ values of the unpacked caches.  A decode step packs
    only the appended position (the same append condition); anything else packs the whole
    tensor.  K takes the operand prologue ``prep`` (Hadamard, Smooth-QK, key offset)."""
    states = getattr(module, _KV_STATE, None) or {}
    states.pop("k", None)  # no bf16 caches beside the packed ones
    states.pop("v", None)
    caches = []
    for name, t, lv, pre in (("k", key, levels["k"], prep), ("v", value, levels["v"], {})):
        attr = f"faquant_{name}_matmul_qdq_cache"
        st = states.get("packed_" + name)
        B, H, L, _ = t.shape
        if _append_allowed(module, attr, st, t, query_length):
            cache = st["buf"]
            if L > cache.capacity:
                cache = cache.grow(_cache_capacity(L + _KV_GROWTH))
            _ops.pack_operand(t[:, :, L - 1 :], levels=lv, out=cache, start=L - 1, **pre)
        else:
            cache = _ops.PackedHiF4KV(B, H, _cache_capacity(L), t.device, lv)
            _ops.pack_operand(t, levels=lv, out=cache, **pre)
        cache.length = L
        states["packed_" + name] = dict(buf=cache, view=cache, length=L, device=t.device, dtype=t.dtype, lead=(B, H))
        setattr(module, attr, cache)
        caches.append(cache)
    setattr(module, _KV_STATE, states)
    return caches


def kv_operands_and_attend(module, q_op: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, query_length: int,
                           qk_quant: bool, pv_quant: bool, levels, k_prep: dict, q_prep=None, **attn) -> torch.Tensor:
    """K/V operands through the module's decode caches (sfa:243-289), then the attention
    kernel (``attn``: the keyword arguments of _ops.attention_fwd).  With packed caches the
    calls that attention_fwd runs on the decode kernel (decode-shaped, no mask beyond the
    causal rule) run on the packed rows; any other call takes bf16 operands of the same
    values, so both cache forms give the same bits.  ``q_prep = (hadamard, levels)``: q_op
    holds the raw bf16 query rows, prepared inside the attention kernel (its q_prep) or, for
    the decode kernel, by operand_prep first; the same bits either way."""
    if q_prep is not None:
        attn = dict(attn, q_prep=q_prep)

    def prepared_q():
        if q_prep is None:
            return q_op
        return _ops.operand_prep(q_op, levels=q_prep[1], hadamard=q_prep[0], round_dtype=torch.bfloat16)[0]

    key_length = key.shape[2]
    B, Hq, Hkv = q_op.shape[0], q_op.shape[1], key.shape[1]
    plain = not (attn.get("ranges") is not None or attn.get("softcap") or attn.get("pv_probe") is not None
                 or attn.get("dense_mask") is not None or attn.get("out_levels"))
    # decode steps (too few query rows to fill the GPU, all of a KV head's rows in one MFMA
    # tile, no mask beyond the causal rule) run on the decode kernel: K and V read once
    decode = (plain and _ops.decode_shaped(Hq, Hkv, query_length)
              and _ops._split_count(B, Hq, Hkv, query_length, key_length, _ops._device_cus(q_op.device)) > 1)
    dkw = dict(causal=attn["causal"], scale=attn["scale"], quant_p=attn["quant_p"], p_levels=attn["p_levels"],
               norm_same=attn["norm_same"], out=attn["out"], row_den=attn.get("row_den"))
    if _packed_cache_enabled(module, qk_quant, pv_quant):
        kp, vp = _packed_operands(module, key, value, query_length=query_length, levels=levels, prep=k_prep)
        if decode:
            return _ops.attention_decode(prepared_q(), key_length, packed=(kp, vp), **dkw)
        k_op, _ = _ops.operand_prep(key, levels=levels["k"], **k_prep)
        vt = _ops.operand_prep_vt(value, levels=levels["v"])
        return _ops.attention_fwd(q_op, k_op, vt, key_length, **attn)
    k_op = _key_operand(module, key, enabled=qk_quant, query_length=query_length, levels=levels["k"], **k_prep)
    v_op = _value_operand(module, value, enabled=pv_quant, query_length=query_length, levels=levels["v"])
    if decode:
        return _ops.attention_decode(prepared_q(), key_length, k=k_op, v=v_op, **dkw)
    return _ops.attention_fwd(q_op, k_op, transposed_values(v_op), key_length, **attn)


def _unit_last(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def general_attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, qk_quant: bool, pv_quant: bool,
                   levels, key_chunk: int, **attn) -> torch.Tensor:
    """The simulator's operands and tile loop where the MFMA kernel's bf16 operands do not
    carry them as given: Q, K and V fake-quantized along head_dim in 64-value groups with a
    zero-padded tail (sfa:292-338, 592-619) where their matmul is quantized, taken as they are
    otherwise; P quantized per 64-key group of each key chunk.  K/V are quantized on every
    call: the reference's decode cache (sfa:243-289) holds the same values, since the QDQ is
    per position.

    With key chunks of 128 and head_dim up to 128 the MFMA kernel takes the call whenever its
    bf16 operands hold the values exactly: HiF4 values (at most six significant bits; rounded
    to fp16 they keep that inside bf16's range, fp16 subnormals and infinities included) or
    bf16 inputs.  Operands narrower than 128 are zero-padded to 128 dims, which adds exact zeros
    to every score and fills output columns that are dropped; the fp32 output is rounded to the
    query's dtype once, as the reference's ``.to(query.dtype)`` does.  Everything else (other
    key chunks, head_dim above 128, unquantized fp32 or fp16 operands) runs the general kernel
    (_ops.attention_general)."""
    out = attn.pop("out")
    q_op = _ops.qdq_rows(query, levels["q"]) if qk_quant else _unit_last(query)
    k_op = _ops.qdq_rows(key, levels["k"]) if qk_quant else _unit_last(key)
    v_op = _ops.qdq_rows(value, levels["v"]) if pv_quant else _unit_last(value)
    D = query.shape[-1]
    exact_qk = qk_quant or (q_op.dtype == torch.bfloat16 and k_op.dtype == torch.bfloat16)
    exact_v = pv_quant or v_op.dtype == torch.bfloat16
    if key_chunk == _ops.KEY_TILE and D <= _ops.HEAD_DIM and exact_qk and exact_v:
        def bf(t):  # exact: HiF4 or bf16 values
            t = t.to(torch.bfloat16)
            return torch.nn.functional.pad(t, (0, _ops.HEAD_DIM - D)) if D < _ops.HEAD_DIM else t
        B, Hq, Lq = out.shape[:3]
        out32 = torch.empty((B, Hq, Lq, _ops.HEAD_DIM), device=out.device, dtype=torch.float32)
        _ops.attention_fwd(bf(q_op), bf(k_op), transposed_values(bf(v_op)), key.shape[2], quant_p=pv_quant,
                           p_levels=levels["p"], out=out32, **attn)
        return out.copy_(out32[..., :D])
    return _ops.attention_general(q_op, k_op, v_op, key_tile=key_chunk, quant_p=pv_quant, p_levels=levels["p"],
                                  out=out, **attn)


def simulated_flash_attention_forward(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Optional[torch.Tensor],
    dropout: float = 0.0,
    scaling: Optional[float] = None,
    sliding_window: Optional[int] = None,
    softcap: Optional[float] = None,
    **kwargs: object,
) -> tuple[torch.Tensor, None]:
    """Tiled HiF4 flash attention (reference sfa:457-909) on the MI355X."""
    if dropout:
        raise ValueError("simulated FlashAttention only supports dropout=0 inference")
    if softcap is not None and softcap < 0:
        raise ValueError("softcap must be non-negative")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError("sliding_window must be positive")
    if kwargs.get("output_attentions", False):
        raise ValueError("simulated FlashAttention does not materialize attention weights")
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("simulated FlashAttention expects rank-4 Q/K/V tensors")
    if key.shape != value.shape:
        raise ValueError("simulated FlashAttention requires matching K/V shapes")
    if query.shape[0] != key.shape[0] or query.shape[-1] != key.shape[-1]:
        raise ValueError("simulated FlashAttention received incompatible Q/K shapes")
    if any(kwargs.get(n) is not None for n in ("cu_seq_lens_q", "cu_seq_lens_k", "max_length_q", "max_length_k")):
        raise NotImplementedError("packed cu_seqlens are not supported by the simulator")
    position_ids = kwargs.get("position_ids")
    if attention_mask is None and isinstance(position_ids, torch.Tensor) and position_ids.shape[-1] > 1:
        if torch.any(position_ids[..., 1:] <= position_ids[..., :-1]):
            raise NotImplementedError("packed/reset position_ids are not supported")

    valid_key_length = key.shape[-2]
    if attention_mask is not None:
        valid_key_length = min(valid_key_length, attention_mask.shape[-1])
    cache_position = kwargs.get("cache_position")
    if isinstance(cache_position, torch.Tensor) and cache_position.numel():
        valid_key_length = min(valid_key_length, int(cache_position.max().item()) + 1)
    if valid_key_length < key.shape[-2]:
        key = key[:, :, :valid_key_length]
        value = value[:, :, :valid_key_length]

    batch, query_heads, query_length, head_dim = query.shape
    _, kv_heads, key_length, _ = key.shape
    if query_heads % kv_heads:
        raise ValueError("query heads must be divisible by key/value heads")
    if any(size == 0 for size in query.shape) or key_length == 0:
        raise ValueError("simulated FlashAttention does not support zero dimensions")

    scale = float(scaling if scaling is not None else head_dim**-0.5)
    query_chunk = int(module.faquant_attention_query_chunk_size)
    key_chunk = int(module.faquant_attention_key_chunk_size)
    quant_kwargs = module.faquant_matmul_quant_kwargs
    qk_quant_kwargs = getattr(module, "faquant_qk_matmul_quant_kwargs", quant_kwargs)
    pv_quant_kwargs = getattr(module, "faquant_pv_matmul_quant_kwargs", quant_kwargs)
    qk_quant = bool(module.faquant_qk_matmul_quant)
    pv_quant = bool(module.faquant_pv_matmul_quant)
    mode = getattr(module, "faquant_pv_normalizer_mode", "unquantized")
    if mode not in PV_NORMALIZER_MODES:
        raise ValueError(f"unsupported pv_normalizer_mode {mode!r}; expected one of {PV_NORMALIZER_MODES}")
    requested_causal = kwargs.get("is_causal")
    is_causal = bool(getattr(module, "is_causal", True) if requested_causal is None else requested_causal)
    skip = bool(getattr(module, "faquant_skip_fully_masked_tiles", True))

    if attention_mask is not None and attention_mask.ndim not in (2, 3, 4):
        raise ValueError("attention mask must be rank 2, 3, or 4")
    if key_chunk <= 0:
        raise ValueError("attention key chunk size must be positive")
    if query_chunk <= 0:
        raise ValueError("attention query chunk size must be positive")
    for t in (query, key, value):
        if t.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise NotImplementedError(f"the HIP attention path takes bf16, fp16 or fp32 operands, got {t.dtype}")
    # The MFMA kernel multiplies bf16 operands over key tiles of 128 at head_dim 128.
    # Quantized operands are HiF4 values, exact in bf16; without quantization the reference
    # multiplies the inputs themselves in fp32 (sfa:723-724, 848-850), which only bf16 inputs
    # reproduce on bf16 MFMAs.  Every other shape or operand type (fp16 operands included)
    # runs the general kernel, which multiplies in fp32.
    general = (key_chunk != _ops.KEY_TILE or head_dim != _ops.HEAD_DIM
               or torch.float16 in (query.dtype, key.dtype, value.dtype)
               or (not qk_quant and (query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16))
               or (not pv_quant and value.dtype != torch.bfloat16))
    if general and head_dim > _ops.GENERAL_MAX_DIM:
        raise NotImplementedError(f"the MI355X attention supports head_dim up to {_ops.GENERAL_MAX_DIM}, got {head_dim}")
    if general and key_chunk > _ops.GENERAL_MAX_TILE:
        raise NotImplementedError(
            f"the MI355X attention supports key chunks of up to {_ops.GENERAL_MAX_TILE} keys, got {key_chunk}")
    qk_group = _hif4_group(qk_quant_kwargs, "QK") if qk_quant else 64
    pv_group = _hif4_group(pv_quant_kwargs, "PV") if pv_quant else 64
    diagnostics = getattr(module, "faquant_pv_normalizer_diagnostics", None)
    collect = pv_quant and isinstance(diagnostics, dict)

    levels = HIF4_ATTN_OPERAND_SCALE_LEVELS
    q_levels = levels["q"] if qk_quant else None
    if general:
        q_prep = None
    else:
        # bf16 rows: the attention kernel applies Q's QDQ as it loads them
        q_prep = (0, q_levels) if _ops.raw_q_operand_ok(query, 0) else None
        q_op = query if q_prep is not None else _ops.operand_prep(query, levels=q_levels)[0]

    dense = None
    if attention_mask is not None and attention_mask.ndim in (3, 4):
        # sfa:730-757: a 3-D/4-D mask is added to the scores instead of the causal / window rule
        dense = _ops.dense_attention_mask(attention_mask, batch, query_heads, query_length, key_length)
        ranges, masked = None, True
    else:
        ranges, masked = key_ranges(module, attention_mask, batch=batch, query_length=query_length,
                                    key_length=key_length, causal=is_causal, sliding_window=sliding_window,
                                    device=query.device)
    output = torch.empty((batch, query_length, query_heads, head_dim), device=query.device, dtype=query.dtype)
    probe = (torch.empty((batch, query_heads, query_length, 5), device=query.device, dtype=torch.float32)
             if collect else None)
    if general:
        general_attend(query, key, value, qk_quant=qk_quant, pv_quant=pv_quant, levels=levels, key_chunk=key_chunk,
                       causal=is_causal, scale=scale, norm_same=mode == "quantized_same", out=output.transpose(1, 2),
                       ranges=ranges, softcap=softcap, pv_probe=probe, dense_mask=dense)
    else:
        kv_operands_and_attend(
            module, q_op, key, value, query_length=query_length, qk_quant=qk_quant, pv_quant=pv_quant,
            levels=levels, k_prep={}, q_prep=q_prep, causal=is_causal, scale=scale, quant_p=pv_quant,
            p_levels=levels["p"], norm_same=mode == "quantized_same", out=output.transpose(1, 2), ranges=ranges,
            softcap=softcap, pv_probe=probe, dense_mask=dense,
        )
    p_values_before = module.faquant_simulated_attention_stats["p_quantized_values"]
    count_tiles(
        module.faquant_simulated_attention_stats,
        batch=batch, query_heads=query_heads, query_length=query_length, key_length=key_length,
        head_dim=head_dim, query_chunk=query_chunk, key_chunk=key_chunk, causal=is_causal,
        # the reference skips fully future tiles only without a mask or window (sfa:676-681)
        skip_fully_masked=skip and not masked and sliding_window is None,
        qk_quant=qk_quant, pv_quant=pv_quant, qk_group=qk_group, pv_group=pv_group,
    )
    if collect:
        # every processed P tile counts all its values (sfa:139), as the P QDQ stats do
        _record_probe(diagnostics, probe,
                      module.faquant_simulated_attention_stats["p_quantized_values"] - p_values_before)
    return _lib.forward_only(output, query, key, value), None
