"""Attention golden cases: input builders shared by the fixture writer and the tests.

Each case names an input builder, the simulator module flags, call kwargs, the
HiF4 levels used for every operand and the post-RoPE Q/K Hadamard applied
before the simulator (None, 128-point, or 64-point blocks).
"""

from __future__ import annotations

import numpy as np

from oracle import inputs

# name: (input builder, module kwargs, call kwargs, levels, prologue)
CASES = {
    # configuration 1, fp32, causal, both normalizer modes
    "c1_same": ("c1", dict(qk=True, pv=True, mode="quantized_same"), {}, "123", None),
    "c1_unq": ("c1", dict(qk=True, pv=True, mode="unquantized"), {}, "123", None),
    # Qwen3-8B-shaped GQA (4 q heads / 1 kv head), bf16, RoPE + 128-point Hadamard, 3 key tiles
    "qwen_gqa": ("qwen_small", dict(qk=True, pv=True, mode="quantized_same"), {}, "123", 128),
    # chunked prefill: q_len < k_len, bottom-right causal, ragged tails
    "qwen_chunk": ("qwen_chunk", dict(qk=True, pv=True, mode="quantized_same"), {}, "123", 128),
    # Qwen3-32B-shaped: levels 12, Student-t keys, 64-block Hadamard, GQA 8/1
    "qwen32_l12": ("qwen32_small", dict(qk=True, pv=True, mode="quantized_same"), {}, "12", 64),
    # Wan-shaped non-causal MHA with a ragged key tail
    "wan_nc": ("wan_small", dict(qk=True, pv=True, mode="quantized_same", causal=False), {}, "123", 128),
    # flag combinations (historical normalizer; QK only; PV only)
    "flags_qk": ("qwen_small", dict(qk=True, pv=False, mode="unquantized"), {}, "123", None),
    "flags_pv": ("qwen_small", dict(qk=False, pv=True, mode="unquantized"), {}, "123", None),
    "levels13": ("qwen_small", dict(qk=True, pv=True, mode="quantized_same"), {}, "13", None),
}


def build_inputs(name: str):
    """Return (q, k, v) float32 arrays in [B, H, L, D] and the dtype name they hold."""
    if name == "c1":
        q, k, v = inputs.config1()
        return q, k, v, "float32"
    if name == "qwen_small":
        q, k, v = inputs.qwen(41, 4, 1, 384)
        return q, k, v, "bfloat16"
    if name == "qwen_chunk":
        q, k, v = inputs.qwen(42, 4, 2, 300)
        return np.ascontiguousarray(q[:, :, -130:]), k, v, "bfloat16"
    if name == "qwen32_small":
        q, k, v = inputs.qwen(43, 8, 1, 256, student_t_keys=True)
        return q, k, v, "bfloat16"
    if name == "wan_small":
        q, k, v = inputs.wan(44, 2, 300)
        t = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))  # noqa: E731
        return t(q), t(k), t(v), "bfloat16"
    raise KeyError(name)


def golden_output(golden: dict, case: str) -> np.ndarray:
    if f"{case}__out" in golden:
        return golden[f"{case}__out"]
    bits = golden[f"{case}__out_bf16bits"].astype(np.uint32) << 16
    return bits.view(np.float32)
