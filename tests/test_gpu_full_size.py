"""Parity at the benchmark configurations' full sizes.

The GPU runs the whole hot path on the full synthetic input of each configuration (the
inputs bench.py times): the Q/K prologue (block Hadamard r64 for Qwen3, 128 for Wan, one
bf16 cast, HiF4 QDQ with the configuration's levels), the V QDQ and the attention kernel.
Sampled output rows are then compared with the oracle run from the same raw rows: its own
rotation and cast (qwen3.py:97-130 / wan22_attention.py:186-192), its own Q/K/V QDQ and
the tiled simulator over every key the rows see (sfa:457-909).  Rows come from the last
position block (ragged at Wan 720p), the middle of the sequence and the first block, in the
first, a middle and the last query head, so several work items, XCDs and KV heads are
covered.  A causal row range [p0, p1) is the oracle with Lq = p1 - p0 over keys [0, p1)
(bottom-right alignment puts each row at its true position).
"""

from __future__ import annotations

import time

import numpy as np
import pytest

from oracle import attention as OA
from oracle import hadamard as OH
from oracle import hif4 as OQ
from tests.test_gpu_attention import assert_close_attention

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CASES = {
    # name: (row ranges relative to L, heads relative to Hq)
    "qwen8b_8k": (((-48, 0), (4096 - 16, 4096 + 16)), (0, -1)),
    "qwen8b_32k": (((-48, 0), (16384 - 16, 16384 + 16), (0, 40)), (0, 13, -1)),
    "qwen32b_16k": (((-48, 0), (8192 - 16, 8192 + 16)), (0, 37, -1)),
    "wan480p": (((-40, 0), (16000, 16032)), (0, 21, -1)),
    "wan720p": (((-32, 0), (37888, 37920), (0, 32)), (0, 17, -1)),
}

# Per-configuration bars, about ten times the error reached on MI355X (relative Frobenius /
# max of the largest magnitude; reached in brackets).  Wan 720p scales heads by up to 4, so
# its scores are large and a P-hat code flip (P from exp2 vs numpy exp, a few ulp apart)
# shows in the sampled rows; the other configurations have no flip in them.
TOLERANCE = {
    "qwen8b_8k": (1e-5, 1e-5),    # [1.3e-7 / 2.9e-7]
    "qwen8b_32k": (1e-5, 1e-5),   # [1.4e-7 / 2.5e-7]
    "qwen32b_16k": (1e-5, 3e-5),  # [7.7e-7 / 2.5e-6]
    "wan480p": (1e-5, 1e-5),      # [1.5e-7 / 2.4e-7]
    "wan720p": (5e-4, 2e-3),      # [5.2e-5 / 1.9e-4]
}


@pytest.mark.parametrize("name", list(CASES))
def test_full_size_sampled_rows_match_oracle(dev, name):
    import bench
    from faquant_amd import _ops

    cfg = bench.CONFIGS[name]
    B, Hq, Hkv, L, causal = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["causal"]
    blk, lv = cfg["hadamard"], cfg["levels"]
    t0 = time.time()
    q, k, v = bench.make_inputs(cfg, dev)
    qh, _ = _ops.operand_prep(q, levels=lv, hadamard=blk, round_dtype=torch.bfloat16)
    kh, _ = _ops.operand_prep(k, levels=lv, hadamard=blk, round_dtype=torch.bfloat16)
    vt = _ops.operand_prep_vt(v, levels=lv)
    out = torch.empty((B, L, Hq, 128), device=dev, dtype=torch.float32)
    _ops.attention_fwd(qh, kh, vt, L, causal=causal, scale=128**-0.5, quant_p=True, p_levels=lv, norm_same=True,
                       out=out.transpose(1, 2))
    torch.cuda.synchronize()
    print(f"[full] {name} {B}x{Hq}/{Hkv}x{L} causal={causal} r{blk} levels {lv}: gpu {time.time() - t0:.1f}s",
          flush=True)
    ranges, heads = CASES[name]
    G = Hq // Hkv
    mconf = OA.SimConfig(pv_normalizer_mode="quantized_same", levels=dict.fromkeys("qkpv", lv), is_causal=causal)
    rot = lambda a: OH.qk_rotation(a, block_size=blk, out_round=OQ.bf16_round)  # noqa: E731
    kcache = {}
    for hrel in heads:
        h = hrel % Hq
        hk = h // G
        kend_max = L
        if hk not in kcache:  # the KV head's rotated keys and raw values, all positions
            kcache[hk] = (rot(k[:, hk : hk + 1].float().cpu().numpy()), v[:, hk : hk + 1].float().cpu().numpy())
        kr, vr = kcache[hk]
        for a, b in ranges:
            p0 = a % L if a < 0 else a
            p1 = L if b == 0 and a < 0 else b
            kend = p1 if causal else kend_max
            qs = rot(q[:, h : h + 1, p0:p1].float().cpu().numpy())
            ref = OA.simulated_flash_attention(qs, kr[:, :, :kend], vr[:, :, :kend], mconf)
            got = out[:, p0:p1, h : h + 1].cpu().numpy()
            fro_tol, max_tol = TOLERANCE[name]
            assert_close_attention(got, ref, f"{name} rows {p0}:{p1} head {h}", fro_tol=fro_tol, max_tol=max_tol)
    print(f"[full] {name} checked in {time.time() - t0:.1f}s", flush=True)
