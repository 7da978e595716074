"""HiF4 QK/PV attention benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config qwen8b_32k] [--no-cpu-baseline]

A step is one pass of the hot path over one batch of synthetic, HBM-resident
input: the Q/K prologue (post-RoPE block Hadamard, one bf16 cast, HiF4 QDQ),
the V QDQ (written transposed) and the HiF4 QK/PV flash-attention kernel.
``value`` = algorithmic QK+PV FLOPs / step time (TFLOP/s).  ``roofline`` is the
attention kernel alone: the same FLOPs / its mean launch time measured with HIP
events on the stream it runs on, against the 2.5 PFLOP/s dense bf16 MFMA peak.
``cpu_baseline`` times the numpy oracle (the CPU restatement of the reference
simulator) on a bounded sample of the same workload: the last ``rows`` query rows
of one KV group (``G`` query heads), split over worker processes, scaled by its own
algorithmic FLOPs.
One JSON line is printed on rank 0.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "faquant-public_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

MFMA_BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBPS = 8000.0

# HBM bytes per attention launch, measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE and
# scaled by the same counters on a 256 MiB device copy (bench.py --calibrate-copy), each
# stamped with the hash of the kernel sources it was measured on (KERNEL_SOURCES).  A
# figure whose stamp differs from the sources in the tree is stale: it is reported as
# null, with the stamp, instead of being passed off as this kernel's traffic.
KERNEL_SOURCES = ("faquant-public_amd/csrc/hif4_attention.hip", "faquant-public_amd/csrc/attn_instances.hip",
                  "faquant-public_amd/csrc/hif4_device.h")
MEASURED_TRAFFIC = {
    # config: (bytes per launch, kernel source sha256 prefix, profile)
    "qwen8b_32k": (1.675e9, "00a76ba3d16761b7", "profiles/attn_fwd_qwen8b_32k_counters.md"),
    "qwen8b_8k": (2.159e8, "00a76ba3d16761b7", "profiles/attn_fwd_qwen8b_8k_kernel_trace.md"),
    "qwen32b_16k": (1.099e9, "00a76ba3d16761b7", "profiles/attn_fwd_qwen32b_16k_kernel_trace.md"),
    "wan480p": (3.367e9, "00a76ba3d16761b7", "profiles/attn_fwd_wan480p_kernel_trace.md"),
    "wan720p": (1.873e10, "00a76ba3d16761b7", "profiles/attn_fwd_wan720p_kernel_trace.md"),
}


def kernel_source_sha() -> str:
    """sha256 (first 16 hex digits) of the attention kernel's source files."""
    import hashlib

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(REPO, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def traffic_record(config: str) -> tuple[float | None, dict]:
    """(traffic bytes or None, provenance) for the roofline of `config`."""
    current = kernel_source_sha()
    rec = MEASURED_TRAFFIC.get(config)
    if rec is None:
        return None, {"kernel_src_sha256": current, "note": "no counter run for this configuration"}
    nbytes, stamp, profile = rec
    prov = {"profile": profile, "measured_on_kernel_src_sha256": stamp, "kernel_src_sha256": current}
    if stamp != current:
        prov["note"] = "stale: the kernel sources changed since this traffic was measured"
        return None, prov
    return nbytes, prov


CONFIGS = {
    # name: B, Hq, Hkv, L, causal, hadamard block, levels, key distribution, per-head scale
    "qwen8b_32k": dict(B=1, Hq=32, Hkv=8, L=32768, causal=True, hadamard=64, levels="123", keys="normal",
                       workload="Qwen3-8B causal GQA prefill 32k (32q/8kv, d128), block Hadamard r64, HiF4 123"),
    "qwen8b_8k": dict(B=1, Hq=32, Hkv=8, L=8192, causal=True, hadamard=64, levels="123", keys="normal",
                      workload="Qwen3-8B causal GQA prefill 8k (32q/8kv, d128), block Hadamard r64, HiF4 123"),
    "qwen32b_16k": dict(B=1, Hq=64, Hkv=8, L=16384, causal=True, hadamard=64, levels="12", keys="student_t",
                        workload="Qwen3-32B causal GQA prefill 16k (64q/8kv, d128), r64, Student-t keys, HiF4 12"),
    "wan480p": dict(B=1, Hq=40, Hkv=40, L=32760, causal=False, hadamard=128, levels="123", keys="normal",
                    workload="Wan2.2 DiT self-attention 480p (40 heads, 32760 tokens), Hadamard 128, HiF4 123"),
    "wan720p": dict(B=1, Hq=40, Hkv=40, L=75600, causal=False, hadamard=128, levels="123", keys="normal",
                    head_scale=True,
                    workload="Wan2.2 DiT self-attention 720p (40 heads, 75600 tokens), Hadamard 128, HiF4 123"),
}


def rope_(x, theta=1.0e6):
    """In-place-free HF rotate-half RoPE over positions 0..L-1 (fp32 math, bf16 out)."""
    import torch

    L, D = x.shape[-2], x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, device=x.device, dtype=torch.float64) / D))
    ang = torch.arange(L, device=x.device, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    cos, sin = emb.cos().float(), emb.sin().float()
    xf = x.float()
    rot = torch.cat([-xf[..., D // 2:], xf[..., : D // 2]], dim=-1)
    return (xf * cos + rot * sin).to(torch.bfloat16)


def make_inputs(cfg, dev, seed=0):
    import torch

    gen = torch.Generator(device=dev).manual_seed(seed)
    B, Hq, Hkv, L = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"]
    q = torch.randn((B, Hq, L, 128), device=dev, generator=gen)
    if cfg["keys"] == "student_t":
        # Student-t(3) = N / sqrt(chi2_3 / 3)
        n = torch.randn((B, Hkv, L, 128), device=dev, generator=gen)
        chi = torch.randn((3, B, Hkv, L, 128), device=dev, generator=gen).pow(2).sum(0)
        k = n / (chi / 3).sqrt()
    else:
        k = torch.randn((B, Hkv, L, 128), device=dev, generator=gen)
    v = torch.randn((B, Hkv, L, 128), device=dev, generator=gen)
    if cfg.get("head_scale"):
        s = torch.rand((1, Hq, 1, 1), device=dev, generator=gen) * 3.5 + 0.5
        q, k, v = q * s, k * s, v * s
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    if cfg["causal"]:  # the Qwen configurations apply RoPE to Q/K
        q, k = rope_(q), rope_(k)
    return q, k, v


def _cpu_worker_init() -> None:
    """One BLAS / OpenMP thread per worker process (set before the worker imports numpy)."""
    for var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):
        os.environ[var] = "1"


def _cpu_worker(job):
    """Oracle attention (prologue included) for query rows [i0, i1) of the last `rows`
    rows of one KV group: those rows with the keys they can see (bottom-right causal)."""
    import numpy as np

    sys.path.insert(0, REPO)
    from oracle import attention as OA
    from oracle import hadamard as OH
    from oracle import hif4 as OQ
    from oracle import inputs as OI

    G, L, rows, blk, levels, causal, i0, i1 = job
    g = OI.rng(99)
    q = OQ.bf16_round(g.standard_normal((1, G, rows, 128), dtype=np.float32))[:, :, i0:i1]
    k = OQ.bf16_round(g.standard_normal((1, 1, L, 128), dtype=np.float32))
    v = OQ.bf16_round(g.standard_normal((1, 1, L, 128), dtype=np.float32))
    nk = L - rows + i1 if causal else L  # the last key row i1 - 1 sees
    k, v = k[:, :, :nk], v[:, :, :nk]
    mconf = OA.SimConfig(pv_normalizer_mode="quantized_same", levels=dict.fromkeys("qkpv", levels), is_causal=causal)
    t0 = time.perf_counter()
    qr = OH.qk_rotation(q, block_size=blk, out_round=OQ.bf16_round)
    kr = OH.qk_rotation(k, block_size=blk, out_round=OQ.bf16_round)
    OA.simulated_flash_attention(qr, kr, v, mconf, dtype="bfloat16")
    return time.perf_counter() - t0


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, rows, workers):
    """Time the numpy oracle on the last `rows` query rows of one KV group, split into
    row chunks over `workers` processes (one BLAS thread each).  Runs before the process
    touches the GPU, so the workers start from a process with no GPU state."""
    import multiprocessing as mp

    from faquant_amd._ops import attention_flops

    G, L = cfg["Hq"] // cfg["Hkv"], cfg["L"]
    # one chunk per worker: every chunk re-quantizes the K/V tiles its rows see, so fewer,
    # larger chunks waste the least (over the last `rows` of a long sequence the causal
    # spread of work between chunks is small)
    n_chunks = workers
    bounds = [round(i * rows / n_chunks) for i in range(n_chunks + 1)]
    jobs = [(G, L, rows, cfg["hadamard"], cfg["levels"], cfg["causal"], a, b)
            for a, b in zip(bounds[:-1], bounds[1:]) if b > a]
    ctx = mp.get_context("spawn")
    with ctx.Pool(workers, initializer=_cpu_worker_init) as pool:
        # imports and page-in, untimed: one single-row job per worker
        pool.map(_cpu_worker, [j[:6] + (0, 1) for j in jobs[:workers]], chunksize=1)
        t0 = time.perf_counter()
        busy = sum(pool.map(_cpu_worker, jobs, chunksize=1))
        dt = time.perf_counter() - t0
    flops = attention_flops(1, G, rows, L, cfg["causal"])
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": workers,
        "host_cpus": os.cpu_count(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"numpy oracle (CPU restatement of the reference simulator) on the last {rows} query rows "
                   f"x {G} query heads of one KV group over {L} keys, prologue included, in {len(jobs)} row "
                   f"chunks over {workers} worker processes with one BLAS thread each: {flops / 1e9:.2f} GFLOP in "
                   f"{dt:.2f} s wall ({busy:.1f} s of worker time)"),
    }


def device_info() -> dict:
    """The GPU agent as rocminfo reports it: name, architecture, compute units and maximum
    shader clock, and the dense bf16 MFMA peak they imply (CUs x 4096 FLOP per clock x clock),
    beside the 2.5 PFLOP/s specification figure the roofline uses."""
    import subprocess

    try:
        text = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=120).stdout
    except (OSError, subprocess.SubprocessError) as e:
        return {"error": f"rocminfo: {e}"}
    for block in text.split("\nAgent ")[1:]:
        fields = {}
        for line in block.splitlines():
            key, sep, val = line.strip().partition(":")
            if sep and key not in fields:
                fields[key.strip()] = val.strip()
        if fields.get("Device Type") != "GPU":
            continue
        try:
            cus = int(fields["Compute Unit"])
            mhz = int(fields["Max Clock Freq. (MHz)"])
        except (KeyError, ValueError):
            return {"error": "rocminfo: no compute-unit or clock field"}
        return {"name": fields.get("Marketing Name", ""), "arch": fields.get("Name", ""), "cus": cus,
                "max_sclk_mhz": mhz, "bf16_dense_peak_tflops_at_max_sclk": round(cus * 4096 * mhz * 1e6 / 1e12, 1)}
    return {"error": "rocminfo: no GPU agent"}


def mfma_probe(dev) -> float:
    """The device's sustained dense bf16 MFMA rate (TFLOP/s) in the attention kernel's launch
    shape (faq_mfma_probe: MFMA chains only), timed after the benchmark so the clock is warm:
    the measured reference point beside the specification peak."""
    import torch
    from faquant_amd import _lib

    lib = _lib.load()
    blocks = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 20000
    out = torch.empty(blocks * 512, device=dev, dtype=torch.float32)
    stream = _lib.stream_ptr(dev)
    for _ in range(3):
        _lib.check(lib.faq_mfma_probe(out.data_ptr(), blocks, iters, stream))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    reps = 5
    for _ in range(reps):
        _lib.check(lib.faq_mfma_probe(out.data_ptr(), blocks, iters, stream))
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    return blocks * 8 * iters * 4 * 32768 / (ms * 1e-3) / 1e12


def decode_bench(cfg, context: int, steps: int, warmup: int, layers: int = 1, ranges: int | None = None) -> dict:
    """One decode step (one new query position per head) of `cfg`'s heads over `context` cached
    keys, timed three ways with HIP events on the launch stream: the split-key path
    (faq_attention_fwd_split), the decode kernel over bf16 K/V and over packed HiF4 K/V.
    The roofline is HBM: algorithmic bytes = the K and V cache bytes one step must read
    (bf16: 512 per key and KV head, packed: 144) plus Q and the output.  With `layers` > 1 the
    steps cycle through that many independent caches (as a model's layers do), so that the
    caches together exceed the 256 MB last-level cache and every step reads from HBM.  `ranges`
    replaces decode_split_count's number of key ranges for both decode-kernel paths."""
    import torch

    from faquant_amd import _ops

    dev = torch.device("cuda:0")
    B, Hq, Hkv, L = cfg["B"], cfg["Hq"], cfg["Hkv"], context
    lv = cfg["levels"]
    gen = torch.Generator(device=dev).manual_seed(1)
    q = torch.randn((B, Hq, 1, 128), device=dev, generator=gen).to(torch.bfloat16)
    qh, _ = _ops.operand_prep(q, levels=lv, hadamard=cfg["hadamard"], round_dtype=torch.bfloat16)
    caches = []
    for _ in range(max(1, layers)):
        k = torch.randn((B, Hkv, L, 128), device=dev, generator=gen).to(torch.bfloat16)
        v = torch.randn((B, Hkv, L, 128), device=dev, generator=gen).to(torch.bfloat16)
        kh, _ = _ops.operand_prep(k, levels=lv, hadamard=cfg["hadamard"], round_dtype=torch.bfloat16)
        vt = _ops.operand_prep_vt(v, levels=lv)  # the split path's V^T
        vh, _ = _ops.operand_prep(v, levels=lv)  # the decode cache's natural rows
        kc = _ops.pack_operand(k, levels=lv, hadamard=cfg["hadamard"], round_dtype=torch.bfloat16,
                               out=_ops.PackedHiF4KV(B, Hkv, L, dev, lv))
        vc = _ops.pack_operand(v, levels=lv, out=_ops.PackedHiF4KV(B, Hkv, L, dev, lv))
        caches.append((kh, vt, vh, kc, vc))
        del k, v
    out = torch.empty((B, 1, Hq, 128), device=dev, dtype=torch.bfloat16)
    kw = dict(causal=True, scale=128**-0.5, quant_p=True, p_levels=lv, norm_same=True, out=out.transpose(1, 2))
    cus = _ops._device_cus(dev)
    n_split = _ops._split_count(B, Hq, Hkv, 1, L, cus)
    n_dec = _ops.decode_split_count(B, Hkv, L, cus) if ranges is None else ranges
    n_dec_packed = _ops.decode_split_count(B, Hkv, L, cus, packed=True) if ranges is None else ranges
    turn = [0]

    def layer():
        turn[0] += 1
        return caches[turn[0] % len(caches)]

    def split_step():
        kh, vt, _, _, _ = layer()
        return _ops.attention_fwd(qh, kh, vt, L, split=n_split, **kw)

    def dec_step():
        kh, _, vh, _, _ = layer()
        return _ops.attention_decode(qh, L, k=kh, v=vh, split=n_dec, **kw)

    def packed_step():
        _, _, _, kc, vc = layer()
        return _ops.attention_decode(qh, L, packed=(kc, vc), split=n_dec_packed, **kw)

    paths = {
        "split_path_bf16": (split_step, 512, n_split),
        "decode_bf16": (dec_step, 512, n_dec),
        "decode_packed_hif4": (packed_step, 144, n_dec_packed),
    }
    res = {}
    # steps run back to back in five blocks, one event pair around each block, so that the
    # host's launch time for a step overlaps the device's work on the one before (a decode
    # step is tens of microseconds); us_median is the median of the five block means
    blocks = 5
    per_block = max(1, steps // blocks)
    for name, (fn, per_key, nsplit) in paths.items():
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        evs = []
        for _ in range(blocks):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(per_block):
                fn()
            b.record()
            evs.append((a, b))
        torch.cuda.synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 / per_block for a, b in evs)
        mean = sum(us) / len(us)
        nbytes = B * Hkv * L * per_key + 2 * (q.numel() + out.numel())
        gbps = nbytes / (mean * 1e-6) / 1e9
        res[name] = {"us_mean": round(mean, 2), "us_median": round(us[len(us) // 2], 2), "nsplit": nsplit,
                     "algorithmic_bytes": nbytes, "achieved_gbps": round(gbps, 1),
                     "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)}
    return {
        "metric": "HiF4 decode attention step: HBM GB/s on the K/V cache bytes, 1 GPU",
        "unit": "GB/s",
        "higher_is_better": True,
        "config": {"workload": f"{cfg['workload'].split(' causal')[0]} decode step over {L} cached keys",
                   "batch": B, "q_heads": Hq, "kv_heads": Hkv, "context": L, "hif4_levels": lv,
                   "pv_normalizer": "quantized_same"},
        "steps": steps, "warmup": warmup, "data": "synthetic", "layers": max(1, layers),
        "peak_gbps": HBM_PEAK_GBPS,
        "paths": res,
    }


# Linear layers of one Wan2.2-A14B DiT block (wan22_hif4.py BLOCK_LINEARS): (name, in, out)
WAN_BLOCK_LINEARS = (
    ("self_attn.q", 5120, 5120), ("self_attn.k", 5120, 5120), ("self_attn.v", 5120, 5120),
    ("self_attn.o", 5120, 5120), ("cross_attn.q", 5120, 5120), ("cross_attn.o", 5120, 5120),
    ("ffn.0", 5120, 13824), ("ffn.2", 13824, 5120),
)


def linear_bench(tokens: int, steps: int, warmup: int) -> dict:
    """HiF4 W4A4 Linear (HiF4Linear: one HIP launch for the input QDQ, then the library bf16
    GEMM on the HiF4-exact operands) at the Wan2.2 DiT block shapes over `tokens` rows: per
    layer the QDQ and the GEMM timed with HIP events, the GEMM against the 2.5 PFLOP/s dense
    bf16 peak and the QDQ against the 8 TB/s HBM peak (it reads and writes the activations
    once).  The cross-attention K/V projections act on the text context, not on `tokens`."""
    import torch
    from torch.nn import functional as F

    from faquant_amd import _ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(2)
    layers = []
    for name, k, n in WAN_BLOCK_LINEARS:
        x = torch.randn((tokens, k), device=dev, generator=gen).to(torch.bfloat16)
        w = _ops.act_qdq_rows(torch.randn((n, k), device=dev, generator=gen).to(torch.bfloat16) * 0.02, levels="123")
        qx = torch.empty_like(x)

        def timed(fn):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(steps):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / steps

        q_ms = timed(lambda: _ops.act_qdq_rows(x, levels="123", out=qx))
        g_ms = timed(lambda: F.linear(qx, w))
        flops = 2.0 * tokens * k * n
        qbytes = 2 * 2 * tokens * k
        layers.append({"layer": name, "in": k, "out": n, "qdq_us": round(q_ms * 1e3, 1),
                       "qdq_hbm_frac": round(qbytes / (q_ms * 1e-3) / (HBM_PEAK_GBPS * 1e9), 3),
                       "gemm_us": round(g_ms * 1e3, 1), "gemm_tflops": round(flops / (g_ms * 1e-3) / 1e12, 1),
                       "gemm_frac": round(flops / (g_ms * 1e-3) / (MFMA_BF16_PEAK_TFLOPS * 1e12), 3),
                       "qdq_share": round(q_ms / (q_ms + g_ms), 3)})
        del x, w, qx
    tq = sum(l["qdq_us"] for l in layers)
    tg = sum(l["gemm_us"] for l in layers)
    fl = sum(2.0 * tokens * l["in"] * l["out"] for l in layers)
    return {"metric": "HiF4 W4A4 Linear (Wan2.2 DiT block shapes): input QDQ + bf16 GEMM, 1 GPU",
            "tokens": tokens, "steps": steps, "warmup": warmup, "layers": layers,
            "block": {"qdq_us": round(tq, 1), "gemm_us": round(tg, 1), "qdq_share": round(tq / (tq + tg), 3),
                      "tflops": round(fl / ((tq + tg) * 1e-6) / 1e12, 1),
                      "frac": round(fl / ((tq + tg) * 1e-6) / (MFMA_BF16_PEAK_TFLOPS * 1e12), 3)}}


# (name, in_features) of the Qwen3-8B Linear inputs: attention projections and the MLP
QWEN8B_LINEAR_INPUTS = (("q/k/v/o_proj, gate/up_proj", 4096), ("down_proj", 12288))


# Qwen3-8B projection shapes (out_features, in_features) of one decoder layer
QWEN8B_PROJECTIONS = (("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096),
                      ("o_proj", 4096, 4096), ("gate_proj", 12288, 4096), ("up_proj", 12288, 4096),
                      ("down_proj", 4096, 12288))


def linear_decode_bench(rows: int, steps: int, warmup: int, layers: int = 4) -> dict:
    """The HiF4 W4A4 Linear's contraction at the Qwen3-8B projection shapes over `rows` input
    rows (decode steps, small batches): F.linear on the bf16 weight QDQ (the drop-in's path,
    hipBLASLt) against faq_hif4_linear_packed on the packed weight (4.5 bits per weight).  Each
    timed sequence runs the seven projections of `layers` layers (distinct weights, so that
    every call reads its weight from HBM: 4 layers hold 436 MB packed, 1.55 GB bf16), captured
    in a HIP graph and replayed, so that host launch time does not enter; HIP events around
    `steps` replays.  Roofline: HBM, algorithmic bytes = the weight (2 or 0.5625 bytes per
    weight) plus x and y."""
    import torch

    from faquant_amd import _ops
    from faquant_amd.quantization import fake_quantize

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(5)
    shapes = QWEN8B_PROJECTIONS
    bf = [[None] * len(shapes) for _ in range(layers)]
    pk = [[None] * len(shapes) for _ in range(layers)]
    xs = {}
    for li in range(layers):
        for si, (_, n, k) in enumerate(shapes):
            w = (torch.randn((n, k), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
            pk[li][si] = _ops.PackedHiF4Weight(w, "123")
            bf[li][si] = fake_quantize(w, quant_format="hif4", bits=4, group_size=64, hif4_levels="123")
            xs.setdefault(k, _ops.act_qdq_rows(torch.randn((rows, k), device=dev, generator=gen).to(torch.bfloat16),
                                              levels="123"))
            del w

    def seq_bf16():
        for li in range(layers):
            for si, (_, n, k) in enumerate(shapes):
                torch.nn.functional.linear(xs[k], bf[li][si])

    def seq_packed():
        for li in range(layers):
            for si, (_, n, k) in enumerate(shapes):
                _ops.linear_packed(xs[k], pk[li][si])

    def timed(fn):
        for _ in range(2):
            fn()  # buffers (the packed path's counters and workspace) exist before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1000 / steps / layers  # us per layer (seven projections)

    us_bf16, us_packed = timed(seq_bf16), timed(seq_packed)
    w_elems = sum(n * k for _, n, k in shapes)
    io = sum(rows * (k + n) * 2 for _, n, k in shapes)
    out = {
        "metric": "HiF4 W4A4 Linear decode contraction: one Qwen3-8B layer's seven projections, 1 GPU",
        "unit": "us per layer",
        "higher_is_better": False,
        "rows": rows,
        "layers_rotated": layers,
        "steps": steps,
        "warmup": warmup,
        "data": "synthetic",
        "paths": {
            "f_linear_bf16_weight": {"us": round(us_bf16, 2), "bytes": w_elems * 2 + io,
                                     "hbm_frac": round((w_elems * 2 + io) / (us_bf16 * 1e-6) / 8e12, 4)},
            "packed_hif4_weight": {"us": round(us_packed, 2), "bytes": w_elems * 9 // 16 + io,
                                   "hbm_frac": round((w_elems * 9 // 16 + io) / (us_packed * 1e-6) / 8e12, 4)},
        },
        "speedup": round(us_bf16 / us_packed, 3),
    }
    return out


def linear_prep_bench(tokens: int, steps: int, warmup: int) -> dict:
    """The quantized Linear's activation path over `tokens` bf16 rows at the Qwen3-8B input
    widths: the fused prologue without extras (act_qdq_rows: HiF4 QDQ only), the full path
    with the HiSQ rotation (signs, permutation, block Hadamard of 1024), clamp and companding,
    and the generalized online Hadamard of the whole row (act_prep_rows), each against the
    8 TB/s HBM peak on the activation bytes it must move (read and write once)."""
    import torch

    from faquant_amd import _ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    rows = []
    for name, k in QWEN8B_LINEAR_INPUTS:
        x = torch.randn((tokens, k), device=dev, generator=gen).to(torch.bfloat16)
        y = torch.empty_like(x)
        signs = (torch.randint(0, 2, (k,), device=dev, generator=gen) * 2 - 1).to(torch.int8)
        # the kernel's forms of the vectors (int32 permutation, fp32 companding scale holding
        # bf16 values), as FakeQuantLinear caches them
        perm = torch.randperm(k, device=dev, generator=gen).to(torch.int32)
        comp = torch.rand((k,), device=dev, generator=gen).mul(2).sub(1).exp().to(torch.bfloat16).float()
        comp_rcp = _ops.act_compand_rcp(comp, torch.bfloat16)  # a per-layer constant the module keeps

        def timed(fn):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(steps):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / steps

        nbytes = 2 * 2 * tokens * k
        entry = {"inputs": name, "in_features": k}
        for label, fn in (
            ("qdq_only", lambda: _ops.act_qdq_rows(x, levels="123", out=y)),
            ("hisq_clamp_compand", lambda: _ops.act_prep_rows(x, levels="123", rot_signs=signs, rot_perm=perm,
                                                              rot_block=1024, act_min=-8.0, act_max=8.0,
                                                              compand=comp, compand_rcp=comp_rcp, out=y)),
            # the online Hadamard without a block size: the whole row (12 x 1024 at 12288)
            ("online_generalized", lambda: _ops.act_prep_rows(x, levels="123", hadamard_generalized=True, out=y)),
        ):
            ms = timed(fn)
            entry[label] = {"us": round(ms * 1e3, 1),
                            "hbm_frac": round(nbytes / (ms * 1e-3) / (HBM_PEAK_GBPS * 1e9), 3)}
        rows.append(entry)
        del x, y
    return {"metric": "quantized Linear activation path (Qwen3-8B input widths), 1 GPU", "tokens": tokens,
            "steps": steps, "warmup": warmup, "dtype": "bf16", "layers": rows}


GENERAL_SHAPES = (
    # (label, head_dim, key tile, operand dtype, P quantized with the quantized_same normalizer)
    ("key_chunk_64", 128, 64, "bf16", True),
    ("key_chunk_256", 128, 256, "bf16", True),
    ("head_dim_256", 256, 128, "bf16", True),
    ("head_dim_64_key_chunk_64", 64, 64, "bf16", True),
    ("fp32_unquantized", 128, 128, "fp32", False),
)


def general_bench(length: int, steps: int, warmup: int) -> dict:
    """The general attention kernel (faq_attention_fwd_general: key tiles and head dims the
    MFMA kernel does not take, fp32 operands) on Qwen3-8B heads (32 query / 8 KV heads),
    causal prefill over `length` tokens, HIP events around `steps` launches.  The kernel
    multiplies in fp32 on the VALU; its roofline is MI355X's fp32 peak (157.3 TFLOP/s)."""
    import torch

    from faquant_amd import _ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(5)
    B, Hq, Hkv = 1, 32, 8
    rows = []
    for label, D, T, dt, quant in GENERAL_SHAPES:
        dtype = torch.bfloat16 if dt == "bf16" else torch.float32
        q, k, v = (torch.randn((B, h, length, D), device=dev, generator=gen).to(dtype) for h in (Hq, Hkv, Hkv))
        out = torch.empty((B, Hq, length, D), device=dev, dtype=dtype)

        def call():
            _ops.attention_general(q, k, v, key_tile=T, causal=True, scale=D**-0.5, quant_p=quant, p_levels="123",
                                   norm_same=quant, out=out)

        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            call()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / steps
        tflops = _ops.attention_flops(B, Hq, length, length, True, head_dim=D) / (ms * 1e-3) / 1e12
        rows.append({"shape": label, "head_dim": D, "key_chunk": T, "dtype": dt, "quant_p": quant,
                     "ms": round(ms, 3), "tflops": round(tflops, 2), "fp32_peak_frac": round(tflops / 157.3, 3)})
        del q, k, v, out
    return {"metric": "general attention kernel, Qwen3-8B heads, causal prefill, 1 GPU", "seq_len": length,
            "steps": steps, "warmup": warmup, "shapes": rows}


def stream_reference() -> dict:
    """This device's practical rates for plain streams, the measured reference points beside
    the 8 TB/s specification for the HBM-bound decode kernels: torch's copy and sum over
    1 GiB of fp32 (beyond the 256 MiB last-level cache), and the library's read probe
    (faq_stream_probe: coalesced 16-byte loads, four in flight per thread) over 1 GiB and
    over 128 MiB (about a 32k-key decode step's K and V, which the last-level cache holds
    from one read to the next)."""
    import torch

    from faquant_amd import _lib

    dev = torch.device("cuda:0")
    n = (1 << 30) // 4
    x = torch.randn(n, device=dev)
    y = torch.empty_like(x)
    lib = _lib.load()
    stream = _lib.stream_ptr(dev)
    blocks = 4 * _ops_cus(dev)
    out = torch.empty(blocks, device=dev)

    def probe(nbytes):
        return lambda: _lib.check(lib.faq_stream_probe(x.data_ptr(), nbytes, out.data_ptr(), blocks, stream))

    res = {}
    for name, fn, nbytes in (("copy", lambda: y.copy_(x), 8 * n), ("sum", lambda: x.sum(), 4 * n),
                             ("read_probe_1GiB", probe(4 * n), 4 * n), ("read_probe_128MiB", probe(1 << 27), 1 << 27)):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(20):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / 20
        res[name] = {"bytes": nbytes, "us": round(ms * 1e3, 1), "gbps": round(nbytes / ms / 1e6, 1)}
    return {"stream_reference": "1 GiB fp32 through torch copy_ (read + write) and sum (read); faq_stream_probe "
                                "reads of 1 GiB and 128 MiB", **res}


def _ops_cus(dev) -> int:
    from faquant_amd import _ops

    return _ops._device_cus(dev)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the GPU clock settles after a few tens of ms of load: by default the warmup runs at least
    # 10 steps and at least 0.3 s of them (an 8k step is 0.6 ms); --warmup W runs exactly W
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", default="qwen8b_32k", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-rows", type=int, default=16384)  # about 15 s on 16 cores at 32k
    # the CPU share of one GPU on the GPU boxes is 16 cores
    ap.add_argument("--cpu-workers", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--q-prologue", choices=("fused", "separate"), default="fused",
                    help="fused: the attention kernel prepares the raw Q rows as it loads them (faq_attn_opts.q_prep); "
                         "separate: faq_operand_prep writes the Q operand first")
    ap.add_argument("--decode", type=int, default=0, metavar="CONTEXT",
                    help="time one decode step over CONTEXT cached keys of --config's heads instead")
    ap.add_argument("--decode-layers", type=int, default=1, metavar="N",
                    help="with --decode: cycle the steps through N independent K/V caches (N x the cache bytes "
                         "beyond the 256 MB last-level cache makes every step read HBM)")
    ap.add_argument("--decode-ranges", type=int, default=None, metavar="N",
                    help="with --decode: N key ranges for the decode kernel (default: decode_split_count)")
    ap.add_argument("--linear", type=int, default=0, metavar="TOKENS",
                    help="time the HiF4 W4A4 Linear at the Wan2.2 DiT block shapes over TOKENS rows instead")
    ap.add_argument("--linear-decode", type=int, default=0, metavar="ROWS",
                    help="time the HiF4 W4A4 Linear's contraction at the Qwen3-8B projection shapes over ROWS "
                         "input rows: F.linear on bf16 weights against the packed-weight kernel")
    ap.add_argument("--linear-prep", type=int, default=0, metavar="TOKENS",
                    help="time the quantized Linear's activation path (HiSQ rotation, clamp, companding) "
                         "at the Qwen3-8B input widths over TOKENS rows instead")
    ap.add_argument("--general", type=int, default=0, metavar="TOKENS",
                    help="time the general attention kernel (key chunks and head dims other than 128, fp32 "
                         "operands) on Qwen3-8B heads over a causal prefill of TOKENS instead")
    ap.add_argument("--stream-reference", action="store_true",
                    help="measure only the device's practical HBM stream rate (torch copy and sum over 1 GiB)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 256 MiB device copy (the reference kernel for FETCH_SIZE/WRITE_SIZE scaling)")
    args = ap.parse_args()
    warmup = args.warmup if args.warmup is not None else 10  # the other modes' fixed default
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (got --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from faquant_amd import _ops

    if args.linear:
        print(json.dumps(linear_bench(args.linear, args.steps, warmup)), flush=True)
        return

    if args.linear_prep:
        print(json.dumps(linear_prep_bench(args.linear_prep, args.steps, warmup)), flush=True)
        return

    if args.linear_decode:
        print(json.dumps(linear_decode_bench(args.linear_decode, args.steps, warmup)), flush=True)
        return

    if args.general:
        print(json.dumps(general_bench(args.general, args.steps, warmup)), flush=True)
        return

    if args.stream_reference:
        print(json.dumps(stream_reference()), flush=True)
        return

    if args.decode:
        print(json.dumps(decode_bench(CONFIGS[args.config], args.decode, args.steps, warmup, args.decode_layers,
                                      args.decode_ranges)),
              flush=True)
        return

    if args.calibrate_copy:
        src = torch.empty(64 << 20, device="cuda:0", dtype=torch.float32).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4,
                          "launches": 3}), flush=True)
        return

    cfg = CONFIGS[args.config]
    cpu = None if args.no_cpu_baseline else cpu_baseline(cfg, args.cpu_rows, args.cpu_workers)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, k, v = make_inputs(cfg, dev)
    B, Hq, Hkv, L = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"]
    causal = cfg["causal"]
    levels = cfg["levels"]
    flops = _ops.attention_flops(B, Hq, L, L, causal)
    out = torch.empty((B, L, Hq, 128), device=dev, dtype=torch.bfloat16)
    qh = torch.empty((B, Hq, L, 128), device=dev, dtype=torch.bfloat16)
    kh = torch.empty((B, Hkv, L, 128), device=dev, dtype=torch.bfloat16)

    ev = []
    pev = []

    fused_q = args.q_prologue == "fused"

    def step(record=False):
        if record:
            p0 = torch.cuda.Event(enable_timing=True)
            p0.record()
        if not fused_q:
            _ops.operand_prep(q, levels=levels, hadamard=cfg["hadamard"], round_dtype=torch.bfloat16, out=qh)
        _ops.operand_prep(k, levels=levels, hadamard=cfg["hadamard"], round_dtype=torch.bfloat16, out=kh)
        vt = _ops.operand_prep_vt(v, levels=levels)
        if record:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            pev.append((p0, a))
        # fused: the kernel applies Q's prologue (Hadamard, bf16 cast, QDQ) to the raw rows
        _ops.attention_fwd(q if fused_q else qh, kh, vt, L, causal=causal, scale=128**-0.5, quant_p=True,
                           p_levels=levels, norm_same=True, out=out.transpose(1, 2),
                           q_prep=(cfg["hadamard"], levels) if fused_q else None)
        if record:
            b.record()
            ev.append((a, b))

    warm = 0
    t_warm = time.perf_counter()
    while warm < (args.warmup if args.warmup is not None else 10) or (
            args.warmup is None and time.perf_counter() - t_warm < 0.3):
        step()
        warm += 1
        if warm % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(record=True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    kern_ms = sorted(a.elapsed_time(b) for a, b in ev)
    kern_mean = sum(kern_ms) / len(kern_ms)
    kern_median = kern_ms[len(kern_ms) // 2]
    achieved = flops / (kern_mean * 1e-3) / 1e12
    value = flops / (ms_step * 1e-3) / 1e12
    # the Q/K/V prologue (HBM-bound): operand reads, bf16 Q/K writes, the padded V^T write
    pro_ms = sum(a.elapsed_time(b) for a, b in pev) / len(pev)
    lpad = -(-L // 128) * 128
    # (with the fused Q prologue the kernel reads the raw Q rows itself: no Q bytes here)
    q_bytes = 0 if fused_q else q.numel() * q.element_size() + 2 * qh.numel()
    pro_bytes = (q_bytes + k.numel() * k.element_size() + v.numel() * v.element_size()
                 + 2 * (kh.numel() + B * Hkv * 128 * lpad))
    pro_gbps = pro_bytes / (pro_ms * 1e-3) / 1e9

    traffic, traffic_prov = traffic_record(args.config)
    result = {
        "metric": "HiF4 QK/PV attn TFLOP/s + % MFMA peak, Qwen3-8B causal prefill 32k, 1 GPU",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warm,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": cfg["workload"],
            "name": args.config,
            "batch": B, "q_heads": Hq, "kv_heads": Hkv, "seq_len": L, "head_dim": 128,
            "causal": causal, "qk_hadamard_block": cfg["hadamard"], "hif4_levels": levels,
            "pv_normalizer": "quantized_same", "key_tile": 128, "q_prologue": args.q_prologue,
            "flops_per_step": flops,
        },
        "pct_mfma_peak": round(100.0 * value / MFMA_BF16_PEAK_TFLOPS, 2),
        "attention_kernel_ms_mean": round(kern_mean, 4),
        "attention_kernel_ms_median": round(kern_median, 4),
        "prologue_ms": round(pro_ms, 4),
        "prologue_roofline": {
            "bound": "hbm",
            "achieved": round(pro_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(pro_gbps / HBM_PEAK_GBPS, 4),
            "bytes": pro_bytes,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "traffic_provenance": traffic_prov,
        },
    }
    probe = mfma_probe(dev)
    result["mfma_probe"] = {
        "tflops": round(probe, 1),
        "pct_spec_peak": round(100.0 * probe / MFMA_BF16_PEAK_TFLOPS, 2),
        "kernel_frac_of_probe": round(achieved / probe, 4),
    }
    result["device"] = device_info()
    if cpu is not None:
        result["cpu_baseline"] = cpu
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
