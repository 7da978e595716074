"""Build libfaquant_amd.so in-tree with hipcc for gfx950.

    python faquant-public_amd/build.py

Flags: -ffp-contract=off keeps every `a * b + c` of the HiF4 arithmetic as two
roundings (the reference's separate elementwise ops); packed fp32 VALU forms are
disabled for the whole device build.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "faquant_amd", "libfaquant_amd.so")
ATTN_MASK_FORMS = 5  # attn_instances.hip is compiled once per masking form

COMPILE = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")
    return path


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with status {proc.returncode}")


def build(verbose: bool = False) -> str:
    """Compile the C ABI, the decode kernels and the attention instantiations (one object
    per masking form), in parallel, and link libfaquant_amd.so."""
    with tempfile.TemporaryDirectory(prefix="faq_build_") as tmp:
        units = [(os.path.join(CSRC, "capi.hip"), [], os.path.join(tmp, "capi.o")),
                 (os.path.join(CSRC, "attn_decode.hip"), [], os.path.join(tmp, "attn_decode.o")),
                 (os.path.join(CSRC, "hif4_linear.hip"), [], os.path.join(tmp, "hif4_linear.o")),
                 (os.path.join(CSRC, "attn_generic.hip"), [], os.path.join(tmp, "attn_generic.o"))]
        for m in range(ATTN_MASK_FORMS):
            units.append((os.path.join(CSRC, "attn_instances.hip"), [f"-DFAQ_ATTN_MASK={m}"],
                          os.path.join(tmp, f"attn_m{m}.o")))
        jobs = min(len(units), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
        with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
            futures = [pool.submit(_run, [hipcc(), *COMPILE, *defs, "-c", src, "-o", obj], verbose)
                       for src, defs, obj in units]
            for f in futures:
                f.result()
        tmp_out = OUT + ".tmp"
        _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *(obj for _, _, obj in units), "-o", tmp_out],
             verbose)
        os.replace(tmp_out, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
