"""Build libdsk.so (all HIP sources of this directory) for gfx950 with hipcc.

Usage: python build.py [--out PATH]

The library links only libamdhip64 (no torch, no CUDA-compat headers). Packed
FP32 instructions are disabled (-packed-fp32-ops) on purpose.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
DEFAULT_OUT = os.path.join(PKG, "ds_kernels", "libdsk.so")
SOURCES = ["dsk_errors.hip", "gate.hip", "moe_route.hip", "gemm.hip", "gemv.hip", "mla.hip", "mla_decode.hip",
           "moe_layer.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libdsk.so)")


def build(out: str = DEFAULT_OUT, extra: list[str] | None = None, verbose: bool = False) -> str:
    tmp = out + ".tmp"
    cmd = [
        hipcc(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-shared", "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result", "-o", tmp,
    ] + [os.path.join(HERE, s) for s in SOURCES] + (extra or [])
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    # Keep only real diagnostics (the host pass does not know the gfx feature flag).
    noise = "is not a recognized feature for this target"
    msgs = [l for l in (res.stdout + res.stderr).splitlines() if noise not in l and l.strip()]
    if msgs and verbose:
        print("\n".join(msgs))
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=DEFAULT_OUT)
    args, extra = ap.parse_known_args()  # anything else is passed to hipcc (e.g. -D options)
    path = build(args.out, extra=extra, verbose=True)
    print("built", path)
