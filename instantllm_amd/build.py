"""Builds the HIP engine library in-tree: instantllm_amd/libillhip.so (gfx950).

Flags: -O3, -ffp-contract=off (every multiply-add in the kernels is written as an explicit
fmaf, so the per-row arithmetic is the same instruction sequence in every T-instantiation),
and packed-FP32 instruction selection disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc" / "ill_engine.hip"
OUT = HERE / "libillhip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-value",
    f"-Wl,--version-script={HERE / 'csrc' / 'exports.map'}",
]


def build(verbose: bool = False) -> Path:
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, str(SRC), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    p = build(verbose=True)
    print("built", p, p.stat().st_size, "bytes")
    sys.exit(0)
