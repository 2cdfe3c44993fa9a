"""Builds ``libmi355x_sampler.so`` (the HIP kernels + C-ABI) in-tree with hipcc for gfx950.

    python inferrsi-minicpm-o-4.5-npu_amd/mi355x_sampler/build.py

Cross-compiles without a GPU.  The library lands next to this file, where
``_lib`` loads it from; it is git-ignored but travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG_ROOT = HERE.parent
REPO = PKG_ROOT.parent
SOURCES = [PKG_ROOT / "csrc" / "sampler.hip"]
INCLUDE = REPO / "include"
OUT = HERE / "libmi355x_sampler.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Every float product and sum rounds on its own, as torch's eager ops do.
    "-ffp-contract=off",
    # No packed FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the sampler library)")


def build(verbose: bool = False) -> Path:
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", "-o", str(tmp), *map(str, SOURCES)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


def build_probe(src: Path, out: Path, verbose: bool = False) -> Path:
    """A test-only HIP library from one source next to the tests (same flags and headers as the sampler)."""
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{PKG_ROOT / 'csrc'}", "-o", str(tmp), str(src)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out_txt = "\n".join(line for line in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{out_txt}")
    if verbose and out_txt.strip():
        print(out_txt, file=sys.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
