"""Builds libt2t_hip.so (all HIP kernels + the C ABI) in-tree for gfx950.

Usage: python -m token2tile_amd.build [--debug]

The library is written next to this file so that it travels with the source
tree; ``token2tile_amd._lib`` loads it and never builds on its own.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libt2t_hip.so"
OBJ = PKG / "_obj"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    # packed fp32 ops stay off: hipcc would otherwise emit them from plain
    # float code on gfx950.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(PKG.parent / "include"),
]


# per-file extra compiler flags.  kmeans.hip: MFMA accumulators in VGPRs
# rather than AGPRs; the assignment's min tree reads all 16 per block, and the
# AGPR form spent 16 v_accvgpr_read per block on moving them out
EXTRA: dict = {"kmeans.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, debug: bool) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if debug:
        cmd += ["-g"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    warn = [l for l in r.stderr.splitlines()
            if l.strip() and "packed-fp32-ops" not in l and "ignoring feature" not in l]
    if warn:
        sys.stderr.write("\n".join(warn) + "\n")
    return obj


def build(debug: bool = False, jobs: int = 8) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, debug), srcs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(debug="--debug" in sys.argv))
