"""Build libifx_fp8.so (gfx950) in-tree with hipcc.

    python -m instinctflash_amd.build          # compile and report

The library is plain HIP C++ behind the C ABI of include/ifx_fp8.h; no torch
headers are involved, so the build is a single hipcc invocation.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libifx_fp8.so"
OBJ = PKG / "_build"
SOURCES = ("quant.hip", "gemm.hip", "norm.hip", "rope.hip", "attention.hip", "clock.hip")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # IEEE round-to-nearest FP32 division is part of the quantization recipe.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # Keep FP32 denormals (bf16 subnormal inputs must quantize exactly).
    "-fno-gpu-flush-denormals-to-zero",
    # Packed-FP32 VALU forms are disabled on this platform.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    # the DMA helper's inline asm sets M0 (a reserved register) on purpose
    "-Wno-inline-asm",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile each source to an object (in parallel), then link the library."""
    OBJ.mkdir(exist_ok=True)
    objs = [OBJ / (Path(s).stem + ".o") for s in SOURCES]
    cc = hipcc()
    cmds = [[cc, *FLAGS, f"-I{ROOT / 'include'}", "-c", str(CSRC / s), "-o", str(o)] for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose=True)
    print(f"built {path}", file=sys.stderr)
