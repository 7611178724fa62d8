"""Build libnsa_hip.so (gfx950) from ../csrc with hipcc.

Every translation unit is compiled separately (in parallel) into ../_build and then
linked into a shared library next to this file, where the ctypes loader finds it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
LIB = PKG_DIR / "libnsa_hip.so"
ARCH = os.environ.get("NSA_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 VALU forms are disabled for every HIP unit (hipcc would otherwise
# generate them from ordinary float code).
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wno-unused-result",
]
# Units whose floating-point results must match the CPU restatement bit for bit:
# no contraction of a*b+c into fma beyond the explicit fmaf() calls.
STRICT_FP = {"nsa_score.hip"}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libnsa_hip.so)")


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    flags = list(COMMON)
    if src.name in STRICT_FP:
        flags += ["-ffp-contract=off"]
    cmd = [_hipcc(), *flags, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip unit and link libnsa_hip.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} units", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
