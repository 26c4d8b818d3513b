"""Builds accelep_amd/libaccel_hip.so in-tree for gfx950.

Kernel files (csrc/*.hip) are compiled by hipcc for gfx950 only; host files (csrc/*.cc) by
g++ against the HIP runtime headers; the shared object links libamdhip64 with -z defs.

    python -m accelep_amd.build          # or: python accelep_amd/build.py
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libaccel_hip.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    # Packed fp32 (v_pk_*_f32) stays off: the compiler may only emit scalar fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-fvisibility=hidden",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
GXX_FLAGS = [
    "-O2", "-fPIC", "-std=c++17", "-Wall", "-Wextra", "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__",
    f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = ("is not a recognized feature for this target",)
    lines = [ln for ln in proc.stdout.splitlines() if not any(n in ln for n in noise)]
    if proc.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(map(str, cmd)) + "\n" + "\n".join(lines))
    return "\n".join(lines)


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [str(ROCM / "bin" / "hipcc"), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["g++", *GXX_FLAGS, "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the library. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cc"))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([str(ROCM / "bin" / "hipcc"), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", str(tmp),
          *map(str, objs), f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"])
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
