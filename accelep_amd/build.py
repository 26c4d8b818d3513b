"""Builds the in-tree libraries for gfx950 and the C++ test programs.

* accelep_amd/libaccel_hip.so: the C-ABI (include/accel_hip.h). Kernel files (csrc/*.hip)
  are compiled by hipcc for gfx950 only, host files (csrc/*.cc) by g++ against the HIP
  runtime headers; linked against libamdhip64 with -z defs.
* accelep_amd/libaccel_runtime.so: the C++ accel:: device and runtime (include/accel/*.h,
  host/*.cc) over the C-ABI.
* tests/cpp/bin/*: the C++ tests (tests/cpp/*.cc), linked against both, and
  libbpe_host.so (tests/cpp/lib/bpe_host.cc over csrc/tokenizer.cc, no HIP) for the CPU
  tokenizer tests.

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
HOST = PKG / "host"
RUNTIME_LIB = PKG / "libaccel_runtime.so"
CPP_TESTS = ROOT / "tests" / "cpp"
CPP_TEST_BIN = CPP_TESTS / "bin"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    # Packed fp32 (v_pk_*_f32) stays off: the compiler may only emit scalar fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel arguments preloaded into SGPRs at wave launch (gfx950 kernarg preload): a wave
    # issues its first global loads without a scalar-load round trip to the kernarg segment.
    # Kernels also keep a prologue that loads them, for firmware without preload.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-result", "-fvisibility=hidden",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
GXX_FLAGS = [
    "-O2", "-fPIC", "-std=c++17", "-Wall", "-Wextra", "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__",
    f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}", f"-I{CSRC}",
]


HOST_FLAGS = ["-O2", "-fPIC", "-std=c++20", "-ffp-contract=off", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}"]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = ("is not a recognized feature for this target",)
    lines = [ln for ln in proc.stdout.splitlines() if not any(n in ln for n in noise)]
    if proc.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(map(str, cmd)) + "\n" + "\n".join(lines))
    return "\n".join(lines)


def _compile(src: Path) -> Path:
    if src.parent == HOST:
        obj = BUILD / ("host_" + src.name + ".o")
        cmd = ["g++", *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    elif src.suffix == ".hip":
        obj = BUILD / (src.name + ".o")
        cmd = [str(ROCM / "bin" / "hipcc"), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        obj = BUILD / (src.name + ".o")
        cmd = ["g++", *GXX_FLAGS, "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def _link_runtime(objs) -> Path:
    tmp = RUNTIME_LIB.with_suffix(".so.tmp")
    _run(["g++", "-shared", "-Wl,-z,defs", "-o", str(tmp), *map(str, objs), f"-L{PKG}", "-laccel_hip",
          "-Wl,-rpath,$ORIGIN"])
    tmp.replace(RUNTIME_LIB)
    return RUNTIME_LIB


def _build_cpp_test(src: Path) -> Path:
    CPP_TEST_BIN.mkdir(exist_ok=True)
    exe = CPP_TEST_BIN / src.stem
    _run(["g++", *HOST_FLAGS, "-o", str(exe), str(src), f"-L{PKG}", "-laccel_runtime", "-laccel_hip",
          "-Wl,-rpath,$ORIGIN/../../../accelep_amd"])
    return exe


def _build_bpe_host() -> Path:
    CPP_TEST_BIN.mkdir(exist_ok=True)
    out = CPP_TEST_BIN / "libbpe_host.so"
    _run(["g++", *HOST_FLAGS, "-shared", "-fvisibility=hidden", f"-I{CSRC}", "-o", str(out),
          str(CPP_TESTS / "lib" / "bpe_host.cc"), str(CSRC / "tokenizer.cc")])
    return out


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the library. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cc"))
    host_sources = sorted(HOST.glob("*.cc"))
    jobs = min(len(sources) + len(host_sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(_compile, sources))
        host_objs = list(pool.map(_compile, host_sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([str(ROCM / "bin" / "hipcc"), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", str(tmp),
          *map(str, objs), f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"])
    tmp.replace(LIB)
    _link_runtime(host_objs)
    tests = sorted(CPP_TESTS.glob("*.cc"))
    with ThreadPoolExecutor(max_workers=max(1, min(len(tests), jobs))) as pool:
        list(pool.map(_build_cpp_test, tests))
    _build_bpe_host()
    if verbose:
        print(f"built {LIB}, {RUNTIME_LIB} and {len(tests)} C++ test programs")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
