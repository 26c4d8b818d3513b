"""The C++ runtime over the HIP device (accel::CreateHipDevice + Execute*), run as the
compiled test program tests/cpp/bin/test_runtime_hip (source: tests/cpp/test_runtime_hip.cc).
It restates AccelEP tests/test_runtime.cc's checks on the GPU and checks that the fused
epilogue store matches the reference's pass sequence bit for bit."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "bin"


@pytest.mark.parametrize("program", ["test_runtime_hip"])
def test_cpp_program(program):
    exe = BIN / program
    if not exe.exists():
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    print(f"running {exe}", flush=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stderr[-4000:]
