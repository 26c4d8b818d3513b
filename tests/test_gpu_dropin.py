"""AccelEP's own runtime (src/runtime.cc, compiled from the reference tree by oracle/Makefile)
driving the MI355X device: the program oracle/_ref/ref_runtime_hip (source
tests/cpp/ref/ref_runtime_hip.cc) runs the plugin's operand binding and RunKernel step
sequences (plain, has_rms, has_skip; src/ep.cc:1430-1463,1602-1650) through ExecuteMatMul,
ExecuteGemm, ExecuteFusedMatMul, RmsNorm and ResidualAdd on CreateHipDevice(): the
dequantize KAT Y[0,0] = -48.5 (tests/test_ep.py:336-370) with its counters, the residual's
orientation, exact step values, the transpose error of a packed weight, live allocations, and
the decode GEMV shape within the gamma_K bound."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent.parent / "oracle" / "_ref" / "ref_runtime_hip"


def test_reference_runtime_over_hip_device():
    if not EXE.exists():
        pytest.skip(f"{EXE} is built from the reference sources (make -C oracle dropin), absent here")
    print(f"running {EXE}", flush=True)
    proc = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "0 failures" in proc.stdout
