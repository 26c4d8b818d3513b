"""AccelEP's own device-call recorder (tests/recording_device.cc of the reference, compiled by
oracle/Makefile) records the reference runtime's Execute* steps and a small Llama generation
(the reference's own llama_model.cc) on SimDevice; the program oracle/_ref/ref_trace_replay_hip
(source tests/cpp/ref/ref_trace_replay_hip.cc) replays every recorded call on the MI355X device
with exact products on and compares each call's output with the recorder's FNV-1a hash:
bit for bit for MatMul, Transpose, the Relu/none epilogues, Embedding, Rope, AppendCache,
ResidualAdd and SampleToken; within stated tolerances for the Gelu epilogue, SiluMul, Attention
and RmsNorm (device erf/exp, a reordered double sum)."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent.parent / "oracle" / "_ref" / "ref_trace_replay_hip"


def test_reference_trace_replays_on_hip_device():
    if not EXE.exists():
        pytest.skip(f"{EXE} is built from the reference sources (make -C oracle dropin), absent here")
    print(f"running {EXE}", flush=True)
    proc = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert " 0 failures" in proc.stdout
