"""The drop-in boundary, on the CPU: the C-ABI library loads and exports every entry point
include/accel_hip.h declares, the Python mirror binds each of them, and the C++ runtime
library exports the accel:: API of include/accel/{device,runtime,hip_device}.h. No call
here touches a GPU."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "accel_hip.h"
LLAMA_HEADER = ROOT / "include" / "accel_llama.h"
SIM_HEADER = ROOT / "include" / "accel_sim.h"
LIB = ROOT / "accelep_amd" / "libaccel_hip.so"
RUNTIME_LIB = ROOT / "accelep_amd" / "libaccel_runtime.so"


def declared_entry_points():
    text = HEADER.read_text()
    names = re.findall(r"ACCEL_HIP_API\s+[\w\s\*]+?\b(accel_hip_\w+)\s*\(", text)
    assert len(names) == len(set(names))
    return names


def test_header_declares_the_seam():
    names = set(declared_entry_points())
    # One entry point per accel::Device virtual, plus MatMulQuantized, the heap, stats and probes.
    for want in ["allocate", "free", "copy_h2d", "copy_d2h", "matmul", "matmul_quantized", "transpose",
                 "gemm_epilogue", "embedding", "rms_norm", "rope", "append_cache", "attention", "silu_mul",
                 "residual_add", "sample_token", "live_allocs", "get_stats", "reset_stats",
                 "packed_matmul_calls", "packed_k_trips", "reset_packed_probes", "last_error"]:
        assert f"accel_hip_{want}" in names


def test_library_exports_every_declared_symbol():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_entry_points() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_mirror_binds_every_symbol():
    from accelep_amd.capi import SIGNATURES

    assert set(declared_entry_points()) == set(SIGNATURES)


def declared_llama_entry_points():
    return re.findall(r"ACCEL_LLAMA_API\s+[\w\s\*]+?\b(accel_llama_\w+)\s*\(", LLAMA_HEADER.read_text())


def declared_sim_entry_points():
    return re.findall(r"ACCEL_SIM_API\s+[\w\s\*]+?\b(accel_sim_\w+)\s*\(", SIM_HEADER.read_text())


def test_library_exports_nothing_else():
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert exported == set(declared_entry_points()) | set(declared_llama_entry_points()) | set(
        declared_sim_entry_points())


def test_llama_api_mirrors_the_reference_names():
    from accelep_amd.capi import LLAMA_SIGNATURES

    names = set(declared_llama_entry_points())
    assert names == set(LLAMA_SIGNATURES)
    for want in ["create", "destroy", "weight", "tokenizer", "generate", "encode", "decode", "complete",
                 "complete_stream", "forward_ids", "logit_max_abs", "reset", "last_error"]:
        assert f"accel_llama_{want}" in names


def test_sim_api_mirrors_the_reference_names():
    """The standalone calls of include/accel/sim_api.h:16-37, which serve/sim.py and
    serve/llama.py bind."""
    from accelep_amd.capi import SIM_SIGNATURES

    names = set(declared_sim_entry_points())
    assert names == set(SIM_SIGNATURES)
    assert names == {f"accel_sim_{n}" for n in ["create", "destroy", "upload", "release", "matmul", "reset_stats",
                                                 "matmuls", "bytes_to_device", "bytes_to_host", "last_error"]}


CPP_API = [
    "accel::CreateHipDevice()", "accel::LiveDeviceAllocs()", "accel::PackedMatMulCalls()", "accel::PackedKTrips()",
    "accel::ResetPackedGemmProbes()", "accel::MatMulQuantized(", "accel::ExecuteMatMul(", "accel::ExecuteFusedMatMul(",
    "accel::ExecuteGemm(", "accel::Upload(", "accel::PretransposeLastTwo(", "accel::InferMatMulShape(",
    "accel::InferFusedMatMulShape(", "accel::InferGemmShape(", "accel::ElementCount(", "accel::GetAcceleratorStats()",
    "accel::ResetAcceleratorStats()", "accel::NoteConstantTouch(", "accel::ConstantTouchCount()",
    "accel::AppendProfileRecord(", "accel::WriteProfile(", "accel::KvTableStore::Create(", "accel::OwnedBuffer::Reset()",
    "accel::ActivationName(", "accel::HipMatMulFused(", "accel::HipMatMulQuantizedFused(", "accel::IsHipDevice(",
    "accel::HipPrepareQuantized(",
]


def test_runtime_library_exports_the_cpp_api():
    if not RUNTIME_LIB.exists():
        pytest.fail(f"{RUNTIME_LIB} is not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-DC", "--defined-only", str(RUNTIME_LIB)], capture_output=True, text=True,
                         check=True).stdout
    missing = [sym for sym in CPP_API if sym not in out]
    assert not missing, missing
