"""The drop-in boundary, proven with the reference's own sources (CPU, no GPU call).

oracle/Makefile (`make -C oracle dropin`) builds AccelEP's plugin as a HIP build: the
reference's src/ep.cc with the device switched to CreateHipDevice (the two-line change of
INTEGRATION.md, applied at compile time), its src/runtime.cc and src/device_buffer.cc, and this
repository's accelep_amd/host/hip_device.cc, all against the reference's own include/ with
-Werror, linked -z defs against libaccel_hip.so into oracle/_ref/libaccel_ep_hip.so. This test
rebuilds it from the sources where they lie and checks that the result loads and exports the
plugin's ABI: CreateEpFactories, ReleaseEpFactory and the 18 AccelEp* counter/profile/touch
functions (src/ep.cc:1983-2024), that it resolves its device through libaccel_hip.so, and that
no simulator code (SimDevice, CreateSimDevice) is inside. Test infrastructure only: no product
code links the reference."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
PLUGIN = ROOT / "oracle" / "_ref" / "libaccel_ep_hip.so"
HIP_LIB = ROOT / "accelep_amd" / "libaccel_hip.so"

# src/ep.cc:1983-2024
EP_EXPORTS = [
    "CreateEpFactories", "ReleaseEpFactory", "AccelEpResetStats", "AccelEpMatmulOps", "AccelEpGemmOps",
    "AccelEpKernelMatmuls", "AccelEpReluEpilogues", "AccelEpGeluEpilogues", "AccelEpAddEpilogues",
    "AccelEpDeviceTransposes", "AccelEpBytesToDevice", "AccelEpBytesToHost", "AccelEpWriteProfile",
    "AccelEpIsStreamAware", "AccelEpLiveDeviceAllocs", "AccelEpClearConstantTouches", "AccelEpConstantTouchCount",
    "AccelEpConstantTouchId", "AccelEpConstantTouchAddress", "AccelEpConstantTouchBytes",
]


@pytest.fixture(scope="module")
def plugin():
    if not (REF / "src" / "ep.cc").exists():
        pytest.skip("the reference tree is not present (the plugin is built from its sources)")
    if not HIP_LIB.exists():
        pytest.fail(f"{HIP_LIB} is not built (run __graft_entry__.build())")
    proc = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "dropin"], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert PLUGIN.exists()
    return PLUGIN


def test_plugin_exports_the_ep_abi(plugin):
    out = subprocess.run(["nm", "-D", "--defined-only", str(plugin)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert len(EP_EXPORTS) == 20
    missing = [n for n in EP_EXPORTS if n not in exported]
    assert not missing, missing
    lib = ctypes.CDLL(str(plugin))
    for name in EP_EXPORTS:
        assert hasattr(lib, name), name
    lib.AccelEpIsStreamAware.restype = ctypes.c_int
    assert lib.AccelEpIsStreamAware() == 0  # not stream aware (src/ep.cc:100-102)


def test_plugin_runs_on_the_hip_device(plugin):
    needed = subprocess.run(["readelf", "-d", str(plugin)], capture_output=True, text=True, check=True).stdout
    assert "libaccel_hip.so" in needed
    syms = subprocess.run(["nm", "-C", str(plugin)], capture_output=True, text=True, check=True).stdout
    assert "accel::CreateHipDevice" in syms
    assert "SimDevice" not in syms and "CreateSimDevice" not in syms
    undefined = subprocess.run(["nm", "-D", "--undefined-only", str(plugin)], capture_output=True, text=True,
                               check=True).stdout
    assert "accel_hip_matmul_quantized" in undefined  # MatMulQuantized goes to the HIP library
    assert "accel_hip_allocate" in undefined
