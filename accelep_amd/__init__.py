"""accelep_amd: an MI355X (gfx950) backend for AccelEP's device seam.

The product is libaccel_hip.so (accelep_amd/csrc, built in-tree by accelep_amd.build):
hand-written HIP kernels behind the C-ABI of include/accel_hip.h, the C++ accel::Device
implementation and runtime of include/accel/*.h, and the accel_llama_* C API. This
package only binds it (ctypes) for tests and benchmarks.
"""

from .capi import HipError, lib  # noqa: F401
