"""Host-side handles for device memory held through the C-ABI heap (accel_hip_allocate).

`DeviceArray` owns one allocation, like accel::OwnedBuffer (include/accel/device.h:35-65):
it frees on `free()` or garbage collection. Copies are the counted Device copies.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from .capi import Buffer, QuantPlane, check, lib


class DeviceArray:
    def __init__(self, shape, dtype=np.float32, nbytes=None):
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        count = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = int(nbytes) if nbytes is not None else count * self.dtype.itemsize
        self.buffer = Buffer()
        check(lib().accel_hip_allocate(self.nbytes, C.byref(self.buffer)))
        self._live = True

    @classmethod
    def from_numpy(cls, host) -> "DeviceArray":
        host = np.ascontiguousarray(host)
        arr = cls(host.shape, host.dtype)
        arr.upload(host)
        return arr

    @property
    def ptr(self) -> int:
        return int(self.buffer.data)

    def at(self, elements: int) -> int:
        """Device address of element `elements` (a slice pointer, id 0)."""
        return self.ptr + int(elements) * self.dtype.itemsize

    def upload(self, host):
        host = np.ascontiguousarray(host, dtype=self.dtype)
        if host.nbytes:
            check(lib().accel_hip_copy_h2d(self.buffer, host.ctypes.data, host.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if out.nbytes:
            check(lib().accel_hip_copy_d2h(out.ctypes.data, self.buffer, out.nbytes))
        return out

    def peek(self) -> np.ndarray:
        """Uncounted read (the reference reads device memory through raw pointers)."""
        out = np.empty(self.shape, self.dtype)
        if out.nbytes:
            check(lib().accel_hip_peek(out.ctypes.data, C.c_void_p(self.ptr), out.nbytes))
        return out

    def free(self):
        if self._live:
            self._live = False
            check(lib().accel_hip_free(self.buffer))

    def __del__(self):
        try:
            if self._live:
                self._live = False
                lib().accel_hip_free(self.buffer)
        except Exception:
            pass


def quant_plane(q: DeviceArray, scale: DeviceArray, zero: DeviceArray | None, shape, axis, offset=0) -> QuantPlane:
    plane = QuantPlane()
    plane.q = q.ptr
    plane.scale = scale.ptr
    plane.zero = zero.ptr if zero is not None else None
    plane.rank = len(shape)
    for i, d in enumerate(shape):
        plane.shape[i] = int(d)
    plane.axis = int(axis)
    plane.offset = int(offset)
    return plane


def synchronize():
    check(lib().accel_hip_synchronize())
