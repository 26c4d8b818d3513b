"""Helpers for the GPU parity tests: device round trips through the C-ABI and the
tolerances the comparisons use."""

from __future__ import annotations

import ctypes as C

import numpy as np

from accelep_amd.capi import Buffer, Epilogue, HipError, QuantPlane, Stats, check, lib
from accelep_amd.device import DeviceArray, quant_plane

U = 2.0 ** -24


def gamma(k: int) -> float:
    """gamma_K of Higham's inner-product bound (any summation order)."""
    return k * U / (1 - k * U)


def assert_gamma_bound(got, a, w, extra_rel=0.0):
    """|got - A@W| <= 2 gamma_K (|A| @ |W|) elementwise, A@W exact in float64.

    The factor 2 covers the reference's own rounding of the dequantized weight and a
    per-column scale applied after the sum; `extra_rel` widens for a trailing epilogue."""
    a64 = np.asarray(a, np.float64)
    w64 = np.asarray(w, np.float64)
    exact = a64 @ w64
    mag = np.abs(a64) @ np.abs(w64)
    k = a64.shape[1]
    bound = 2 * gamma(max(k, 1)) * mag + extra_rel * np.abs(exact) + 1e-30
    err = np.abs(np.asarray(got, np.float64) - exact)
    bad = err > bound
    assert not bad.any(), (f"{bad.sum()} elements exceed 2*gamma_K*(|A||W|); worst ratio "
                           f"{float(np.max(err / bound)):.3g} at {np.unravel_index(np.argmax(err / bound), err.shape)}")
    return float(err.max()), float(np.max(err / bound))


def assert_plugin_tolerance(got, a, w, rtol=1e-5, atol=1e-5):
    """allclose(got, A@W, rtol, atol) against the float64 product: the plugin tests' tolerance
    (AccelEP tests/test_ep.py:98-100) for fp32 products with K <= 1024. Returns the worst
    |got - A@W| / (atol + rtol |A@W|)."""
    exact = np.asarray(a, np.float64) @ np.asarray(w, np.float64)
    got = np.asarray(got, np.float64)
    ratio = np.abs(got - exact) / (atol + rtol * np.abs(exact))
    bad = ratio > 1
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements beyond rtol={rtol}, atol={atol} of the float64 "
                           f"product; worst ratio {float(ratio.max()):.3g} at {np.unravel_index(np.argmax(ratio), ratio.shape)}")
    return float(ratio.max())


def same_bits(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    both_nan = np.isnan(got) & np.isnan(want)
    diff = (got.view(np.uint32) != want.view(np.uint32)) & ~both_nan
    assert not diff.any(), f"{diff.sum()} elements differ; first at {np.argwhere(diff)[0]}"


def dev(host, dtype=None) -> DeviceArray:
    host = np.ascontiguousarray(host if dtype is None else np.asarray(host, dtype))
    return DeviceArray.from_numpy(host)


def stats() -> Stats:
    s = Stats()
    lib().accel_hip_get_stats(C.byref(s))
    return s


def plane_from_spec(spec):
    """Uploads a quant spec of golden_cases and returns (plane, keepalive)."""
    q = dev(spec["q"])
    s = dev(spec["scale"])
    z = dev(spec["zero"]) if spec["zero"] is not None else None
    return quant_plane(q, s, z, spec["shape"], spec["axis"], spec["offset"]), (q, s, z)


def matmul_quantized(case, fused: Epilogue | None = None):
    """Runs accel_hip_matmul_quantized(_fused) on a golden_cases quant case; returns C."""
    m, k, n = case["m"], case["k"], case["n"]
    keep = []
    aq = bq = None
    a_ptr = b_ptr = None
    if case.get("aq") is not None:
        aq, kk = plane_from_spec(case["aq"])
        keep.append(kk)
    else:
        a_d = dev(case["a"], np.float32)
        keep.append(a_d)
        a_ptr = a_d.ptr
    if case.get("bq") is not None:
        bq, kk = plane_from_spec(case["bq"])
        keep.append(kk)
    else:
        b_d = dev(case["b"], np.float32)
        keep.append(b_d)
        b_ptr = b_d.ptr
    c = dev(np.full((m, n), 3.0, np.float32))
    L = lib()
    if fused is None:
        check(L.accel_hip_matmul_quantized(a_ptr, C.byref(aq) if aq else None, b_ptr, C.byref(bq) if bq else None,
                                           c.ptr, m, k, n))
    else:
        check(L.accel_hip_matmul_quantized_fused(a_ptr, C.byref(aq) if aq else None, b_ptr,
                                                 C.byref(bq) if bq else None, c.ptr, m, k, n, C.byref(fused)))
    return c.numpy()


def dequant_host(spec, rows, cols):
    """fl((q - z) * s) of the [rows, cols] matrix at spec['offset'] (numpy float32)."""
    q = np.asarray(spec["q"], np.int8)
    shape = list(spec["shape"])
    axis = spec["axis"]
    off = spec["offset"]
    if len(shape) == 2 and off == 0 and axis in (0, 1):
        qf = q[: rows * cols].reshape(rows, cols).astype(np.float32)
        scale = np.asarray(spec["scale"], np.float32)
        zero = spec["zero"]
        if axis == 1:
            z = np.zeros(cols, np.float32) if zero is None else np.asarray(zero, np.float32)
            return ((qf - z[None, :]).astype(np.float32) * scale[None, :]).astype(np.float32)
        z = np.zeros(rows, np.float32) if zero is None else np.asarray(zero, np.float32)
        return ((qf - z[:, None]).astype(np.float32) * scale[:, None]).astype(np.float32)
    idx = off + np.arange(rows * cols, dtype=np.int64)
    scale = np.asarray(spec["scale"], np.float32)
    zero = spec["zero"]
    if axis < 0:
        s = np.full(idx.shape, scale[0], np.float32)
        z = np.full(idx.shape, 0 if zero is None else zero[0], np.float32)
    else:
        stride = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
        coord = (idx // stride) % shape[axis]
        s = scale[coord]
        z = np.zeros(idx.shape, np.float32) if zero is None else np.asarray(zero, np.float32)[coord]
    w = ((q[idx].astype(np.float32) - z).astype(np.float32) * s).astype(np.float32)
    return w.reshape(rows, cols)


__all__ = ["Buffer", "Epilogue", "HipError", "QuantPlane", "DeviceArray", "assert_gamma_bound", "assert_plugin_tolerance",
           "check", "dev",
           "dequant_host", "gamma", "lib", "matmul_quantized", "plane_from_spec", "quant_plane", "same_bits", "stats"]
