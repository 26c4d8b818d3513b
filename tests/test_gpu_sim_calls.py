"""The standalone calls of include/accel_sim.h (accel_sim_create / upload / matmul / release and
the stats) on the GPU, against the compiled reference's results on the same inputs
(tests/golden/sim_calls.json, AccelEP src/sim_api.cc:32-115 through oracle/_ref).

* status and error text equal the reference's, including a B smaller than k x n;
* C is bit-exact where every partial sum is an integer (the reference's own serve test,
  tests/test_serve.py:239-251, and small integers); for N(0,1) data it is within the γ_K
  bound of the product, the fp32 GEMM's tolerance elsewhere in these tests;
* kernel matmuls and the bytes to and from the device equal the reference's counters;
* the invalid-argument checks give the reference's messages.
"""

from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

from accelep_amd.capi import F32P, lib

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "sim_calls.json"


def _golden():
    return json.loads(GOLDEN.read_text())


def _gamma(k):
    u = 2.0 ** -24
    return k * u / (1 - k * u)


@pytest.fixture(scope="module")
def sim():
    L = lib()
    h = L.accel_sim_create()
    assert h, L.accel_sim_last_error()
    yield L, C.c_void_p(h)
    L.accel_sim_destroy(C.c_void_p(h))


@pytest.mark.parametrize("name", [c["name"] for c in json.loads(GOLDEN.read_text())["cases"]])
def test_matmul_matches_the_reference(sim, name):
    L, h = sim
    case = next(c for c in _golden()["cases"] if c["name"] == name)
    m, k, n = case["m"], case["k"], case["n"]
    print(f"sim matmul {name}: {m}x{k}x{n}", flush=True)
    a = np.asarray(case["a"], np.float32)
    b = np.asarray(case["b"], np.float32)
    L.accel_sim_reset_stats()
    count = b.size if case["upload_count"] is None else case["upload_count"]
    buf = L.accel_sim_upload(h, b.ctypes.data_as(F32P), count)
    assert buf, L.accel_sim_last_error()
    c = np.full(max(m * n, 1), 7.0, np.float32)
    rc = L.accel_sim_matmul(h, a.ctypes.data_as(F32P) if a.size else None, m, k, C.c_void_p(buf), n,
                            c.ctypes.data_as(F32P))
    err = L.accel_sim_last_error().decode()
    L.accel_sim_release(h, C.c_void_p(buf))
    counters = dict(matmuls=L.accel_sim_matmuls(), bytes_to_device=L.accel_sim_bytes_to_device(),
                    bytes_to_host=L.accel_sim_bytes_to_host())
    assert (rc, err) == (case["rc"], case["error"])
    assert counters == case["counters"]
    if rc != 0:
        return
    got = c[: m * n]
    want = np.asarray(case["c"], np.float32)
    if case["exact"]:
        np.testing.assert_array_equal(got, want)
    else:
        a2 = a.reshape(m, k).astype(np.float64)
        b2 = b.reshape(k, n).astype(np.float64)
        exact = (a2 @ b2).reshape(-1)
        bound = 2 * _gamma(k) * (np.abs(a2) @ np.abs(b2)).reshape(-1)
        assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)
        assert np.all(np.abs(want.astype(np.float64) - exact) <= bound)  # the reference meets it too


def test_invalid_arguments_match_the_reference(sim):
    L, h = sim
    inv = _golden()["invalid"]
    assert (L.accel_sim_matmul(h, None, 1, 1, None, 1, None), L.accel_sim_last_error().decode()) == \
        (inv["matmul_no_b"]["rc"], inv["matmul_no_b"]["error"])
    assert (L.accel_sim_matmul(h, None, -1, 1, C.c_void_p(1), 1, None), L.accel_sim_last_error().decode()) == \
        (inv["matmul_negative"]["rc"], inv["matmul_negative"]["error"])
    assert (L.accel_sim_upload(h, None, -1) or 0, L.accel_sim_last_error().decode()) == \
        (inv["upload_negative"]["rc"], inv["upload_negative"]["error"])
    assert (L.accel_sim_upload(h, None, 3) or 0, L.accel_sim_last_error().decode()) == \
        (inv["upload_no_data"]["rc"], inv["upload_no_data"]["error"])
    L.accel_sim_release(h, None)  # no-op, as in the reference
    L.accel_sim_release(None, None)


def test_uploads_are_counted_and_released(sim):
    L, h = sim
    L.accel_hip_live_allocs.restype = C.c_int64
    before = L.accel_hip_live_allocs()
    L.accel_sim_reset_stats()
    data = np.arange(1000, dtype=np.float32)
    buf = L.accel_sim_upload(h, data.ctypes.data_as(F32P), data.size)
    assert buf and L.accel_sim_bytes_to_device() == 4000 and L.accel_sim_bytes_to_host() == 0
    empty = L.accel_sim_upload(h, None, 0)
    assert empty, L.accel_sim_last_error()
    L.accel_sim_release(h, C.c_void_p(buf))
    L.accel_sim_release(h, C.c_void_p(empty))
    assert L.accel_hip_live_allocs() == before
