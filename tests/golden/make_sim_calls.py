"""Writes tests/golden/sim_calls.json: the compiled reference's standalone calls
(accel_sim_create / upload / matmul / release and the stats, AccelEP src/sim_api.cc:32-115
through oracle/_ref/libaccel_ref.so) on small matrices.

    make -C oracle && python3 tests/golden/make_sim_calls.py

Each case resets the stats, uploads B, multiplies and releases, and keeps the status, the
error text, C and the counters (kernel matmuls, bytes to the device and to the host).
"""

from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from oracle_ctypes import REF_SO  # noqa: E402

F32P = C.POINTER(C.c_float)


def bind():
    if not REF_SO.exists():
        raise SystemExit("oracle/_ref/libaccel_ref.so is missing: run `make -C oracle` with the reference tree present")
    L = C.CDLL(str(REF_SO))
    L.accel_sim_create.restype = C.c_void_p
    L.accel_sim_destroy.argtypes = [C.c_void_p]
    L.accel_sim_upload.restype = C.c_void_p
    L.accel_sim_upload.argtypes = [C.c_void_p, F32P, C.c_int64]
    L.accel_sim_release.argtypes = [C.c_void_p, C.c_void_p]
    L.accel_sim_matmul.restype = C.c_int
    L.accel_sim_matmul.argtypes = [C.c_void_p, F32P, C.c_int64, C.c_int64, C.c_void_p, C.c_int64, F32P]
    for name in ("accel_sim_matmuls", "accel_sim_bytes_to_device", "accel_sim_bytes_to_host"):
        getattr(L, name).restype = C.c_int64
    L.accel_sim_last_error.restype = C.c_char_p
    return L


def run(L, sim, a, b, m, k, n, upload_count=None):
    """One case: reset, upload b (upload_count floats of it), matmul, release."""
    L.accel_sim_reset_stats()
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    count = b.size if upload_count is None else upload_count
    buf = L.accel_sim_upload(sim, b.ctypes.data_as(F32P), count)
    assert buf, L.accel_sim_last_error()
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    c = np.full(max(m * n, 1), 7.0, np.float32)
    rc = L.accel_sim_matmul(sim, a.ctypes.data_as(F32P) if a.size else None, m, k, C.c_void_p(buf), n,
                            c.ctypes.data_as(F32P))
    err = L.accel_sim_last_error().decode()
    L.accel_sim_release(sim, C.c_void_p(buf))
    return dict(rc=rc, error=err, c=c[: m * n].tolist() if rc == 0 else None,
                counters=dict(matmuls=L.accel_sim_matmuls(), bytes_to_device=L.accel_sim_bytes_to_device(),
                              bytes_to_host=L.accel_sim_bytes_to_host()))


def main():
    L = bind()
    sim = L.accel_sim_create()
    assert sim
    sim = C.c_void_p(sim)
    r = np.random.default_rng(20261202)
    cases = []

    def add(name, a, b, m, k, n, exact, upload_count=None):
        out = run(L, sim, a, b, m, k, n, upload_count)
        cases.append(dict(name=name, a=np.asarray(a, np.float32).reshape(-1).tolist(),
                          b=np.asarray(b, np.float32).reshape(-1).tolist(), m=m, k=k, n=n, exact=exact,
                          upload_count=upload_count, **out))

    # AccelEP tests/test_serve.py:239-251.
    add("serve_test", np.arange(6).reshape(2, 3), np.arange(12).reshape(3, 4), 2, 3, 4, True)
    add("integers", r.integers(-8, 9, (5, 7)), r.integers(-8, 9, (7, 3)), 5, 7, 3, True)
    add("normal", r.standard_normal((33, 100)), r.standard_normal((100, 17)), 33, 100, 17, False)
    add("row", r.standard_normal((1, 64)), r.standard_normal((64, 130)), 1, 64, 130, False)
    add("k_zero", np.zeros(0), np.zeros(0), 3, 0, 4, True)
    add("m_zero", np.zeros(0), r.standard_normal((5, 2)), 0, 5, 2, True)
    add("b_too_small", r.standard_normal((2, 3)), r.standard_normal((3, 4)), 2, 3, 4, True, upload_count=11)
    # Invalid arguments, checked before any device work.
    L.accel_sim_reset_stats()
    invalid = dict(
        matmul_no_b=(L.accel_sim_matmul(sim, None, 1, 1, None, 1, None), L.accel_sim_last_error().decode()),
        matmul_negative=(L.accel_sim_matmul(sim, None, -1, 1, C.c_void_p(1), 1, None),
                         L.accel_sim_last_error().decode()),
        upload_negative=(L.accel_sim_upload(sim, None, -1) or 0, L.accel_sim_last_error().decode()),
        upload_no_data=(L.accel_sim_upload(sim, None, 3) or 0, L.accel_sim_last_error().decode()),
    )
    L.accel_sim_destroy(sim)
    out = dict(cases=cases, invalid={k: dict(rc=v[0], error=v[1]) for k, v in invalid.items()})
    (HERE / "sim_calls.json").write_text(json.dumps(out, indent=1) + "\n", encoding="utf-8")
    for c in cases:
        print(c["name"], c["rc"], c["error"], c["counters"])
    print(out["invalid"])


if __name__ == "__main__":
    main()
