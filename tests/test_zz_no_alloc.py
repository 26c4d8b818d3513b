"""accel_hip_matmul_quantized_fused_noalloc (include/accel_hip.h) against
accel_hip_matmul_quantized_fused, through the C-ABI: the same bits on the same inputs, for
the kernels that use scratch (the split-bf16 GEMV with its arrival counters, the split-K
GEMV and GEMM with their partial sums, a plane layout dequantized into a temporary) and for
the m = 1 GEMV, each on two calls in a row with the second smaller than the first. The
no-allocation call runs first on a fresh weight (W read in place) and again after the
allocating call has staged W (the staged copy read); both must equal the allocating call's
result to the bit where the same kernel runs, and meet the gamma_K bound where W is read in
place by another kernel. A request larger than the fixed scratch is refused with
ACCEL_HIP_INVALID_ARGUMENT, and the live allocation count never moves."""

import ctypes as C

import numpy as np
import pytest

from hip_helpers import Epilogue, assert_gamma_bound, check, dequant_host, dev, lib, quant_plane, same_bits

pytestmark = pytest.mark.gpu

INVALID_ARGUMENT = 1


@pytest.fixture(scope="module", autouse=True)
def device():
    check(lib().accel_hip_init())
    yield


def _problem(m, k, n, seed, axis=1, zero=False):
    r = np.random.default_rng(seed)
    q = r.integers(-127, 128, size=k * n, dtype=np.int8)
    scale_len = n if axis == 1 else k
    s = r.uniform(1e-3, 1e-2, size=scale_len).astype(np.float32)
    z = r.integers(-3, 4, size=scale_len, dtype=np.int8) if zero else None
    a = r.standard_normal((m, k)).astype(np.float32)
    return dict(q=q, s=s, z=z, a=a, m=m, k=k, n=n, axis=axis)


def _run(p, noalloc, epi=None):
    L = lib()
    m, k, n = p["m"], p["k"], p["n"]
    p.setdefault("qd", dev(p["q"]))
    p.setdefault("sd", dev(p["s"]))
    if p["z"] is not None:
        p.setdefault("zd", dev(p["z"]))
    p.setdefault("ad", dev(p["a"]))
    plane = quant_plane(p["qd"], p["sd"], p.get("zd"), [k, n], p["axis"])
    out = dev(np.full((m, n), 3.0, np.float32))
    fn = L.accel_hip_matmul_quantized_fused_noalloc if noalloc else L.accel_hip_matmul_quantized_fused
    rc = fn(p["ad"].ptr, None, None, C.byref(plane), out.ptr, m, k, n, C.byref(epi) if epi is not None else None)
    return rc, out


# (m, k, n): split-bf16 GEMV (4 splits, arrival counters), split-K narrow GEMV (few tiles),
# m = 1 entry GEMV, bf16 GEMM with split K (small grid), bf16 GEMM from the activation image
# (staged bf16 weight), fp32-panel GEMM (per-row scale, zero points) with split K.
CASES = [
    ("split_bf16_gemv", (16, 4096, 2048), dict()),
    ("split_k_gemv", (2, 4096, 512), dict()),
    ("m1_gemv", (1, 2048, 4096), dict()),
    ("bf16_gemm_split", (100, 2048, 264), dict()),
    ("bf16_gemm_image", (512, 256, 8192), dict()),
    ("f32_gemm_zero_rowscale", (40, 1024, 96), dict(axis=0, zero=True)),
]


@pytest.mark.parametrize("name,shape,kw", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_allocating_entry(name, shape, kw):
    L = lib()
    m, k, n = shape
    big = _problem(m, k, n, 7 + m, **kw)
    small = _problem(max(1, m // 2), k // 2, n // 2, 9 + m, **kw)
    live0 = L.accel_hip_live_allocs()
    for p in (big, small):  # two calls in a row, the second smaller
        print(f"{name}: m={p['m']} k={p['k']} n={p['n']}", flush=True)
        w = dequant_host(dict(q=p["q"], scale=p["s"], zero=p["z"], shape=[p["k"], p["n"]], axis=p["axis"], offset=0),
                         p["k"], p["n"])
        # Fresh weight: nothing staged yet, the no-allocation call reads W in place.
        rc, first = _run(p, True)
        assert rc == 0, L.accel_hip_last_error()
        got_first = first.numpy()
        assert_gamma_bound(got_first, p["a"], w)
        rc, ref = _run(p, False)  # stages W where the GEMV wants a staged copy
        check(rc)
        want = ref.numpy()
        rc, again = _run(p, True)  # now reads the staged copy: the same kernel, the same bits
        assert rc == 0, L.accel_hip_last_error()
        same_bits(again.numpy(), want)
        for d in (first, ref, again):
            d.free()
    # Fused epilogue (bias, gelu, residual) on the split GEMV of the big problem.
    p = big
    r = np.random.default_rng(3)
    bias = dev(r.standard_normal(p["n"]).astype(np.float32))
    resid = dev(r.standard_normal((p["m"], p["n"])).astype(np.float32))
    e = Epilogue(alpha=1.25, beta=0.5, bias=bias.ptr, bias_rank=1, activation=2, residual=resid.ptr)
    e.bias_shape[0] = p["n"]
    rc, ref = _run(p, False, e)
    check(rc)
    rc, got = _run(p, True, e)
    assert rc == 0, L.accel_hip_last_error()
    same_bits(got.numpy(), ref.numpy())
    for d in (ref, got, bias, resid):
        d.free()
    assert L.accel_hip_live_allocs() == live0 + sum(1 for q in (big, small) for key in ("qd", "sd", "zd", "ad") if key in q)


def test_noalloc_refuses_scratch_beyond_its_size():
    """A plane layout the kernels do not index directly (a per-element offset pattern) is
    dequantized into scratch: 64 MiB holds at most 16 Mi floats, so a 4096 x 8192 weight
    (32 Mi floats) is refused with invalid_argument, and nothing is written."""
    L = lib()
    k, n = 4096, 8192
    q = np.zeros(k * n + 5, np.int8)
    s = np.ones(3, np.float32)
    qd, sd = dev(q), dev(s)
    a = dev(np.ones((1, k), np.float32))
    out = dev(np.full((1, n), 3.0, np.float32))
    plane = quant_plane(qd, sd, None, [3, (k * n + 5) // 3 + 1], 0, 5)  # scale index changes inside rows
    rc = L.accel_hip_matmul_quantized_fused_noalloc(a.ptr, None, None, C.byref(plane), out.ptr, 1, k, n, None)
    msg = L.accel_hip_last_error().decode()
    assert rc == INVALID_ARGUMENT, (rc, msg)
    assert "no-allocation scratch" in msg
    assert (out.numpy() == 3.0).all()
