"""Parity of the HIP kernels (through the C-ABI) with the compiled reference's outputs
(tests/golden/reference_outputs.npz) and the CPU oracle.

Tolerances:
  * integer/index work (ids, KV rows, gathers, greedy argmax, sampling): bit-exact;
  * elementwise steps with no transcendental (relu/none epilogues, rope, add, copies):
    bit-exact;
  * fp32 matmuls: every element within 2*gamma_K*(|A|@|W|) of the float64 product (Higham's
    inner-product bound, any summation order), and for K <= 1024 also within rtol = atol =
    1e-5 of the float64 product (allclose), the reference's plugin-test tolerance
    (tests/test_ep.py:98-100);
  * erf/exp-based steps (gelu, silu, attention softmax): within a few ulp (stated per test).
"""

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from golden_cases import (attention_cases, embed_cases, epilogue_cases, quant_cases, rmsnorm_cases, rope_cases,
                          sample_cases, silu_add_cases)
from hip_helpers import (Buffer, Epilogue, HipError, DeviceArray, assert_gamma_bound, assert_plugin_tolerance, check,
                         dev, dequant_host, lib, matmul_quantized, plane_from_spec, quant_plane, same_bits, stats)

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_outputs.npz"


@pytest.fixture(scope="module", autouse=True)
def device():
    check(lib().accel_hip_init())
    assert lib().accel_hip_device_arch().decode().startswith("gfx950")
    yield


def oracle():
    from oracle_ctypes import oracle as _o

    return _o()


# ---- heap and copies (src/sim_device.cc:133-183) -------------------------------------------

def test_heap_semantics():
    L = lib()
    before = L.accel_hip_live_allocs()
    a = Buffer()
    check(L.accel_hip_allocate(128, C.byref(a)))
    b = Buffer()
    check(L.accel_hip_allocate(0, C.byref(b)))
    assert a.data and b.data and b.bytes == 0 and b.id > a.id > 0
    assert L.accel_hip_live_allocs() == before + 2
    out = np.full(32, 7, np.float32)
    check(L.accel_hip_copy_d2h(out.ctypes.data, a, 128))
    assert not out.any()  # zero-filled
    with pytest.raises(HipError) as e:
        check(L.accel_hip_copy_d2h(out.ctypes.data, a, 256))
    assert e.value.kind == "invalid_argument"
    bogus = Buffer(a.data, a.bytes, a.id + 1000)
    with pytest.raises(HipError) as e:
        check(L.accel_hip_free(bogus))
    assert e.value.kind == "logic_error"
    check(L.accel_hip_free(Buffer(None, 0, 0)))  # null is a no-op
    check(L.accel_hip_free(a))
    check(L.accel_hip_free(b))
    assert L.accel_hip_live_allocs() == before
    c = Buffer()
    check(L.accel_hip_allocate(128, C.byref(c)))
    assert c.id > b.id  # ids are never reused
    # A reused block is zero again.
    check(L.accel_hip_copy_d2h(out.ctypes.data, c, 128))
    assert not out.any()
    check(L.accel_hip_free(c))


def test_copies_are_counted_and_private():
    L = lib()
    L.accel_hip_reset_stats()
    host = np.arange(4, dtype=np.float32)
    d = dev(host)
    host[0] = 99
    back = d.numpy()
    assert back.tolist() == [0, 1, 2, 3]
    s = stats()
    assert s.bytes_to_device == 16 and s.bytes_to_host == 16
    d.peek()
    assert stats().bytes_to_host == 16  # peek is not counted


# ---- matmul (src/sim_device.cc:185-196, 387-402) -------------------------------------------

def run_matmul(a, b):
    m, k = a.shape
    n = b.shape[1]
    A, B = dev(a, np.float32), dev(b, np.float32)
    Cd = dev(np.full((m, n), 5, np.float32))
    check(lib().accel_hip_matmul(A.buffer, B.buffer, Cd.buffer, m, k, n))
    return Cd.numpy()


def test_matmul_known_answer():
    assert run_matmul(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]])).tolist() == [[19, 22], [43, 50]]


def test_matmul_reference_fixtures(gold):
    for key in [k[:-2] for k in gold if k.startswith("matmul_") and k.endswith("_a")]:
        a, b = gold[key + "_a"], gold[key + "_b"]
        got = run_matmul(a, b)
        assert_gamma_bound(got, a, b)
        want = gold[key + "_device"]
        scale = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
        assert np.all(np.abs(got - want) <= 1e-5 * np.maximum(scale, 1.0))


@pytest.fixture
def exact_products():
    L = lib()
    check(L.accel_hip_set_exact_products(1))
    assert L.accel_hip_exact_products() == 1
    yield
    check(L.accel_hip_set_exact_products(0))


def test_exact_products_reproduce_reference_bits(gold, exact_products):
    """With exact products on, MatMul and MatMulQuantized store the compiled reference's
    bits (src/sim_device.cc:387-402,541-602) on every fixture, incl. the split-product KAT."""
    kat = run_matmul(np.array([[0xBE2694CD, 0x3E41AF7D]], np.uint32).view(np.float32),
                     np.array([[0x3F800000], [0x3F5C2CB8]], np.uint32).view(np.float32))
    assert kat.view(np.uint32)[0, 0] == 0xB5200000
    for key in [k[:-2] for k in gold if k.startswith("matmul_") and k.endswith("_a")]:
        same_bits(run_matmul(gold[key + "_a"], gold[key + "_b"]), gold[key + "_device"])
    for case in quant_cases():
        same_bits(matmul_quantized(case), gold[f"quant_{case['name']}_out"])


def test_matmul_probes_and_zero_k():
    L = lib()
    L.accel_hip_reset_packed_probes()
    L.accel_hip_reset_stats()
    run_matmul(np.ones((3, 7)), np.ones((7, 5)))
    assert L.accel_hip_packed_matmul_calls() == 1 and L.accel_hip_packed_k_trips() == 7
    assert stats().kernel_matmuls == 1
    A = dev(np.zeros(1, np.float32))
    B = dev(np.zeros(1, np.float32))
    Cd = dev(np.full((2, 3), 7, np.float32))
    check(L.accel_hip_matmul(A.buffer, B.buffer, Cd.buffer, 2, 0, 3))
    assert not Cd.numpy().any()  # k == 0 overwrites C with zeros
    with pytest.raises(HipError) as e:
        check(L.accel_hip_matmul(A.buffer, B.buffer, Cd.buffer, 2, 4, 3))
    assert e.value.kind == "invalid_argument" and "MatMul A is out of range" in e.value.message


@pytest.mark.parametrize("m,k,n", [(256, 1024, 4096), (256, 4096, 1024), (77, 300, 129), (1, 576, 49), (64, 64, 64),
                                   (128, 4096, 256), (64, 512, 64), (64, 2048, 192), (128, 1536, 128), (64, 1088, 704),
                                   (1024, 2048, 1024)])
def test_matmul_against_oracle(m, k, n):
    """fp32 GEMM. The 64 x 64 wave-split kernel on the bf16 matrix cores (each fp32 operand as
    three exact bf16 parts, six part products; 4 waves, each over a quarter of the workgroup's K)
    takes small full-tile grids: 8 groups of 32 k per wave unrolled (256 x 1024 x 4096; and, with
    K also split over workgroups and summed by SplitReduceKernel, 256 x 4096 x 1024 and
    128 x 4096 x 256 in 4 splits, 64 x 2048 x 192 in 2), and the looped form (64 x 512 x 64: 4
    groups; 128 x 1536 x 128: 12; 1024 x 2048 x 1024: 16). The LDS kernel on the fp32 matrix
    cores takes the rest (ragged shapes, K not a multiple of 256). Every element within 2 gamma_K
    of the float64 product, and within rtol = atol = 1e-5 of it for K <= 1024."""
    r = np.random.default_rng(m * 7 + k)
    a = r.standard_normal((m, k)).astype(np.float32)
    b = (r.standard_normal((k, n)) * 0.02).astype(np.float32)
    got = run_matmul(a, b)
    assert_gamma_bound(got, a, b)
    if k <= 1024:
        np.testing.assert_allclose(got, oracle().reference_matmul(a, b), rtol=1e-5, atol=1e-5)
        assert_plugin_tolerance(got, a, b)


# ---- MatMulQuantized (src/sim_device.cc:541-602) -------------------------------------------

# The int8 LCG fixtures of tests/test_runtime.cc:325-348 (weights up to 187, |C| up to 1e6): the
# reference's own bits are 12 and 21 times the plugin tolerance away from the float64 product
# there, as is numpy's float32 product, so those two are held to the gamma_K bound only.
LCG_FIXTURES = ("row_scale_zero", "scalar_scale")


def test_quantized_reference_fixtures(gold):
    for case in quant_cases():
        got = matmul_quantized(case)
        want = gold[f"quant_{case['name']}_out"]
        if case["k"] == 0:
            same_bits(got, want)
            continue
        if case.get("aq") is not None:
            a = dequant_host(case["aq"], case["m"], case["k"])
            w = case["b"]
        else:
            a = case["a"]
            w = dequant_host(case["bq"], case["k"], case["n"])
        assert_gamma_bound(got, a, w)
        if case["name"] not in LCG_FIXTURES:
            assert_plugin_tolerance(got, a, w)
        if case["name"] == "dq_kat":
            assert got[0, 0] == np.float32(-48.5)
        if case["name"].startswith("col_"):
            np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def c3_case(m, k, n, seed, zero=False, axis=1):
    r = np.random.default_rng(seed)
    q = r.integers(-127, 128, size=k * n, dtype=np.int8)
    cnt = n if axis == 1 else k
    scale = r.uniform(1e-3, 1e-2, size=cnt).astype(np.float32)
    z = r.integers(-3, 4, size=cnt, dtype=np.int8) if zero else None
    a = r.standard_normal((m, k)).astype(np.float32)
    return dict(name="c3", m=m, k=k, n=n, a=a, bq=dict(q=q, scale=scale, zero=z, shape=[k, n], axis=axis, offset=0))


@pytest.mark.parametrize("m", [1, 4, 16])
def test_gemv_c3_shape(m):
    """int8 W[4096, 14336], per-column scale: the decode GEMV sweep at full size."""
    case = c3_case(m, 4096, 14336, 1000 + m)
    got = matmul_quantized(case)
    w = dequant_host(case["bq"], 4096, 14336)
    worst_abs, worst_ratio = assert_gamma_bound(got, case["a"], w)
    assert worst_ratio < 1.0


@pytest.mark.parametrize("m,k,n,zero,axis", [
    (3, 2048, 4096, True, 1), (5, 1000, 1000, True, 0), (2, 576, 1536, False, 0), (9, 333, 77, True, 1),
    # staged 8-column tiles: odd k (pad row, unpaired A loads), n not a multiple of 8,
    # split K for m = 1 and m = 4, per-row zero, a k smaller than one row pair
    (1, 4097, 1001, True, 1), (1, 8192, 520, False, 1), (4, 12288, 264, True, 0), (2, 999, 17, True, 1),
    (3, 5, 9, True, 0), (1, 1, 3, False, 1)])
def test_gemv_modes(m, k, n, zero, axis):
    case = c3_case(m, k, n, 7 * m + k, zero=zero, axis=axis)
    got = matmul_quantized(case)
    w = dequant_host(case["bq"], k, n)
    assert_gamma_bound(got, case["a"], w)
    if k <= 1024:
        assert_plugin_tolerance(got, case["a"], w)


@pytest.mark.parametrize("m", [1, 2, 4])
def test_gemv_unaligned_a(m):
    """A at a 4-byte (not 8-byte) aligned address: the row-pair loads of A must not be used."""
    k, n = 1024, 200
    case = c3_case(m, k, n, 500 + m)
    plane, keep = plane_from_spec(case["bq"])
    a_d = dev(np.concatenate([np.zeros(1, np.float32), case["a"].ravel()]))
    c = dev(np.zeros((m, n), np.float32))
    check(lib().accel_hip_matmul_quantized(a_d.at(1), None, None, C.byref(plane), c.ptr, m, k, n))
    assert_gamma_bound(c.numpy(), case["a"], dequant_host(case["bq"], k, n))
    assert_plugin_tolerance(c.numpy(), case["a"], dequant_host(case["bq"], k, n))


# ---- split-bf16 MFMA GEMV: 2 < m <= 16, no zero points, k a multiple of 32 --------------------
# Each activation enters three bf16 MFMAs as hi + mid + lo (exact), each weight byte as an
# exact bf16; only the fp32 accumulation rounds. A product with m <= 4 too small to give every
# CU a workgroup of that kernel (GemvWantsGroups) runs on the narrow kernel's 8-column tiles
# instead, so the m <= 4 cases of small shapes below check that route, and each has a twin
# with m = 5 or 6 on the split-bf16 kernel.

def _split_case(m, k, n, seed, whole_scale=False, a=None, q=None):
    r = np.random.default_rng(seed)
    if q is None:
        q = r.integers(-127, 128, size=k * n, dtype=np.int8)
    scale = r.uniform(1e-3, 1e-2, size=1 if whole_scale else n).astype(np.float32)
    if a is None:
        a = r.standard_normal((m, k)).astype(np.float32)
    return dict(name="split", m=m, k=k, n=n, a=a,
                bq=dict(q=q, scale=scale, zero=None, shape=[k, n], axis=-1 if whole_scale else 1, offset=0))


@pytest.mark.parametrize("m,k,n,whole", [
    (2, 32, 8, False), (3, 64, 1001, False), (6, 64, 1001, False), (5, 576, 1536, False), (8, 1024, 77, True),
    (4, 96, 14336, False), (5, 96, 14336, False), (13, 4096, 264, False), (16, 8192, 130, False),
    (16, 12288, 2048, True)])
def test_gemv_split_bf16_bound(m, k, n, whole):
    """Ragged n (tiles past the end of the last 16-tile group), one block, split K, a
    whole-tensor scale: within 2 gamma_K of the float64 product, and for k <= 1024 also the
    plugin tolerance."""
    case = _split_case(m, k, n, 31 * m + k, whole_scale=whole)
    got = matmul_quantized(case)
    w = dequant_host(case["bq"], k, n)
    assert_gamma_bound(got, case["a"], w)
    if k <= 1024:
        assert_plugin_tolerance(got, case["a"], w)


@pytest.mark.parametrize("m,k,n", [(4, 576, 1536), (5, 576, 1536), (16, 1024, 264), (7, 4096, 136)])
def test_gemv_split_bf16_integer_sums_exact(m, k, n):
    """Integer A with |a| <= 16: every partial sum is an integer below 2^24, so any order of
    summation gives the exact sum S and C = fl(S * scale) bit for bit. A row, column or k
    slot paired wrongly anywhere changes S."""
    r = np.random.default_rng(m * k + n)
    a = r.integers(-16, 17, size=(m, k)).astype(np.float32)
    case = _split_case(m, k, n, 5 + m, a=a)
    got = matmul_quantized(case)
    s = a.astype(np.int64) @ case["bq"]["q"].reshape(k, n).astype(np.int64)
    assert np.abs(s).max() < 2 ** 24
    same_bits(got, (s.astype(np.float32) * case["bq"]["scale"][None, :]).astype(np.float32))


@pytest.mark.parametrize("m,k,n", [(16, 4096, 1001), (3, 96, 64), (6, 96, 64), (9, 1024, 520)])
def test_gemv_split_bf16_full_precision_a(m, k, n):
    """One nonzero weight per column, a power of two: C = fl(a * w * scale) exactly, which
    needs all 24 significand bits of every activation (N(0, 1) values) to reach the sum;
    dropping the mid or lo bf16 part, or pairing a k slot wrongly, changes bits."""
    r = np.random.default_rng(k + n)
    rows = r.integers(0, k, size=n)
    vals = r.choice(np.array([-64, -8, -2, -1, 1, 4, 16, 64], np.int8), size=n)
    q = np.zeros((k, n), np.int8)
    q[rows, np.arange(n)] = vals
    case = _split_case(m, k, n, 9 + m, q=q.ravel())
    got = matmul_quantized(case)
    a = case["a"]
    prod = (a[:, rows] * vals.astype(np.float32)[None, :]).astype(np.float32)  # exact: power-of-two w
    same_bits(got, (prod * case["bq"]["scale"][None, :]).astype(np.float32))


def _gemv_m1_pair(case, epi=None):
    """C from an 8-byte aligned A (the m = 1 entry kernel, for an even k <= 4096 without zero
    points) and from the same A at a 4-byte offset (the general narrow kernel, single A loads)."""
    k, n = case["k"], case["n"]
    plane, keep = plane_from_spec(case["bq"])
    a_al = dev(case["a"])
    a_un = dev(np.concatenate([np.zeros(1, np.float32), case["a"].ravel()]))
    out = []
    for a_ptr in (a_al.ptr, a_un.at(1)):
        c = dev(np.full((1, n), 3.0, np.float32))
        if epi is None:
            check(lib().accel_hip_matmul_quantized(a_ptr, None, None, C.byref(plane), c.ptr, 1, k, n))
        else:
            check(lib().accel_hip_matmul_quantized_fused(a_ptr, None, None, C.byref(plane), c.ptr, 1, k, n,
                                                         C.byref(epi)))
        out.append(c.numpy())
    return out


@pytest.mark.parametrize("k,n,axis", [(2, 3, 1), (510, 49, 1), (576, 1001, 1), (1000, 64, 1), (1536, 576, 1),
                                      (4094, 17, 1), (4096, 264, -1)])
def test_gemv_m1_entry_kernel_matches_general_kernel(k, n, axis):
    """m = 1 with an even k <= 4096: the entry kernel issues only the 512-row steps k needs
    (k = 510, 1000 and 4094 end inside a step) and must store the general kernel's bits;
    n off a multiple of 8 leaves a partial last tile; axis -1 is one scale for the tensor."""
    case = c3_case(1, k, n, 3 * k + n, axis=max(axis, 0) if axis >= 0 else 1)
    if axis < 0:
        case["bq"]["scale"] = np.array([0.0042], np.float32)
        case["bq"]["axis"] = -1
    entry, general = _gemv_m1_pair(case)
    same_bits(entry, general)
    assert_gamma_bound(entry, case["a"], dequant_host(case["bq"], k, n))
    if k <= 1024:
        assert_plugin_tolerance(entry, case["a"], dequant_host(case["bq"], k, n))


@pytest.mark.parametrize("k,n,axis", [(2, 16389, 1), (130, 16384, 1), (576, 49152, 1), (1022, 20000, -1),
                                      (1024, 16392, 1)])
def test_gemv_wave_tile_kernel(k, n, axis):
    """m = 1 with k <= 1024 over at least 2048 tiles (the LM head's shape, 576 x 49152): one wave
    per 8-column tile, four tiles a workgroup. k = 2 is one row pair, 130 and 1022 end inside a
    lane's last load, 1024 fills 8 loads; n = 16389 leaves a partial last tile and dead waves;
    axis -1 is one scale for the tensor. Within 2 gamma_K and the plugin tolerance of float64,
    and with integer activations (every partial sum an exact integer) fl(S * scale) bit for bit."""
    case = c3_case(1, k, n, 11 * k + n, axis=max(axis, 0) if axis >= 0 else 1)
    if axis < 0:
        case["bq"]["scale"] = np.array([0.0042], np.float32)
        case["bq"]["axis"] = -1
    w = dequant_host(case["bq"], k, n)
    got = matmul_quantized(case)
    assert_gamma_bound(got, case["a"], w)
    assert_plugin_tolerance(got, case["a"], w)
    r = np.random.default_rng(k)
    case["a"] = r.integers(-16, 17, size=(1, k)).astype(np.float32)
    got = matmul_quantized(case)
    s = case["a"].astype(np.int64) @ case["bq"]["q"].reshape(k, n).astype(np.int64)
    assert np.abs(s).max() < 2 ** 24
    scale = case["bq"]["scale"] if axis >= 0 else np.full(n, case["bq"]["scale"][0], np.float32)
    same_bits(got, (s.astype(np.float32) * scale[None, :]).astype(np.float32))


def test_gemv_m1_entry_kernel_epilogues():
    """alpha, beta * bias, Relu / exact Gelu and the residual on the m = 1 entry kernel, whose
    epilogue inputs are loaded before the sums: the general kernel's bits and the composed
    oracle's values."""
    o = oracle()
    r = np.random.default_rng(48)
    k, n = 576, 203
    case = c3_case(1, k, n, 49)
    bias = r.standard_normal(n).astype(np.float32)
    resid = r.standard_normal((1, n)).astype(np.float32)
    bias_d = dev(bias)
    res_d = dev(resid)
    w = dequant_host(case["bq"], k, n)
    base = o.reference_matmul(case["a"], w)
    for act in (0, 1, 2):
        e = Epilogue(alpha=1.5, beta=0.5, bias=bias_d.ptr, bias_rank=1, activation=act, residual=res_d.ptr)
        e.bias_shape[0] = n
        entry, general = _gemv_m1_pair(case, e)
        same_bits(entry, general)
        want = o.gemm_epilogue(base, 1.5, bias, [n], 0.5, act) + resid
        np.testing.assert_allclose(entry, want, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("m,k,n", [(512, 576, 1536), (64, 4096, 1024), (100, 200, 300), (2048, 576, 192)])
def test_gemm_int8_panels(m, k, n):
    """m > 16: the bf16-MFMA GEMM with split K (these grids have fewer 128 x 128 tiles than
    CUs), or the fp32-MFMA GEMM with the int8 panel dequantized in LDS (zero points, k not a
    multiple of 32)."""
    case = c3_case(m, k, n, 31 * m + n, zero=(m == 100))
    got = matmul_quantized(case)
    w = dequant_host(case["bq"], k, n)
    assert_gamma_bound(got, case["a"], w)
    if k <= 1024:
        # Against the float64 product: numpy's own float32 product misses this tolerance on
        # about 100 elements of the 512 x 576 x 1536 case.
        assert_plugin_tolerance(got, case["a"], w)


# ---- int8 GEMM on the bf16 matrix cores: m > 16, k % 32 == 0, at least one 128 x 128 tile per
# CU (256 on MI355X); activations enter as three exact bf16 parts, weights as exact bf16 ------

@pytest.mark.parametrize("m,k,n,whole", [(512, 256, 8192, False), (500, 96, 8200, True), (2048, 32, 2048, False),
                                         (260, 1024, 16384, False)])
def test_gemm_q8_bf16_bound(m, k, n, whole):
    """Ragged m and n (clamped loads, masked stores), one chunk, a whole-tensor scale: within
    2 gamma_K of the float64 product, and within the plugin tolerance of it. (At k = 1024 these
    weights give outputs of std 13 and up to 100; numpy's own float32 product misses 1e-5 of
    the float64 product on about 2300 elements of that case, the two-accumulator bf16 sum on
    none.)"""
    case = _split_case(m, k, n, m + k + n, whole_scale=whole)
    got = matmul_quantized(case)
    w = dequant_host(case["bq"], k, n)
    assert_gamma_bound(got, case["a"], w)
    assert_plugin_tolerance(got, case["a"], w)


@pytest.mark.parametrize("m,k,n", [(256, 4096, 16384), (100, 2048, 264), (512, 576, 3072)])
def test_gemm_q8_bf16_integer_sums_exact(m, k, n):
    """Integer A with |a| <= 16: every partial sum is an integer below 2^24, so C = fl(S *
    scale) bit for bit; a row, column or k slot paired wrongly changes S. The last two
    shapes have fewer tiles than CUs: 100 x 2048 x 264 splits K (21 splits), 512 x 576 x 3072
    (k <= 768) runs on the small kernel."""
    r = np.random.default_rng(91 + m)
    a = r.integers(-16, 17, size=(m, k)).astype(np.float32)
    case = _split_case(m, k, n, 92 + m, a=a)
    got = matmul_quantized(case)
    s = a.astype(np.float64) @ case["bq"]["q"].reshape(k, n).astype(np.float64)  # integers below 2^53: exact
    assert np.abs(s).max() < 2 ** 24
    same_bits(got, (s.astype(np.float32) * case["bq"]["scale"][None, :]).astype(np.float32))


def test_gemm_q8_bf16_full_precision_a():
    """One power-of-two weight per column: C = fl(a * w * scale) exactly, which needs all 24
    significand bits of every N(0, 1) activation (all three bf16 parts) to reach the sum."""
    m, k, n = 640, 512, 6656
    r = np.random.default_rng(93)
    rows = r.integers(0, k, size=n)
    vals = r.choice(np.array([-64, -8, -2, -1, 1, 4, 16, 64], np.int8), size=n)
    q = np.zeros((k, n), np.int8)
    q[rows, np.arange(n)] = vals
    case = _split_case(m, k, n, 94, q=q.ravel())
    got = matmul_quantized(case)
    prod = (case["a"][:, rows] * vals.astype(np.float32)[None, :]).astype(np.float32)
    same_bits(got, (prod * case["bq"]["scale"][None, :]).astype(np.float32))


def test_gemm_q8_bf16_epilogues():
    """alpha, beta * bias, Relu / exact Gelu and a same-shape residual applied to the scaled
    sums, against the oracle's epilogue of the float64 product."""
    m, k, n = 512, 128, 8192
    case = _split_case(m, k, n, 95)
    r = np.random.default_rng(96)
    bias = r.standard_normal(n).astype(np.float32)
    resid = r.standard_normal((m, n)).astype(np.float32)
    bias_d, res_d = dev(bias), dev(resid)
    base = (case["a"].astype(np.float64) @ dequant_host(case["bq"], k, n).astype(np.float64)).astype(np.float32)
    o = oracle()
    for act in (1, 2):
        e = Epilogue(alpha=1.5, beta=0.5, bias=bias_d.ptr, bias_rank=1, activation=act, residual=res_d.ptr)
        e.bias_shape[0] = n
        got = matmul_quantized(case, e)
        want = o.gemm_epilogue(base, 1.5, bias, [n], 0.5, act) + resid
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


# ---- int8 GEMM for a short k on the small kernel: m > 16, k <= 768 or 1536, a grid below the 128-tile
# image path. 16-row blocks over all of k; the activation rows split into three exact bf16 parts
# in LDS; the weight read from its bf16 copy in the B-operand order of the 16x16x32 MFMA ------

@pytest.mark.parametrize("m,k,n,whole", [(17, 32, 8, False), (37, 96, 1000, True), (100, 768, 136, False),
                                         (512, 576, 960, False), (333, 160, 3080, False),
                                         (512, 1536, 576, False), (40, 1536, 200, True)])
def test_gemm_q8_small_bound(m, k, n, whole):
    """A partial 16-row block, column blocks and groups partly past n, one 32-row block, the
    largest k of the generic kernel, a whole-tensor scale, and k = 1536 on its own instance (the
    Llama prompt's down projection): within 2 gamma_K of the float64 product, and within the
    plugin tolerance of it for k <= 1024."""
    case = _split_case(m, k, n, 7 * m + k + n, whole_scale=whole)
    got = matmul_quantized(case)
    w = dequant_host(case["bq"], k, n)
    assert_gamma_bound(got, case["a"], w)
    if k <= 1024:
        assert_plugin_tolerance(got, case["a"], w)


@pytest.mark.parametrize("m,k,n", [(48, 768, 264), (530, 576, 576), (64, 1536, 136)])
def test_gemm_q8_small_integer_sums_exact(m, k, n):
    """Integer A with |a| <= 16 on the small kernel: C = fl(S * scale) bit for bit; a row,
    column or k slot paired wrongly anywhere changes S."""
    r = np.random.default_rng(17 + m)
    a = r.integers(-16, 17, size=(m, k)).astype(np.float32)
    case = _split_case(m, k, n, 18 + m, a=a)
    got = matmul_quantized(case)
    s = a.astype(np.float64) @ case["bq"]["q"].reshape(k, n).astype(np.float64)
    assert np.abs(s).max() < 2 ** 24
    same_bits(got, (s.astype(np.float32) * case["bq"]["scale"][None, :]).astype(np.float32))


def test_gemm_q8_small_full_precision_a():
    """One power-of-two weight per column on the small kernel: C = fl(a * w * scale) exactly,
    which needs all three bf16 parts of every N(0, 1) activation to reach the sum."""
    m, k, n = 40, 256, 264
    r = np.random.default_rng(19)
    rows = r.integers(0, k, size=n)
    vals = r.choice(np.array([-64, -8, -2, -1, 1, 4, 16, 64], np.int8), size=n)
    q = np.zeros((k, n), np.int8)
    q[rows, np.arange(n)] = vals
    case = _split_case(m, k, n, 20, q=q.ravel())
    got = matmul_quantized(case)
    prod = (case["a"][:, rows] * vals.astype(np.float32)[None, :]).astype(np.float32)
    same_bits(got, (prod * case["bq"]["scale"][None, :]).astype(np.float32))


def test_gemm_q8_small_epilogues():
    """alpha, beta * bias, Relu / exact Gelu and a same-shape residual at the small kernel's
    store, against the oracle's epilogue of the float64 product."""
    m, k, n = 200, 384, 1000
    case = _split_case(m, k, n, 21)
    r = np.random.default_rng(22)
    bias = r.standard_normal(n).astype(np.float32)
    resid = r.standard_normal((m, n)).astype(np.float32)
    bias_d, res_d = dev(bias), dev(resid)
    base = (case["a"].astype(np.float64) @ dequant_host(case["bq"], k, n).astype(np.float64)).astype(np.float32)
    o = oracle()
    for act in (1, 2):
        e = Epilogue(alpha=1.5, beta=0.5, bias=bias_d.ptr, bias_rank=1, activation=act, residual=res_d.ptr)
        e.bias_shape[0] = n
        got = matmul_quantized(case, e)
        want = o.gemm_epilogue(base, 1.5, bias, [n], 0.5, act) + resid
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("m,k,n", [(4, 4096, 1792), (100, 2048, 264)])
def test_split_products_replay_from_graph(m, k, n):
    """A product whose K is split (the split-bf16 GEMV with its per-group arrival counters,
    16 splits; the bf16 GEMM with its workspace, 21 splits) captured in a HIP graph and
    replayed three times, with other eager products between the replays: every replay stores
    the eager result's bits (the counters are left zero by each launch)."""
    L = lib()
    r = np.random.default_rng(m + n)
    q = r.integers(-127, 128, size=k * n, dtype=np.int8)
    s = r.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    a = r.standard_normal((m, k)).astype(np.float32)
    qd, sd, ad = dev(q), dev(s), dev(a)
    plane = quant_plane(qd, sd, None, [k, n], 1)
    out = dev(np.zeros((m, n), np.float32))

    def call():
        check(L.accel_hip_matmul_quantized(ad.ptr, None, None, C.byref(plane), out.ptr, m, k, n))

    call()
    want = out.numpy()
    call()  # warm (staging, workspace) before the capture
    check(L.accel_hip_capture_begin())
    call()
    g = C.c_void_p()
    check(L.accel_hip_capture_end(C.byref(g)))
    try:
        other = _split_case(8, 1024, 1000, 7)
        for _ in range(3):
            out.upload(np.zeros((m, n), np.float32))
            check(L.accel_hip_graph_launch(g, 1))
            same_bits(out.numpy(), want)
            matmul_quantized(other)  # eager work between the replays
    finally:
        check(L.accel_hip_graph_destroy(g))


def test_gemm_c4_shape_with_fused_rmsnorm():
    """The prefill product at full size, X[2048, 4096] @ int8 W[4096, 14336] per-column scale
    with the RMSNormalization of the output rows fused: 40 sampled rows (first, last, random)
    meet the gamma_K bound against float64, and the fused RMS rows equal the oracle's RMSNorm
    of the stored product rows."""
    m, k, n = 2048, 4096, 14336
    case = c3_case(m, k, n, 4242)
    r = np.random.default_rng(4243)
    gamma_w = (1 + 0.1 * r.standard_normal(n)).astype(np.float32)
    g_d = dev(gamma_w)
    out = dev(np.zeros((m, n), np.float32))
    e = Epilogue(alpha=1.0, beta=1.0, rms_weight=g_d.ptr, rms_eps=1e-5, rms_out=out.ptr)
    got = matmul_quantized(case, e)
    y = out.numpy()
    rows = np.unique(np.concatenate([[0, 1, 127, 128, m - 1], r.choice(m, 35, replace=False)]))
    w = dequant_host(case["bq"], k, n)
    assert_gamma_bound(got[rows], case["a"][rows], w)
    want = oracle().rmsnorm(np.ascontiguousarray(got[rows]), gamma_w, rows.size, n, 1e-5)
    np.testing.assert_allclose(y[rows], want, rtol=1e-6, atol=1e-6)
    assert np.isfinite(y).all()


def test_gemm_image_path_fused_rmsnorm_ragged():
    """The 128-tile GEMM from the activation image and the staged bf16 weight, with ragged m
    and n, alpha, bias and Gelu before a fused RMSNormalization: the stored product meets the
    gamma_K bound (plus the epilogue's roundings), and every normalized row equals the oracle's
    RMSNorm of the stored row to 1e-6 (the row sums of squares are added per tile, in double)."""
    m, k, n = 300, 256, 12296
    case = _split_case(m, k, n, 4300)
    r = np.random.default_rng(4301)
    gamma_w = (1 + 0.1 * r.standard_normal(n)).astype(np.float32)
    bias = (0.1 * r.standard_normal(n)).astype(np.float32)
    g_d, b_d = dev(gamma_w), dev(bias)
    out = dev(np.zeros((m, n), np.float32))
    e = Epilogue(alpha=1.25, beta=1.0, bias=b_d.ptr, bias_rank=1, activation=2, rms_weight=g_d.ptr, rms_eps=1e-5,
                 rms_out=out.ptr)
    e.bias_shape[0] = n
    got = matmul_quantized(case, e)
    y = out.numpy()
    w = dequant_host(case["bq"], k, n)
    o = oracle()
    want = o.gemm_epilogue((case["a"].astype(np.float64) @ w.astype(np.float64)).astype(np.float32), 1.25, bias, [n],
                           1.0, 2)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(y, o.rmsnorm(np.ascontiguousarray(got), gamma_w, m, n, 1e-5), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("m, k, n, rms", [(4000, 256, 5120, True), (2048, 128, 10240, False)])
def test_gemm_wide_grid(m, k, n, rms):
    """Shapes whose tiles divide evenly over the 256 CUs of an MI355X take the wide grid
    (128 x 256 tiles of 8 waves, then one round of 128 x 128 tiles): 4000 rows (32 row tiles,
    the last one ragged) x 5120 columns with alpha, bias, Gelu and a fused RMSNormalization,
    and 2048 x 10240 with bias and a residual. The stored product meets the gamma_K bound (plus
    the epilogue's roundings) and the normalized rows equal the oracle's RMSNorm of the stored
    rows."""
    case = _split_case(m, k, n, 4400 + m)
    r = np.random.default_rng(4401 + m)
    bias = (0.1 * r.standard_normal(n)).astype(np.float32)
    b_d = dev(bias)
    w = dequant_host(case["bq"], k, n)
    o = oracle()
    prod = (case["a"].astype(np.float64) @ w.astype(np.float64)).astype(np.float32)
    if rms:
        gamma_w = (1 + 0.1 * r.standard_normal(n)).astype(np.float32)
        g_d = dev(gamma_w)
        out = dev(np.zeros((m, n), np.float32))
        e = Epilogue(alpha=1.25, beta=1.0, bias=b_d.ptr, bias_rank=1, activation=2, rms_weight=g_d.ptr,
                     rms_eps=1e-5, rms_out=out.ptr)
        e.bias_shape[0] = n
        got = matmul_quantized(case, e)
        want = o.gemm_epilogue(prod, 1.25, bias, [n], 1.0, 2)
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)
        np.testing.assert_allclose(out.numpy(), o.rmsnorm(np.ascontiguousarray(got), gamma_w, m, n, 1e-5), rtol=1e-6,
                                   atol=1e-6)
    else:
        res = r.standard_normal((m, n)).astype(np.float32)
        res_d = dev(res)
        e = Epilogue(alpha=1.0, beta=1.0, bias=b_d.ptr, bias_rank=1, residual=res_d.ptr)
        e.bias_shape[0] = n
        got = matmul_quantized(case, e)
        want = o.gemm_epilogue(prod, 1.0, bias, [n], 1.0, 0) + res
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("m", [2, 4])
def test_staged_weight_follows_rewrites(m):
    """The GEMV reads a staged copy of W (8-column tiles at m = 2, the group-interleaved form
    at m = 4); rewriting W (host copy, or W used as a kernel output) must be seen by the next
    call."""
    r = np.random.default_rng(77)
    k, n = 256, 320
    q1 = r.integers(-127, 128, size=k * n, dtype=np.int8)
    q2 = r.integers(-127, 128, size=k * n, dtype=np.int8)
    s = r.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    a = r.standard_normal((m, k)).astype(np.float32)
    qd, sd, ad = dev(q1), dev(s), dev(a)
    plane = quant_plane(qd, sd, None, [k, n], 1)
    out = dev(np.zeros((m, n), np.float32))

    def run():
        check(lib().accel_hip_matmul_quantized(ad.ptr, None, None, C.byref(plane), out.ptr, m, k, n))
        return out.numpy()

    w1 = dequant_host(dict(q=q1, scale=s, zero=None, shape=[k, n], axis=1, offset=0), k, n)
    w2 = dequant_host(dict(q=q2, scale=s, zero=None, shape=[k, n], axis=1, offset=0), k, n)
    assert_gamma_bound(run(), a, w1)
    assert_gamma_bound(run(), a, w1)  # second call reads the staged copy
    qd.upload(q2)
    assert_gamma_bound(run(), a, w2)
    # W's allocation overwritten by a kernel output (residual add over its bytes as floats).
    zeros = dev(np.zeros(k * n // 4, np.float32))
    check(lib().accel_hip_residual_add(qd.buffer, zeros.buffer, k * n // 4))  # adds 0.0: bytes of q2 kept
    qd.upload(q1)
    assert_gamma_bound(run(), a, w1)


def test_quantized_errors_and_counters():
    L = lib()
    L.accel_hip_reset_stats()
    L.accel_hip_reset_packed_probes()
    case = c3_case(2, 64, 32, 5)
    matmul_quantized(case)
    assert stats().kernel_matmuls == 1 and L.accel_hip_packed_k_trips() == 64
    with pytest.raises(HipError) as e:
        check(L.accel_hip_matmul_quantized(None, None, None, None, None, 2, 3, 4))
    assert e.value.kind == "invalid_argument"


# ---- fused epilogue -------------------------------------------------------------------------

def test_fused_epilogue_matches_composed_oracle():
    o = oracle()
    r = np.random.default_rng(44)
    m, k, n = 8, 512, 384
    case = c3_case(m, k, n, 45)
    bias = r.standard_normal(n).astype(np.float32)
    resid = r.standard_normal((m, n)).astype(np.float32)
    bias_d = dev(bias)
    res_d = dev(resid)
    for act in (0, 1, 2):
        e = Epilogue(alpha=1.5, beta=0.5, bias=bias_d.ptr, bias_rank=1, activation=act, residual=res_d.ptr)
        e.bias_shape[0] = n
        got = matmul_quantized(case, e)
        w = dequant_host(case["bq"], k, n)
        base = o.reference_matmul(case["a"], w)
        want = o.gemm_epilogue(base, 1.5, bias, [n], 0.5, act) + resid
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


def test_fused_rmsnorm_epilogue():
    r = np.random.default_rng(46)
    m, k, n = 12, 256, 1000
    case = c3_case(m, k, n, 47)
    gamma_w = (1 + 0.1 * r.standard_normal(n)).astype(np.float32)
    g_d = dev(gamma_w)
    out = dev(np.zeros((m, n), np.float32))
    e = Epilogue(alpha=1.0, beta=1.0, rms_weight=g_d.ptr, rms_eps=1e-5, rms_out=out.ptr)
    c = matmul_quantized(case, e)
    y = out.numpy()
    want = oracle().rmsnorm(c, gamma_w, m, n, 1e-5)  # normalizes the stored C rows
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-6)


# ---- GemmEpilogue (src/sim_device.cc:211-245) ------------------------------------------------

def test_epilogue_reference_fixtures(gold):
    L = lib()
    for case in epilogue_cases():
        cd = dev(case["c"])
        m, n = case["c"].shape
        shape = (C.c_int64 * 2)(*(list(case["bias_shape"]) + [0, 0])[:2])
        if case["bias"] is not None:
            bd = dev(case["bias"])
            check(L.accel_hip_gemm_epilogue(cd.buffer, m, n, case["alpha"], C.byref(bd.buffer), len(case["bias_shape"]),
                                            shape, case["beta"], case["act"]))
        else:
            check(L.accel_hip_gemm_epilogue(cd.buffer, m, n, case["alpha"], None, 0, shape, case["beta"], case["act"]))
        got = cd.numpy()
        want = gold[f"epi_{case['name']}_out"]
        if case["act"] == 2:
            # Device erff vs glibc erff differ by a few ulp; 1 + erf(x) cancels for negative x,
            # so the bound is relative to the gelu input scale: |d| <= 1e-6*|want| + 2e-7.
            fin = np.isfinite(want)
            assert np.array_equal(np.isnan(got), np.isnan(want))
            assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])
            np.testing.assert_allclose(got[fin], want[fin], rtol=1e-6, atol=2e-7)
        else:
            same_bits(got, want)


def test_nonfinite_relu_bits():
    # tests/test_runtime.cc:427-459: inf*0 -> NaN survives relu, -inf -> +0, -1*0 -> -0.
    L = lib()
    vals = np.array([np.nan, -np.inf, 0.0], np.float32)
    cd = dev(vals[None, :])
    check(L.accel_hip_gemm_epilogue(cd.buffer, 1, 3, -1.0, None, 0, (C.c_int64 * 2)(), 0.0, 1))
    got = cd.numpy()[0]
    assert np.isnan(got[0]) and got.view(np.uint32)[1] == 0x7F800000 and got.view(np.uint32)[2] == 0x80000000


# ---- named decode kernels --------------------------------------------------------------------

def test_rmsnorm_reference_fixtures(gold):
    for c in rmsnorm_cases():
        x = dev(c["x"])
        w = dev(c["w"])
        y = dev(np.full((c["rows"], c["dim"]), 42.0, np.float32))
        check(lib().accel_hip_rms_norm(x.buffer, w.buffer, y.buffer, c["rows"], c["dim"], c["eps"], c["row_offset"]))
        np.testing.assert_allclose(y.numpy(), gold[f"rms_{c['name']}_out"], rtol=2e-7, atol=1e-7)


def test_embedding_reference_fixtures(gold):
    for c in embed_cases():
        ids = dev(c["ids"])
        table = dev(c["table"])
        out = dev(np.zeros((c["seq"], c["table"].shape[1]), np.float32))
        rc = lib().accel_hip_embedding(ids.buffer, c["id_offset"], table.buffer, out.buffer, c["seq"],
                                       c["table"].shape[1], c["table"].shape[0])
        if int(gold[f"embed_{c['name']}_rc"]) != 0:
            assert rc == 1 and "outside the vocabulary" in lib().accel_hip_last_error().decode()
        else:
            assert rc == 0
            same_bits(out.numpy(), gold[f"embed_{c['name']}_out"])


def test_rope_reference_fixtures(gold):
    for c in rope_cases():
        st = dev(c["states"])
        cs = dev(c["cos"])
        sn = dev(c["sin"])
        check(lib().accel_hip_rope(st.buffer, cs.buffer, sn.buffer, c["seq"], c["heads"], c["head_dim"],
                                   c["position"]))
        same_bits(st.numpy(), gold[f"rope_{c['name']}_out"])


def test_append_cache_exact():
    src = np.arange(12, dtype=np.float32)
    cache = dev(np.full(20, -5, np.float32))
    s = dev(src)
    check(lib().accel_hip_append_cache(s.buffer, cache.buffer, 2, 1, 2, 3))
    want = np.full(20, -5, np.float32)
    want[6:18] = src
    same_bits(cache.numpy(), want)


def test_attention_reference_fixtures(gold):
    for c in attention_cases():
        q, k, v = dev(c["q"]), dev(c["k"]), dev(c["v"])
        total = c["seq"] + c["position"]
        scores = dev(np.zeros(total, np.float32))
        out = dev(np.zeros(c["q"].shape, np.float32))
        check(lib().accel_hip_attention(q.buffer, k.buffer, v.buffer, scores.buffer, out.buffer, c["seq"],
                                        c["position"], c["heads"], c["kv_heads"], c["head_dim"]))
        np.testing.assert_allclose(out.numpy(), gold[f"attn_{c['name']}_out"], rtol=1e-5, atol=2e-6)


def test_silu_add_reference_fixtures(gold):
    for c in silu_add_cases():
        g, u = dev(c["gate"]), dev(c["up"])
        check(lib().accel_hip_silu_mul(g.buffer, u.buffer, c["gate"].size))
        np.testing.assert_allclose(g.numpy(), gold[f"silu_{c['name']}_out"], rtol=1e-6, atol=1e-30)
        d, e = dev(c["gate"]), dev(c["up"])
        check(lib().accel_hip_residual_add(d.buffer, e.buffer, c["gate"].size))
        same_bits(d.numpy(), gold[f"add_{c['name']}_out"])


def test_sampling_reference_fixtures(gold):
    ids = []
    states = []
    chosen = dev(np.full(3, -1, np.int32))
    for c in sample_cases():
        lg = dev(c["logits"])
        st = C.c_uint32(c["rng"])
        check(lib().accel_hip_sample_token(lg.buffer, chosen.buffer, 1, c["logits"].size, c["temperature"],
                                           C.byref(st), c["top_k"]))
        ids.append(int(chosen.numpy()[1]))
        states.append(st.value)
    want_ids = gold["sample_ids"]
    want_states = gold["sample_rng_after"]
    mism = [i for i in range(len(ids)) if ids[i] != want_ids[i] or states[i] != want_states[i]]
    assert not mism, f"{len(mism)} sampling cases differ, first {mism[:5]}"


def _greedy_cases():
    r = np.random.default_rng(77)
    v = 49152
    base = lambda: r.standard_normal(v).astype(np.float32)
    x = base()
    yield "random", x
    x = base(); top = float(x.max()) + 1.0
    x[[40000, 3001, 3000, 17000]] = top  # equal maxima in three workgroups: the earliest id wins
    yield "ties", x
    x = -np.abs(base()) - 1.0
    x[30000], x[5000] = 0.0, -0.0  # -0 equals +0: the earlier id wins
    yield "signed_zero", x
    x = base(); x[0] = np.nan
    yield "nan_at_0", x
    x = base(); x[[1, 2048, 40000]] = np.nan; x[9999] = 50.0
    yield "nan_elsewhere", x
    x = np.full(v, np.nan, np.float32); x[0] = -3.0
    yield "all_nan_but_0", x
    yield "all_neg_inf", np.full(v, -np.inf, np.float32)
    x = base(); x[-1] = np.inf
    yield "inf_last", x
    x = r.standard_normal(49156).astype(np.float32)  # a partial last workgroup
    x[49155] = 99.0
    yield "ragged_tail", x
    yield "odd_vocab", r.standard_normal(4097).astype(np.float32)  # one-workgroup path


@pytest.mark.parametrize("name", [n for n, _ in _greedy_cases()])
def test_greedy_pick_matches_oracle(name):
    """Greedy SampleToken (temperature 0) over a 49152-id row runs on many workgroups, each
    reducing 2048 ids to an order-preserving key, the last to arrive picking the largest. Its
    id must equal the reference's strict > scan (the oracle's orc_sample_token): the earliest
    id among equal maxima, -0 equal to +0, NaNs never chosen, 0 when id 0 holds a NaN. Two
    launches in a row check that the arrival count is left at zero."""
    x = dict(_greedy_cases())[name]
    want, _ = oracle().sample_token(x, 0.0, 1, 0)
    lg = dev(x)
    chosen = dev(np.full(2, -1, np.int32))
    for _ in range(2):
        st = C.c_uint32(1)
        check(lib().accel_hip_sample_token(lg.buffer, chosen.buffer, 1, x.size, 0.0, C.byref(st), 0))
        got = int(chosen.numpy()[1])
        print(f"greedy {name}: gpu {got} oracle {want}", flush=True)
        assert got == want
