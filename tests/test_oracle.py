"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Three independent anchors:
  * the reference tests' own known answers (tests/test_runtime.cc, tests/test_sim_kernels.cc,
    tests/test_ep.py), hand values and bit patterns;
  * tests/golden/reference_outputs.npz, outputs of the compiled reference (oracle/_ref) on
    seeded inputs, compared bit for bit;
  * mathematics: float64 products and error bounds, closed forms, invariants.
When oracle/_ref was built (reference tree present), randomized inputs are also compared
against it directly.
"""

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from golden_cases import (attention_cases, embed_cases, epilogue_cases, llama_cases, llama_config, llama_weights,
                          quant_cases, rmsnorm_cases, rope_cases, sample_cases, silu_add_cases)
from oracle_ctypes import (F32P, I32P, LlamaConfig, bits, fill_lcg, from_bits, make_plane, oracle, reference)

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_outputs.npz"


def same_bits(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape
    both_nan = np.isnan(got) & np.isnan(want)
    diff = (bits(got) != bits(want)) & ~both_nan
    assert not diff.any(), f"{diff.sum()} elements differ; first at {np.argwhere(diff)[0]}"


def run_quant(lib, case):
    planes = {}
    keep = []
    for side in ("a", "b"):
        spec = case.get(side + "q")
        if spec is None:
            planes[side] = None
            continue
        plane, k = make_plane(spec["q"], spec["scale"], spec["zero"], spec["shape"], spec["axis"], spec["offset"])
        planes[side] = plane
        keep.append(k)
    return lib.matmul_quantized(case.get("a"), planes["a"], case.get("b"), planes["b"], case["m"], case["k"],
                                case["n"])


# ---- known answers from the reference's tests ----------------------------------------------

def test_known_matmul():
    # tests/test_runtime.cc:39-46
    c = oracle().reference_matmul(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]]))
    assert c.tolist() == [[19, 22], [43, 50]]


def test_split_product_bits():
    # tests/test_runtime.cc:413-425: no fused multiply-add.
    a = from_bits([[0xBE2694CD, 0x3E41AF7D]])
    b = from_bits([[0x3F800000], [0x3F5C2CB8]])
    assert int(bits(oracle().reference_matmul(a, b))[0, 0]) == 0xB5200000
    fused = np.float32(np.float64(a[0, 0]) * np.float64(b[0, 0]) + np.float64(a[0, 1]) * np.float64(b[1, 0]))
    assert int(bits(fused)) != 0xB5200000  # the fused answer is a different float


def test_dq_kat():
    # tests/test_ep.py:336-343: DQ axis 0 with zero point, want[0,0] == -48.5 exactly.
    case = [c for c in quant_cases() if c["name"] == "dq_kat"][0]
    out = run_quant(oracle(), case)
    assert out[0, 0] == np.float32(-48.5)


def test_gemm_trans_bias_kat():
    # tests/test_runtime.cc:71-84: transB, alpha 2, bias [1, 3] -> {9, 13, 21, 25}.
    o = oracle()
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b_stored = np.array([[1, 0, 1], [0, 1, 1]], np.float32)
    bt = np.zeros((3, 2), np.float32)
    o.lib.orc_transpose.argtypes = [F32P, F32P, C.c_int64, C.c_int64]
    o.lib.orc_transpose(b_stored.ctypes.data_as(F32P), bt.ctypes.data_as(F32P), 2, 3)
    c = o.reference_matmul(a, bt)
    c = o.gemm_epilogue(c, 2.0, np.array([1, 3], np.float32), [2], 1.0, 0)
    assert c.tolist() == [[9, 13], [21, 25]]


def test_nonfinite_epilogue_bits():
    # tests/test_runtime.cc:427-459.
    o = oracle()
    inf = np.float32(np.inf)
    c = o.reference_matmul(np.array([[inf]]), np.array([[0.0]]))
    c = o.gemm_epilogue(c, 1.0, None, [], 0.0, 1)
    assert np.isnan(c[0, 0])
    c = o.reference_matmul(np.array([[-inf]]), np.array([[1.0]]))
    assert int(bits(o.gemm_epilogue(c, 1.0, None, [], 0.0, 1))[0, 0]) == 0x00000000
    c = o.reference_matmul(np.array([[0.0]]), np.array([[1.0]]))
    assert int(bits(o.gemm_epilogue(c, -1.0, None, [], 0.0, 1))[0, 0]) == 0x80000000
    c = o.reference_matmul(np.array([[1.0]]), np.array([[1.0]]))
    assert int(bits(o.gemm_epilogue(c, 2.0, None, [], 0.0, 0))[0, 0]) == 0x40000000


def test_rmsnorm_closed_form():
    # tests/test_sim_kernels.cc:22-41,72-98: double formula within 1e-6; row_offset reads row 1.
    o = oracle()
    x = np.array([1, -1, 2, 0, 4, -2, 0.5, 3], np.float32)
    w = np.array([1, 2, 0.5, 1.5], np.float32)
    for row in (0, 1):
        y = o.rmsnorm(x, w, 1, 4, 1e-5, row)
        r = x[4 * row:4 * row + 4].astype(np.float64)
        inv = 1.0 / np.sqrt(np.sum(r * r) / 4 + np.float64(np.float32(1e-5)))
        np.testing.assert_allclose(y[0], r * inv * w, atol=1e-6, rtol=0)


def test_named_kernel_hand_values():
    # tests/test_sim_kernels.cc:47-185.
    o = oracle()
    table = np.arange(1, 9, dtype=np.float32).reshape(4, 2)
    rc, out = o.embed(np.array([2, 0], np.int32), 0, table, 2)
    assert rc == 0 and out.ravel().tolist() == [5, 6, 1, 2]
    rc, _ = o.embed(np.array([9], np.int32), 0, table, 1)
    assert rc != 0
    kept = o.rope(np.array([8, -1, 0.5, 4], np.float32), np.ones(4), np.zeros(4), 1, 1, 4, 0)
    assert kept.tolist() == [8, -1, 0.5, 4]
    turned = o.rope(np.array([1, 2, 3, 4], np.float32), np.array([1, 1, 1, 1, 0, 0, 0, 0]),
                    np.array([0, 0, 0, 0, 1, 1, 1, 1]), 1, 1, 4, 1)
    assert turned.tolist() == [-3, -4, 1, 2]
    cache = o.append_cache(np.array([9, 8, 7, 6], np.float32), np.full(8, -5, np.float32), 2, 1, 1, 2)
    assert cache.tolist() == [-5, -5, 9, 8, 7, 6, -5, -5]
    out = o.attention(np.array([1.0]), np.array([1.0]), np.array([3.0]), 1, 0, 1, 1, 1)
    assert out.ravel().tolist() == [3.0]
    assert o.silu_mul(np.array([0.0]), np.array([2.0])).tolist() == [0.0]
    assert o.add(np.array([1.0, 2.0]), np.array([3.0, 4.0])).tolist() == [4.0, 6.0]


def test_sampling_kats():
    # tests/test_sim_kernels.cc:187-231.
    o = oracle()
    assert o.sample_token(np.array([1, 3, 3]), 0.0, 1, 2)[0] == 1
    assert o.sample_token(np.array([1, 3, 3]), -1.0, 1, 0)[0] == 1
    assert o.sample_token(np.array([1, 3, 0]), 1.0, 1856, 2)[0] == 0
    assert o.sample_token(np.array([1, 3, 0]), 1.0, 1856, 0)[0] == 1
    assert o.sample_token(np.array([1, 3, 0]), 1.0, 0, 0) == (0, 0)
    assert o.sample_token(np.zeros(65), 1.0, 1000, 65)[0] == 4
    assert o.sample_token(np.zeros(65), 1.0, 1000, 64)[0] == 3


# ---- bit-exact against the compiled reference's outputs (committed fixtures) ---------------

def test_matmul_matches_reference_fixtures(gold):
    o = oracle()
    for key in [k[:-2] for k in gold if k.startswith("matmul_") and k.endswith("_a")]:
        got = o.reference_matmul(gold[key + "_a"], gold[key + "_b"])
        same_bits(got, gold[key + "_reference"])
        same_bits(got, gold[key + "_device"])  # SimDevice's packed kernel keeps the k order


def test_quantized_matches_reference_fixtures(gold):
    for case in quant_cases():
        same_bits(run_quant(oracle(), case), gold[f"quant_{case['name']}_out"])


def test_epilogue_matches_reference_fixtures(gold):
    for case in epilogue_cases():
        got = oracle().gemm_epilogue(case["c"], case["alpha"], case["bias"], case["bias_shape"], case["beta"],
                                     case["act"])
        same_bits(got, gold[f"epi_{case['name']}_out"])


def test_named_kernels_match_reference_fixtures(gold):
    o = oracle()
    for c in rmsnorm_cases():
        same_bits(o.rmsnorm(c["x"], c["w"], c["rows"], c["dim"], c["eps"], c["row_offset"]), gold[f"rms_{c['name']}_out"])
    for c in embed_cases():
        rc, out = o.embed(c["ids"], c["id_offset"], c["table"], c["seq"])
        assert (rc != 0) == (int(gold[f"embed_{c['name']}_rc"]) != 0)
        same_bits(out, gold[f"embed_{c['name']}_out"])
    for c in rope_cases():
        same_bits(o.rope(c["states"], c["cos"], c["sin"], c["seq"], c["heads"], c["head_dim"], c["position"]),
                  gold[f"rope_{c['name']}_out"])
    for c in attention_cases():
        same_bits(o.attention(c["q"], c["k"], c["v"], c["seq"], c["position"], c["heads"], c["kv_heads"],
                              c["head_dim"]), gold[f"attn_{c['name']}_out"])
    for c in silu_add_cases():
        same_bits(o.silu_mul(c["gate"], c["up"]), gold[f"silu_{c['name']}_out"])
        same_bits(o.add(c["gate"], c["up"]), gold[f"add_{c['name']}_out"])


def test_sampling_matches_reference_fixtures(gold):
    o = oracle()
    ids = []
    states = []
    for c in sample_cases():
        i, s = o.sample_token(c["logits"], c["temperature"], c["rng"], c["top_k"])
        ids.append(i)
        states.append(s)
    assert np.array_equal(np.array(ids, np.int32), gold["sample_ids"])
    assert np.array_equal(np.array(states, np.uint32), gold["sample_rng_after"])


def run_oracle_llama(case):
    o = oracle()
    L = o.lib
    cfg = LlamaConfig(**case["config"])
    h = L.orc_llama_create(C.byref(cfg))
    assert h
    try:
        for (kind, layer, w) in case["weights"]:
            w = np.ascontiguousarray(w, np.float32)
            rows, cols = (w.shape[0], 1) if w.ndim == 1 else w.shape
            assert L.orc_llama_weight(h, kind, layer, w.ctypes.data_as(F32P), rows, cols) == 0
        prompt = np.ascontiguousarray(case["prompt"], np.int32)
        assert L.orc_llama_forward_ids(h, prompt.ctypes.data_as(I32P), prompt.size, 1) == 0
        row = np.zeros(case["config"]["vocab"], np.float32)
        assert L.orc_llama_logits(h, row.ctypes.data_as(F32P), row.size) == 0
        ids = np.zeros(case["max_new"], np.int32)
        count = C.c_int32()
        assert L.orc_llama_generate(h, prompt.ctypes.data_as(I32P), prompt.size, case["max_new"], case["eos"],
                                    case["temperature"], case["seed"], case["top_k"], ids.ctypes.data_as(I32P),
                                    C.byref(count)) == 0
        return ids[: count.value], row
    finally:
        L.orc_llama_destroy(h)


def test_llama_matches_reference_fixtures(gold):
    for case in llama_cases():
        ids, row = run_oracle_llama(case)
        assert np.array_equal(ids, gold[f"llama_{case['name']}_ids"]), case["name"]
        same_bits(row, gold[f"llama_{case['name']}_prefill_logits"])


# ---- mathematics ------------------------------------------------------------------------------

def gamma(k):
    u = 2.0 ** -24
    return k * u / (1 - k * u)


def test_matmul_within_inner_product_bound():
    # |fl(A@B) - A@B| <= gamma_K |A|@|B| (Higham 3.5) catches a dropped term or transposed operand.
    r = np.random.default_rng(5)
    for (m, k, n) in [(9, 300, 13), (2, 1024, 40)]:
        a = r.standard_normal((m, k)).astype(np.float32)
        b = r.standard_normal((k, n)).astype(np.float32)
        got = oracle().reference_matmul(a, b).astype(np.float64)
        exact = a.astype(np.float64) @ b.astype(np.float64)
        bound = gamma(k) * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
        assert np.all(np.abs(got - exact) <= bound)


def test_dequant_closed_form():
    # Per-column, per-row, scalar and batch-axis planes against float32 numpy broadcasting.
    o = oracle()
    r = np.random.default_rng(6)
    k, n = 12, 10
    q = r.integers(-128, 128, size=2 * k * n, dtype=np.int8)
    zc = r.integers(-5, 6, size=n, dtype=np.int8)
    sc = r.uniform(0.01, 1, size=n).astype(np.float32)
    zr = r.integers(-5, 6, size=k, dtype=np.int8)
    sr = r.uniform(0.01, 1, size=k).astype(np.float32)
    qf = q.astype(np.float32).reshape(2, k, n)
    want_col = (qf - zc.astype(np.float32)) * sc
    want_row = (qf - zr.astype(np.float32)[:, None]) * sr[:, None]
    sb = np.array([0.5, 3.0], np.float32)
    want_batch = qf * sb[:, None, None]
    for (scale, zero, shape, axis, want) in [(sc, zc, [2, k, n], 2, want_col), (sr, zr, [2, k, n], 1, want_row),
                                             (sb, None, [2, k, n], 0, want_batch)]:
        plane, keep = make_plane(q, scale, zero, shape, axis)
        got = np.array([o.lib.orc_dequant_at(C.byref(plane), i) for i in range(q.size)], np.float32)
        same_bits(got, want.ravel())


def test_quantized_equals_float_matmul_of_dequantized():
    # MatMulQuantized == ReferenceMatMul(A, dequant(W)) bit for bit (tests/test_runtime.cc:365-367).
    o = oracle()
    for case in quant_cases():
        if case.get("bq") is None or case["k"] == 0:
            continue
        spec = case["bq"]
        plane, keep = make_plane(spec["q"], spec["scale"], spec["zero"], spec["shape"], spec["axis"], spec["offset"])
        kn = case["k"] * case["n"]
        w = np.array([o.lib.orc_dequant_at(C.byref(plane), spec["offset"] + i) for i in range(kn)], np.float32)
        same_bits(run_quant(o, case), o.reference_matmul(case["a"], w.reshape(case["k"], case["n"])))


def test_gelu_relu_closed_forms():
    import math

    x = np.linspace(-6, 6, 241).astype(np.float32)[None, :]
    o = oracle()
    relu = o.gemm_epilogue(x, 1.0, None, [], 0.0, 1)
    assert np.array_equal(relu, np.where(x < 0, 0, x))
    gelu = o.gemm_epilogue(x, 1.0, None, [], 0.0, 2).astype(np.float64)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x[0].astype(np.float64)])
    np.testing.assert_allclose(gelu[0], exact, rtol=2e-6, atol=1e-7)


def test_attention_is_softmax_weighted_mean():
    # One query against T keys equals softmax(qK^T/sqrt(d)) V in float64 within 1e-5.
    r = np.random.default_rng(7)
    q = r.standard_normal((1, 2, 8)).astype(np.float32)
    k = r.standard_normal((6, 1, 8)).astype(np.float32)
    v = r.standard_normal((6, 1, 8)).astype(np.float32)
    out = oracle().attention(q, k, v, 1, 5, 2, 1, 8)
    for h in range(2):
        s = (k[:, 0, :].astype(np.float64) @ q[0, h].astype(np.float64)) / np.sqrt(8)
        p = np.exp(s - s.max())
        p /= p.sum()
        np.testing.assert_allclose(out[0, h], p @ v[:, 0, :].astype(np.float64), atol=1e-5)


def test_sampling_distribution_invariants():
    # Greedy is argmax with the first index on ties; top_k=1 always returns the argmax;
    # every draw lands inside the top-k set.
    o = oracle()
    r = np.random.default_rng(8)
    for _ in range(50):
        logits = np.round(r.standard_normal(40) * 2).astype(np.float32)
        assert o.sample_token(logits, 0.0, 1, 0)[0] == int(np.argmax(logits))
        assert o.sample_token(logits, 1.0, int(r.integers(1, 2**31)), 1)[0] == int(np.argmax(logits))
        top5 = set(np.lexsort((np.arange(40), -logits))[:5].tolist())
        assert o.sample_token(logits, 1.3, int(r.integers(1, 2**31)), 5)[0] in top5


# ---- randomized, directly against the compiled reference (this container only) -------------

needs_ref = pytest.mark.skipif(reference() is None, reason="oracle/_ref not built (no reference tree)")


@needs_ref
def test_random_quantized_vs_reference():
    o, ref = oracle(), reference()
    r = np.random.default_rng(9)
    for _ in range(20):
        m, k, n = int(r.integers(1, 20)), int(r.integers(1, 300)), int(r.integers(1, 300))
        axis = int(r.integers(-1, 2))
        count = 1 if axis < 0 else (k if axis == 0 else n)
        q = r.integers(-128, 128, size=k * n, dtype=np.int8)
        s = r.uniform(1e-3, 1, size=count).astype(np.float32)
        z = r.integers(-8, 8, size=count, dtype=np.int8) if r.integers(0, 2) else None
        a = r.standard_normal((m, k)).astype(np.float32)
        plane, keep = make_plane(q, s, z, [k, n], axis)
        same_bits(o.matmul_quantized(a, None, None, plane, m, k, n), ref.matmul_quantized(a, None, None, plane, m, k, n))


@needs_ref
def test_random_kernels_vs_reference():
    o, ref = oracle(), reference()
    r = np.random.default_rng(10)
    for _ in range(10):
        m, n = int(r.integers(1, 9)), int(r.integers(1, 70))
        c = (r.standard_normal((m, n)) * 2).astype(np.float32)
        bias = r.standard_normal(n).astype(np.float32)
        act = int(r.integers(0, 3))
        same_bits(o.gemm_epilogue(c, 0.5, bias, [n], 2.0, act), ref.gemm_epilogue(c, 0.5, bias, [n], 2.0, act))
        x = r.standard_normal((3, 100)).astype(np.float32)
        w = r.standard_normal(100).astype(np.float32)
        same_bits(o.rmsnorm(x, w, 2, 100, 1e-5, 1), ref.rmsnorm(x, w, 2, 100, 1e-5, 1))
        q = r.standard_normal((2, 4, 16)).astype(np.float32)
        kk = r.standard_normal((9, 2, 16)).astype(np.float32)
        v = r.standard_normal((9, 2, 16)).astype(np.float32)
        same_bits(o.attention(q, kk, v, 2, 7, 4, 2, 16), ref.attention(q, kk, v, 2, 7, 4, 2, 16))
        logits = r.standard_normal(300).astype(np.float32)
        seed = int(r.integers(1, 2**32 - 1))
        assert o.sample_token(logits, 0.9, seed, 17) == ref.sample_token(logits, 0.9, seed, 17)


@needs_ref
def test_random_llama_vs_reference():
    # Tiny config, temperature sampling with top-k: ids must agree exactly.
    ref = reference()
    cfg = llama_config("tiny")
    w, _ = llama_weights(cfg, 211)
    prompt = np.random.default_rng(212).integers(0, cfg["vocab"], size=9).astype(np.int32)
    case = dict(name="rand", config=cfg, weights=w, prompt=prompt, max_new=20, eos=-1, temperature=1.1, seed=99,
                top_k=30)
    ids, _ = run_oracle_llama(case)
    from golden.make_golden import run_reference_llama

    ref_ids, _ = run_reference_llama(ref, case)
    assert np.array_equal(ids, ref_ids)
