"""The Llama loop on the GPU (include/accel_llama.h, accelep_amd/csrc/llama.cc) against the
compiled reference's outputs (AccelEP src/llama_model.cc through oracle/_ref, stored in
tests/golden/): the generated ids must be identical (greedy and top-k sampling), the
prefill logit row within max|diff| <= 1e-3 (the repository's logit gate,
tests/test_serve.py:353). The bound is needed because SiLU and attention use the device's
expf (within 1 ulp of glibc's, not bit-identical) and, by default, the matmuls add in
another order; with exact products on, only the expf differences remain.

Weights are the same seeded values given either as floats fl(q*s) (what the reference
receives) or as int8 q with per-row scales s (the HIP engine's int8 path); both must give the
reference's ids.
"""

from __future__ import annotations

import ctypes as C
import time
from pathlib import Path

import numpy as np
import pytest

from accelep_amd.capi import F32P, I8P, I32P, LlamaConfig, check, lib
from golden_cases import llama_cases, llama_config, llama_full_case, llama_weights

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
FULL_GOLDEN = Path(__file__).resolve().parent / "golden" / "llama_smol_full.npz"


class Engine:
    def __init__(self, config, weights, quant=None):
        self.L = lib()
        self.config = config
        self.h = self.L.accel_llama_create(C.byref(LlamaConfig(**config)))
        assert self.h, self.L.accel_llama_last_error()
        for (kind, layer, w) in weights:
            if quant is not None and (kind, layer) in quant:
                q, s = quant[(kind, layer)]
                q = np.ascontiguousarray(q, np.int8)
                s = np.ascontiguousarray(s, np.float32)
                rc = self.L.accel_llama_weight_q8(self.h, kind, layer, q.ctypes.data_as(I8P), s.ctypes.data_as(F32P),
                                                  q.shape[0], q.shape[1])
            else:
                w = np.ascontiguousarray(w, np.float32)
                rows, cols = (w.shape[0], 1) if w.ndim == 1 else w.shape
                rc = self.L.accel_llama_weight(self.h, kind, layer, w.ctypes.data_as(F32P), rows, cols)
            assert rc == 0, self.L.accel_llama_last_error()

    def close(self):
        self.L.accel_llama_destroy(self.h)

    def prefill_logits(self, prompt):
        prompt = np.ascontiguousarray(prompt, np.int32)
        assert self.L.accel_llama_forward_ids(self.h, prompt.ctypes.data_as(I32P), prompt.size, 1) == 0, \
            self.L.accel_llama_last_error()
        row = np.zeros(self.config["vocab"], np.float32)
        assert self.L.accel_llama_logits(self.h, row.ctypes.data_as(F32P), row.size) == 0
        return row

    def generate(self, case):
        prompt = np.ascontiguousarray(case["prompt"], np.int32)
        ids = np.zeros(case["max_new"], np.int32)
        count = C.c_int32()
        rc = self.L.accel_llama_generate(self.h, prompt.ctypes.data_as(I32P), prompt.size, case["max_new"],
                                         case["eos"], case["temperature"], case["seed"], case["top_k"],
                                         ids.ctypes.data_as(I32P), C.byref(count))
        assert rc == 0, self.L.accel_llama_last_error()
        return ids[: count.value]


@pytest.fixture(params=[False, True], ids=["fast", "exact"])
def products(request):
    L = lib()
    check(L.accel_hip_set_exact_products(1 if request.param else 0))
    yield request.param
    check(L.accel_hip_set_exact_products(0))


@pytest.mark.parametrize("weights", ["float", "int8"])
def test_llama_matches_reference_fixtures(gold, weights, products):
    for case in llama_cases():
        print(f"case {case['name']} weights={weights} exact={products}", flush=True)
        quant = llama_weights(case["config"], case["weight_seed"])[1] if weights == "int8" else None
        eng = Engine(case["config"], case["weights"], quant)
        try:
            row = eng.prefill_logits(case["prompt"])
            want = gold[f"llama_{case['name']}_prefill_logits"]
            worst = float(np.abs(row.astype(np.float64) - want).max())
            print(f"  prefill logits max|diff| = {worst:.3g}", flush=True)
            assert worst <= LOGIT_TOL
            assert int(np.argmax(row)) == int(np.argmax(want))
            ids = eng.generate(case)
            np.testing.assert_array_equal(ids, gold[f"llama_{case['name']}_ids"])
        finally:
            eng.close()


def _full_golden():
    if not FULL_GOLDEN.exists():
        pytest.skip("tests/golden/llama_smol_full.npz has not been generated")
    return np.load(FULL_GOLDEN)


def test_llama_full_size_matches_reference():
    """SmolLM2-135M shape (30 layers, 512 prompt ids, 128 greedy tokens), int8 weights: the
    prefill row and the decode rows of steps 1, 32, 64 and 127 within the logit gate of the
    reference's, and the generated ids (graph-replayed decode) identical. The top-1 minus top-2
    gap of each row is printed beside the measured error: an id is only as safe as that gap
    is wide."""
    gold = _full_golden()
    case = llama_full_case()
    eng = Engine(case["config"], case["weights"], case["quant"])
    try:
        vocab = case["config"]["vocab"]
        row = eng.prefill_logits(case["prompt"])
        worst = float(np.abs(row.astype(np.float64) - gold["prefill_logits"]).max())
        gaps = gold["top2_gap"]
        print(f"prefill logits max|diff| = {worst:.3g} (top-2 gap {gaps[0]:.3g})", flush=True)
        assert worst <= LOGIT_TOL
        ids_want = gold["ids"]
        steps = [int(t) for t in gold["decode_steps"]]
        rows = gold["decode_logits"]
        got_row = np.zeros(vocab, np.float32)
        for t in range(1, max(steps) + 1):
            one = np.ascontiguousarray(ids_want[t - 1:t], np.int32)
            assert eng.L.accel_llama_forward_ids(eng.h, one.ctypes.data_as(I32P), 1, 0) == 0, \
                eng.L.accel_llama_last_error()
            if t in steps:
                assert eng.L.accel_llama_logits(eng.h, got_row.ctypes.data_as(F32P), vocab) == 0
                err = float(np.abs(got_row.astype(np.float64) - rows[steps.index(t)]).max())
                print(f"decode step {t}: logits max|diff| = {err:.3g} (top-2 gap {gaps[t]:.3g})", flush=True)
                assert err <= LOGIT_TOL
                if gaps[t] > 2 * err:
                    assert int(np.argmax(got_row)) == int(ids_want[t])
        print(f"smallest top-2 gap over the 128 rows: {gaps.min():.3g} at row {int(np.argmin(gaps))}", flush=True)
        t0 = time.perf_counter()
        ids = eng.generate(case)
        dt = time.perf_counter() - t0
        print(f"generate: 512 prompt + {ids.size} new tokens in {dt * 1e3:.1f} ms", flush=True)
        np.testing.assert_array_equal(ids, ids_want)
    finally:
        eng.close()


def test_llama_full_size_prompt_in_parts_matches_reference():
    """The 512-id prompt fed in three parts (200, 137 and 175 ids, the later ones at positions
    200 and 337 against the cache): the prompt attention's key spans then start at a nonzero
    position and cross the parts' boundary. The last row's logits within the gate of the
    reference's prefill row."""
    gold = _full_golden()
    case = llama_full_case()
    eng = Engine(case["config"], case["weights"], case["quant"])
    try:
        prompt = np.ascontiguousarray(case["prompt"], np.int32)
        for lo, hi in ((0, 200), (200, 337), (337, prompt.size)):
            part = np.ascontiguousarray(prompt[lo:hi])
            assert eng.L.accel_llama_forward_ids(eng.h, part.ctypes.data_as(I32P), part.size, int(lo == 0)) == 0, \
                eng.L.accel_llama_last_error()
        row = np.zeros(case["config"]["vocab"], np.float32)
        assert eng.L.accel_llama_logits(eng.h, row.ctypes.data_as(F32P), row.size) == 0
        worst = float(np.abs(row.astype(np.float64) - gold["prefill_logits"]).max())
        print(f"prompt in three parts: logits max|diff| = {worst:.3g}", flush=True)
        assert worst <= LOGIT_TOL
    finally:
        eng.close()


def test_llama_full_size_sampled_matches_reference():
    """The same model with top-k sampling (temperature 0.8, top 40, seed 11): 128 ids that do
    not settle on a fixed point, so every decode position and KV row takes part. The ids must
    be the reference's, the decode rows of steps 1, 32, 64 and 127 within the logit gate."""
    gold = _full_golden()
    if "topk_ids" not in gold.files:
        pytest.skip("tests/golden/llama_smol_full.npz has no sampled case")
    case = llama_full_case(sampled=True)
    eng = Engine(case["config"], case["weights"], case["quant"])
    try:
        ids = eng.generate(case)
        want = gold["topk_ids"]
        print(f"sampled: {np.unique(want).size} distinct ids of {want.size}", flush=True)
        np.testing.assert_array_equal(ids, want)
        vocab = case["config"]["vocab"]
        eng.prefill_logits(case["prompt"])
        steps = [int(t) for t in gold["topk_decode_steps"]]
        got_row = np.zeros(vocab, np.float32)
        for t in range(1, max(steps) + 1):
            one = np.ascontiguousarray(want[t - 1:t], np.int32)
            assert eng.L.accel_llama_forward_ids(eng.h, one.ctypes.data_as(I32P), 1, 0) == 0
            if t in steps:
                assert eng.L.accel_llama_logits(eng.h, got_row.ctypes.data_as(F32P), vocab) == 0
                err = float(np.abs(got_row.astype(np.float64) - gold["topk_decode_logits"][steps.index(t)]).max())
                print(f"sampled decode step {t}: logits max|diff| = {err:.3g}", flush=True)
                assert err <= LOGIT_TOL
    finally:
        eng.close()


def _decode_row_logits(eng, cfg, prompt, fuse):
    """Last-row logits after a prompt forward of prompt[:-1] and a one-row forward of the last id."""
    assert eng.L.accel_llama_set_fused_inputs(eng.h, fuse) == 0
    head, last = np.ascontiguousarray(prompt[:-1]), np.ascontiguousarray(prompt[-1:])
    assert eng.L.accel_llama_forward_ids(eng.h, head.ctypes.data_as(I32P), head.size, 1) == 0
    assert eng.L.accel_llama_forward_ids(eng.h, last.ctypes.data_as(I32P), 1, 0) == 0
    row = np.zeros(cfg["vocab"], np.float32)
    assert eng.L.accel_llama_logits(eng.h, row.ctypes.data_as(F32P), row.size) == 0
    return row


@pytest.mark.parametrize("count", [9, 64, 65, 150, 8250])
def test_decode_row_fused_kernels_match_separate_passes(count):
    """A one-row forward runs RoPE, the KV append, the chunked attention and its combine as one
    kernel (mask 2): the logits must carry exactly the bits of the three-kernel forward (mask 0).
    With the RMSNorms and SiLU*up inside the GEMVs as well (mask 3, the norm applied to the
    sums), and with the attention in fixed splits combined inside the o-projection GEMV (mask 4
    alone, and 7, the default), they agree to rounding and pick the same id. The prompt
    lengths put the new position inside the first 64-position chunk (and leave three of the
    eight splits empty), at its last slot, at the first slot of the second, in a third chunk,
    and in the 129th (64 splits of 129 positions)."""
    cfg = dict(llama_config("smol3"), layers=2, context=max(160, count + 16))
    w, q = llama_weights(cfg, 103)
    prompt = np.random.default_rng(5).integers(0, cfg["vocab"], size=count).astype(np.int32)
    eng = Engine(cfg, w, q)
    try:
        rows = {fuse: _decode_row_logits(eng, cfg, prompt, fuse) for fuse in (0, 2, 3, 4, 7)}
        np.testing.assert_array_equal(rows[2].view(np.uint32), rows[0].view(np.uint32))
        for fuse in (3, 4, 7):
            assert np.isfinite(rows[fuse]).all()
            err = float(np.abs(rows[fuse] - rows[0]).max())
            print(f"count {count} mask {fuse}: max|logit - separate passes| = {err:.3g}", flush=True)
            np.testing.assert_allclose(rows[fuse], rows[0], rtol=1e-4, atol=1e-4)
            assert int(np.argmax(rows[fuse])) == int(np.argmax(rows[0]))
        assert eng.L.accel_llama_set_fused_inputs(eng.h, 8) == 1
        assert b"enable must be 0 .. 7" in eng.L.accel_llama_last_error()
    finally:
        eng.close()


def test_llama_errors():
    L = lib()
    bad = LlamaConfig(vocab=16, hidden=30, layers=1, heads=4, kv_heads=2, intermediate=8, context=4, eps=1e-5,
                      rope_theta=1e4)
    assert not L.accel_llama_create(C.byref(bad))
    assert b"invalid llama config" in L.accel_llama_last_error()
    cfg = dict(vocab=32, hidden=16, layers=1, heads=2, kv_heads=1, intermediate=8, context=8, eps=1e-5,
               rope_theta=1e4)
    h = L.accel_llama_create(C.byref(LlamaConfig(**cfg)))
    assert h
    try:
        w = np.zeros((5, 5), np.float32)
        assert L.accel_llama_weight(h, 6, 0, w.ctypes.data_as(F32P), 5, 5) == 1
        assert b"invalid weight" in L.accel_llama_last_error()
        prompt = np.array([1, 2], np.int32)
        out = np.zeros(4, np.int32)
        n = C.c_int32()
        assert L.accel_llama_generate(h, prompt.ctypes.data_as(I32P), 2, 4, -1, 0.0, 0, 0, out.ctypes.data_as(I32P),
                                      C.byref(n)) == 1
        assert b"incomplete" in L.accel_llama_last_error()
        weights, _ = llama_weights(cfg, 5, quantize=False)
        eng = Engine.__new__(Engine)
        eng.L, eng.config, eng.h = L, cfg, h
        for (kind, layer, wt) in weights:
            wt = np.ascontiguousarray(wt, np.float32)
            rows, cols = (wt.shape[0], 1) if wt.ndim == 1 else wt.shape
            assert L.accel_llama_weight(h, kind, layer, wt.ctypes.data_as(F32P), rows, cols) == 0
        oov = np.array([1, 99], np.int32)
        assert L.accel_llama_forward_ids(h, oov.ctypes.data_as(I32P), 2, 1) == 1
        assert b"outside the vocabulary" in L.accel_llama_last_error()
        long = np.ones(9, np.int32)
        assert L.accel_llama_forward_ids(h, long.ctypes.data_as(I32P), 9, 1) == 1
        assert b"exceeds context" in L.accel_llama_last_error()
    finally:
        L.accel_llama_destroy(h)


def _head_scale_cases(t, v):
    """Per-row scales of an LM head whose rows repeat 8 int8 patterns, so logit o is
    fl(T[o % 8] * s[o]) with T the 8 sums the hidden row gives (read with s = 1): crafted
    maxima, ties, signed zeros, NaNs and infinities over a ragged vocabulary of v ids."""
    sign = np.where(t[np.arange(v) % 8] < 0, -1.0, 1.0).astype(np.float32)
    r = np.random.default_rng(31)
    base = (r.uniform(1e-3, 1e-2, v) * r.choice([-1.0, 1.0], v)).astype(np.float32)
    yield "random", base
    s = np.ones(v, np.float32)
    yield "ties_across_tiles", s  # every slot's value repeats in every tile: the earliest id wins
    s = (-np.abs(base) * sign).astype(np.float32)  # every logit negative
    s[[3000, 1200]] = 0.0
    s[1200] = -0.0 * sign[1200]  # -0 at 1200, +0 at 3000: equal values, 1200 wins
    yield "signed_zero", s
    s = base.copy(); s[0] = np.nan
    yield "nan_at_0", s
    s = base.copy(); s[[1, 7, 2048, 4000, v - 2]] = np.nan; s[999] = 10.0 * sign[999]
    yield "nan_elsewhere", s
    s = np.full(v, np.nan, np.float32); s[0] = -3.0
    yield "all_nan_but_0", s
    yield "all_neg_inf", (-np.inf * sign).astype(np.float32)
    s = base.copy(); s[v - 1] = np.inf * sign[v - 1]
    yield "inf_in_ragged_tail", s


@pytest.mark.parametrize("vocab", [4099, 16387])
def test_head_greedy_keys_pick_matches_oracle(vocab):
    """The LM head's GEMV stores a greedy key per 8-column tile and one workgroup reduces them:
    a generate's first id equals the oracle's strict > scan over the logits that the same
    forward leaves on the device, for crafted rows (ties across tiles, -0 beside +0, NaN at id 0
    and elsewhere, all NaN, all -inf, +inf in a partial last tile of a ragged vocabulary). With
    4099 ids the head is the one-workgroup-per-tile GEMV after a norm pass; with 16387 (2049
    tiles) it is the one-wave-per-tile GEMV with the norm inside. In exact-products mode (no
    keys) the many-workgroup greedy kernel gives the oracle's id for its own logits too."""
    from oracle_ctypes import oracle

    cfg = dict(llama_config("tiny"), vocab=vocab)
    w, q = llama_weights(cfg, 17)
    w = [(k, l, a) for (k, l, a) in w if k != 3]  # the head is uploaded per case below
    prompt = np.random.default_rng(3).integers(0, cfg["vocab"], size=9).astype(np.int32)
    pattern = np.random.default_rng(4).integers(-127, 128, size=(8, cfg["hidden"])).astype(np.int8)
    head_q = np.ascontiguousarray(pattern[np.arange(cfg["vocab"]) % 8])
    eng = Engine(cfg, w, q)
    try:
        def set_head(scale):
            s = np.ascontiguousarray(scale, np.float32)
            assert eng.L.accel_llama_weight_q8(eng.h, 3, -1, head_q.ctypes.data_as(I8P), s.ctypes.data_as(F32P),
                                               head_q.shape[0], head_q.shape[1]) == 0, eng.L.accel_llama_last_error()

        case = dict(prompt=prompt, max_new=1, eos=-1, temperature=0.0, seed=0, top_k=0)
        for exact in (0, 1):
            check(eng.L.accel_hip_set_exact_products(exact))
            set_head(np.ones(cfg["vocab"], np.float32))
            t = eng.prefill_logits(prompt)[:8].copy()
            assert np.all(t != 0) and np.isfinite(t).all()
            for name, scale in _head_scale_cases(t, cfg["vocab"]):
                set_head(scale)
                got = int(eng.generate(case)[0])
                row = eng.prefill_logits(prompt)
                want, _ = oracle().sample_token(row, 0.0, 1, 0)
                print(f"exact {exact} {name}: gpu {got} oracle {want}", flush=True)
                assert got == want
    finally:
        check(eng.L.accel_hip_set_exact_products(0))
        eng.close()


def test_greedy_pick_in_step_matches_sampler_path():
    """A greedy generate with no eos id and no callback picks each id inside the next decode
    step (GreedyEmbedKernel); with an eos id that never occurs the sampler runs between the
    steps and the host reads each id. Both must give the same ids and count, here through the
    end of the context (48 positions: 40 prompt ids, 8 decode steps, a ninth id with no forward
    after it), and the reference's ids on the golden greedy case."""
    cfg = llama_config("tiny")
    w, q = llama_weights(cfg, 101)
    prompt = np.random.default_rng(9).integers(0, cfg["vocab"], size=40).astype(np.int32)
    eng = Engine(cfg, w, q)
    try:
        base = dict(prompt=prompt, max_new=12, temperature=0.0, seed=0, top_k=0)
        in_step = eng.generate(dict(base, eos=-1))
        sampler = eng.generate(dict(base, eos=cfg["vocab"] + 5))
        print(f"in-step {in_step.tolist()} sampler {sampler.tolist()}", flush=True)
        assert in_step.size == 9
        np.testing.assert_array_equal(in_step, sampler)
    finally:
        eng.close()
