"""Writes tests/golden/*.npz: inputs and the compiled reference's outputs.

The outputs come from oracle/_ref/libaccel_ref.so, i.e. AccelEP's own src/*.cc compiled
by oracle/Makefile (run `make -C oracle` first, with the reference tree present). The
fixtures are data only: seeded inputs plus what the reference computed on them. Tests
check the oracle restatement and the HIP kernels against them where the reference tree
is absent (a GPU host without the reference sources).

Run: python tests/golden/make_golden.py               (reference_outputs.npz)
     python tests/golden/make_golden.py --llama-full   (llama_smol_full.npz: the SmolLM2-135M-shape
                                                       forward, 30 layers, 512 + 128 tokens, greedy
                                                       and top-k; tens of minutes)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from oracle_ctypes import QuantPlane, fill_lcg, lcg_int8, make_plane, reference  # noqa: E402
from golden_cases import (  # noqa: E402
    attention_cases, embed_cases, epilogue_cases, llama_cases, llama_full_case, quant_cases, rmsnorm_cases,
    rope_cases, sample_cases, silu_add_cases)


def main():
    ref = reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libaccel_ref.so is missing: run `make -C oracle` with the reference tree present")
    if "--llama-full" in sys.argv:
        import time
        out = {}
        for case, prefix in ((llama_full_case(), ""), (llama_full_case(sampled=True), "topk_")):
            t0 = time.time()
            toks, logits = run_reference_llama(ref, case)
            steps, rows, gaps = run_reference_decode_rows(ref, case, toks, DECODE_ROW_STEPS)
            out[prefix + "ids"] = toks
            out[prefix + "prefill_logits"] = logits
            out[prefix + "decode_steps"] = steps
            out[prefix + "decode_logits"] = rows
            out[prefix + "top2_gap"] = gaps
            print(f"{case['name']}: {toks.size} ids ({np.unique(toks).size} distinct), min top-2 gap "
                  f"{gaps.min():.3g}, {time.time() - t0:.0f} s", flush=True)
        np.savez_compressed(HERE / "llama_smol_full.npz", **out)
        print(f"wrote {HERE / 'llama_smol_full.npz'}")
        return
    out = {}

    # SimDevice::MatMul and ReferenceMatMul on the reference test's LCG shapes (tests/test_runtime.cc:258-259).
    for (m, k, n, seed) in [(128, 160, 96, 1), (13, 19, 17, 2), (1, 2, 1, 0)]:
        a, s = fill_lcg(m * k, seed)
        b, _ = fill_lcg(k * n, s)
        a = a.reshape(m, k)
        b = b.reshape(k, n)
        key = f"matmul_{m}x{k}x{n}"
        out[key + "_a"] = a
        out[key + "_b"] = b
        out[key + "_device"] = ref.device_matmul(a, b)
        out[key + "_reference"] = ref.reference_matmul(a, b)

    for case in quant_cases():
        name = case["name"]
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
        c = ref.matmul_quantized(case.get("a"), planes["a"], case.get("b"), planes["b"], case["m"], case["k"], case["n"])
        out[f"quant_{name}_out"] = c

    for case in epilogue_cases():
        out[f"epi_{case['name']}_out"] = ref.gemm_epilogue(case["c"], case["alpha"], case["bias"], case["bias_shape"],
                                                           case["beta"], case["act"])

    for case in rmsnorm_cases():
        out[f"rms_{case['name']}_out"] = ref.rmsnorm(case["x"], case["w"], case["rows"], case["dim"], case["eps"],
                                                     case["row_offset"])
    for case in embed_cases():
        rc, o = ref.embed(case["ids"], case["id_offset"], case["table"], case["seq"])
        out[f"embed_{case['name']}_rc"] = np.int32(rc)
        out[f"embed_{case['name']}_out"] = o
    for case in rope_cases():
        out[f"rope_{case['name']}_out"] = ref.rope(case["states"], case["cos"], case["sin"], case["seq"],
                                                   case["heads"], case["head_dim"], case["position"])
    for case in attention_cases():
        out[f"attn_{case['name']}_out"] = ref.attention(case["q"], case["k"], case["v"], case["seq"], case["position"],
                                                        case["heads"], case["kv_heads"], case["head_dim"])
    for case in silu_add_cases():
        out[f"silu_{case['name']}_out"] = ref.silu_mul(case["gate"], case["up"])
        out[f"add_{case['name']}_out"] = ref.add(case["gate"], case["up"])
    ids = []
    states = []
    for case in sample_cases():
        i, st = ref.sample_token(case["logits"], case["temperature"], case["rng"], case["top_k"])
        ids.append(i)
        states.append(st)
    out["sample_ids"] = np.array(ids, np.int32)
    out["sample_rng_after"] = np.array(states, np.uint32)

    for case in llama_cases():
        toks, logits = run_reference_llama(ref, case)
        out[f"llama_{case['name']}_ids"] = toks
        out[f"llama_{case['name']}_prefill_logits"] = logits

    np.savez_compressed(HERE / "reference_outputs.npz", **out)
    print(f"wrote {len(out)} arrays to {HERE / 'reference_outputs.npz'}")


DECODE_ROW_STEPS = (1, 32, 64, 127)


def run_reference_decode_rows(ref, case, toks, keep_steps):
    """Logit rows of decode steps: after the prompt, step t forwards id toks[t - 1] at position
    len(prompt) + t - 1 and its row chooses toks[t]. The rows of `keep_steps` are stored (each
    the reference's own bits: the oracle restatement's row, kept only after the reference
    reports max|ref - row| == 0 at that step), with the top-1 minus top-2 logit gap of every
    row from the prefill (index 0) to the last decode step."""
    import ctypes as C
    from oracle_ctypes import F32P, I32P, LlamaConfig, oracle

    L = ref.lib
    O = oracle().lib
    cfg = LlamaConfig(**case["config"])
    h = L.accel_llama_create(C.byref(cfg))
    o = O.orc_llama_create(C.byref(cfg))
    assert h and o
    vocab = case["config"]["vocab"]
    try:
        for (kind, layer, w) in case["weights"]:
            w = np.ascontiguousarray(w, np.float32)
            rows, cols = (w.shape[0], 1) if w.ndim == 1 else w.shape
            assert L.accel_llama_weight(h, kind, layer, w.ctypes.data_as(F32P), rows, cols) == 0
            assert O.orc_llama_weight(o, kind, layer, w.ctypes.data_as(F32P), rows, cols) == 0
        prompt = np.ascontiguousarray(case["prompt"], np.int32)
        row = np.zeros(vocab, np.float32)
        mx = C.c_float()
        gaps = np.zeros(toks.size, np.float64)
        kept = []
        for t in range(toks.size):
            ids = prompt if t == 0 else np.ascontiguousarray(toks[t - 1:t], np.int32)
            assert L.accel_llama_forward_ids(h, ids.ctypes.data_as(I32P), ids.size, 1 if t == 0 else 0) == 0
            assert O.orc_llama_forward_ids(o, ids.ctypes.data_as(I32P), ids.size, 1 if t == 0 else 0) == 0
            assert O.orc_llama_logits(o, row.ctypes.data_as(F32P), vocab) == 0
            top = np.sort(row.astype(np.float64))[-2:]
            gaps[t] = top[1] - top[0]
            if t in keep_steps:
                assert L.accel_llama_logit_max_abs(h, row.ctypes.data_as(F32P), vocab, C.byref(mx)) == 0
                if mx.value != 0.0:
                    raise SystemExit(f"{case['name']}: oracle logits of step {t} differ from the reference by {mx.value}")
                kept.append(row.copy())
        return np.array(keep_steps, np.int32), np.stack(kept), gaps
    finally:
        L.accel_llama_destroy(h)
        O.orc_llama_destroy(o)


def run_reference_llama(ref, case):
    """Greedy/sampled ids from the reference's accel_llama_generate, plus the prefill logit row.

    The reference's C API never hands the logit row to the host; it compares it in place
    (accel_llama_logit_max_abs, src/llama_model.cc:168-181). The row stored here is the
    oracle restatement's, kept only after the reference reports max|ref - row| == 0 for it,
    i.e. it is the reference's row bit for bit.
    """
    import ctypes as C
    from oracle_ctypes import F32P, I32P, LlamaConfig, oracle

    L = ref.lib
    O = oracle().lib
    cfg = LlamaConfig(**case["config"])
    h = L.accel_llama_create(C.byref(cfg))
    o = O.orc_llama_create(C.byref(cfg))
    assert h, L.accel_llama_last_error()
    assert o
    try:
        for (kind, layer, w) in case["weights"]:
            w = np.ascontiguousarray(w, np.float32)
            rows, cols = (w.shape[0], 1) if w.ndim == 1 else w.shape
            assert L.accel_llama_weight(h, kind, layer, w.ctypes.data_as(F32P), rows, cols) == 0, \
                L.accel_llama_last_error()
            assert O.orc_llama_weight(o, kind, layer, w.ctypes.data_as(F32P), rows, cols) == 0
        prompt = np.ascontiguousarray(case["prompt"], np.int32)
        assert L.accel_llama_forward_ids(h, prompt.ctypes.data_as(I32P), prompt.size, 1) == 0, \
            L.accel_llama_last_error()
        assert O.orc_llama_forward_ids(o, prompt.ctypes.data_as(I32P), prompt.size, 1) == 0
        row = np.zeros(case["config"]["vocab"], np.float32)
        assert O.orc_llama_logits(o, row.ctypes.data_as(F32P), row.size) == 0
        mx = C.c_float()
        assert L.accel_llama_logit_max_abs(h, row.ctypes.data_as(F32P), row.size, C.byref(mx)) == 0
        if mx.value != 0.0:
            raise SystemExit(f"{case['name']}: oracle prefill logits differ from the reference by {mx.value}")
        out_ids = np.zeros(case["max_new"], np.int32)
        count = C.c_int32()
        rc = L.accel_llama_generate(h, prompt.ctypes.data_as(I32P), prompt.size, case["max_new"], case["eos"],
                                    case["temperature"], case["seed"], case["top_k"], out_ids.ctypes.data_as(I32P),
                                    C.byref(count))
        assert rc == 0, L.accel_llama_last_error()
        return out_ids[: count.value].copy(), row
    finally:
        L.accel_llama_destroy(h)
        O.orc_llama_destroy(o)


if __name__ == "__main__":
    main()
