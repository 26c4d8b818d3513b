"""Writes tests/golden/complete_cases.json: the compiled reference's accel_llama_complete_stream
(AccelEP src/llama_model.cc:183-206 and :530-551, through oracle/_ref/libaccel_ref.so) on
text prompts, with the fixture tokenizer (tokenizer_small.json) and the seeded weights of
golden_cases.complete_config() / COMPLETE_WEIGHT_SEED.

    make -C oracle && python3 tests/golden/make_complete.py

Each case keeps the prompt, the sampling arguments and what the reference returned: the ids,
the ids its token callback saw, the completion text, the prompt's token count, and the
simulator's counters over the call (accel_sim_matmuls, bytes to the device and to the host).
"""

from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from golden_cases import COMPLETE_WEIGHT_SEED, complete_config, llama_weights  # noqa: E402
from oracle_ctypes import REF_SO, LlamaConfig  # noqa: E402
from tokenizer_helpers import TOKENIZER_JSON, LlamaBpe  # noqa: E402

F32P = C.POINTER(C.c_float)
I32P = C.POINTER(C.c_int32)
TOKEN_FN = C.CFUNCTYPE(None, C.c_int32, C.c_void_p)


def open_reference():
    if not REF_SO.exists():
        raise SystemExit("oracle/_ref/libaccel_ref.so is missing: run `make -C oracle` with the reference tree present")
    L = C.CDLL(str(REF_SO))
    L.accel_llama_create.argtypes = [C.POINTER(LlamaConfig)]
    L.accel_llama_create.restype = C.c_void_p
    L.accel_llama_weight.argtypes = [C.c_void_p, C.c_int32, C.c_int32, F32P, C.c_int64, C.c_int64]
    L.accel_llama_complete_stream.argtypes = [
        C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.c_int32, C.c_float, C.c_uint32, C.c_int32, C.c_char_p,
        C.c_int32, I32P, I32P, C.c_int32, I32P, I32P, TOKEN_FN, C.c_void_p]
    L.accel_llama_last_error.restype = C.c_char_p
    for name in ("accel_sim_matmuls", "accel_sim_bytes_to_device", "accel_sim_bytes_to_host"):
        getattr(L, name).restype = C.c_int64
    cfg = complete_config()
    h = L.accel_llama_create(C.byref(LlamaConfig(**cfg)))
    assert h, L.accel_llama_last_error()
    h = C.c_void_p(h)
    weights, _ = llama_weights(cfg, COMPLETE_WEIGHT_SEED)
    for kind, layer, w in weights:
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = (w.shape[0], 1) if w.ndim == 1 else w.shape
        assert L.accel_llama_weight(h, kind, layer, w.ctypes.data_as(F32P), rows, cols) == 0, L.accel_llama_last_error()
    bpe = LlamaBpe(L, h)
    bpe.load(TOKENIZER_JSON)
    return L, h, bpe


def complete(L, h, prompt, max_new, eos, temperature, seed, top_k):
    data = prompt.encode("utf-8")
    text = C.create_string_buffer(1 << 16)
    text_len = C.c_int32(-1)
    ids = np.zeros(max(max_new, 1), np.int32)
    count = C.c_int32(-1)
    prompt_tokens = C.c_int32(-1)
    seen = []
    cb = TOKEN_FN(lambda tok, user: seen.append(int(tok)))
    L.accel_sim_reset_stats()
    rc = L.accel_llama_complete_stream(h, data, len(data), max_new, eos, temperature, seed, top_k, text, 1 << 16,
                                       C.byref(text_len), ids.ctypes.data_as(I32P), max_new, C.byref(count),
                                       C.byref(prompt_tokens), cb, None)
    assert rc == 0, L.accel_llama_last_error()
    counters = dict(matmuls=L.accel_sim_matmuls(), bytes_to_device=L.accel_sim_bytes_to_device(),
                    bytes_to_host=L.accel_sim_bytes_to_host())
    return dict(ids=ids[: count.value].tolist(), stream_ids=seen, text=text.raw[: text_len.value].decode("utf-8"),
                prompt_tokens=prompt_tokens.value, counters=counters)


def main():
    L, h, bpe = open_reference()
    cfg = complete_config()
    chat = "<|im_start|>user\nThe capital of France is<|im_end|>\n<|im_start|>assistant\n"
    # A prompt that leaves room for only a few tokens before the context is full.
    long_prompt = next(p for p in ("hello world " * r for r in range(1, 40)) if len(bpe.encode(p)) >= cfg["context"] - 5)
    assert len(bpe.encode(long_prompt)) <= cfg["context"]
    cases = [
        dict(name="greedy", prompt="The capital of France is", max_new=20, eos=-1, temperature=0.0, seed=0, top_k=0),
        dict(name="topk_chat", prompt=chat, max_new=24, eos=-1, temperature=0.8, seed=7, top_k=12),
        dict(name="full_vocab_sample", prompt="café 🎉 123, naïve façade", max_new=16, eos=-1, temperature=1.0,
             seed=3, top_k=0),
        dict(name="nul_and_dropped_bytes", prompt="a\x00b\x04c dog's day", max_new=10, eos=-1, temperature=0.0,
             seed=0, top_k=0),
        dict(name="context_limit", prompt=long_prompt, max_new=20, eos=-1, temperature=0.0, seed=0, top_k=0),
        dict(name="no_new_tokens", prompt="Hello", max_new=0, eos=-1, temperature=0.0, seed=0, top_k=0),
    ]
    for case in cases:
        case.update(complete(L, h, case["prompt"], case["max_new"], case["eos"], case["temperature"], case["seed"],
                             case["top_k"]))
    # Stop at an eos id: the fourth id of the sampled chat case, which the same call reaches again.
    base = next(c for c in cases if c["name"] == "topk_chat")
    eos_case = dict(name="eos_stop", prompt=base["prompt"], max_new=24, eos=base["ids"][3], temperature=0.8, seed=7,
                    top_k=12)
    eos_case.update(complete(L, h, eos_case["prompt"], 24, eos_case["eos"], 0.8, 7, 12))
    assert eos_case["ids"][-1] == eos_case["eos"] and len(eos_case["ids"]) <= 4
    cases.append(eos_case)
    for c in cases:
        assert c["ids"] == c["stream_ids"]
        print(f"{c['name']}: {c['prompt_tokens']} prompt ids, {len(c['ids'])} new: {c['text']!r}")
    out = dict(config=cfg, weight_seed=COMPLETE_WEIGHT_SEED, tokenizer=TOKENIZER_JSON.name, cases=cases)
    (HERE / "complete_cases.json").write_text(json.dumps(out, ensure_ascii=False, indent=1) + "\n", encoding="utf-8")
    print(f"wrote {HERE / 'complete_cases.json'}")


if __name__ == "__main__":
    main()
