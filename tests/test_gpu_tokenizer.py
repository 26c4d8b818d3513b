"""accel_llama_tokenizer / encode / decode / complete / complete_stream through the C-ABI
(include/accel_llama.h) on the GPU engine, against the compiled reference's own completions
(tests/golden/complete_cases.json, from AccelEP's accel_llama_complete_stream) and the
tokenizer oracle (oracle/bpe.py, pinned in tests/test_tokenizer.py).

* encode / decode on a model handle give the fixture ids and text (`tokenizers`' values) and
  the oracle's on seeded random inputs;
* complete and complete_stream give the reference's ids, callback ids, text and prompt token
  count, for float and int8 weights in both product modes (the same ids as
  tests/test_gpu_llama.py requires of generate);
* complete's ids equal generate's on the encoded prompt; the copy counters hold the prompt
  ids in, the ids and the text out (AccelEP tests/test_serve.py:363-364), and accel_sim_matmuls
  and the byte counters read what the reference's read over the same completion;
* every error of src/llama_model.cc:183-206 and :449-551 is raised with its message.
"""

from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

from accelep_amd.capi import F32P, I8P, I32P, TOKEN_FN, LlamaConfig, Stats, check, lib
from golden_cases import COMPLETE_WEIGHT_SEED, complete_config, llama_weights
from oracle.bpe import Bpe
from tokenizer_helpers import TOKENIZER_JSON, LlamaBpe, TokenizerError, cases, random_ids, random_texts

pytestmark = pytest.mark.gpu

COMPLETE_JSON = Path(__file__).resolve().parent / "golden" / "complete_cases.json"


def _golden():
    return json.loads(COMPLETE_JSON.read_text(encoding="utf-8"))


class Model:
    def __init__(self, quant=False, weights=True, tokenizer=True):
        self.L = lib()
        self.cfg = complete_config()
        self.h = self.L.accel_llama_create(C.byref(LlamaConfig(**self.cfg)))
        assert self.h, self.L.accel_llama_last_error()
        if weights:
            w, q = llama_weights(self.cfg, COMPLETE_WEIGHT_SEED)
            for kind, layer, arr in w:
                if quant and (kind, layer) in q:
                    qq, s = (np.ascontiguousarray(x) for x in q[(kind, layer)])
                    rc = self.L.accel_llama_weight_q8(self.h, kind, layer, qq.ctypes.data_as(I8P),
                                                      s.ctypes.data_as(F32P), qq.shape[0], qq.shape[1])
                else:
                    arr = np.ascontiguousarray(arr, np.float32)
                    rows, cols = (arr.shape[0], 1) if arr.ndim == 1 else arr.shape
                    rc = self.L.accel_llama_weight(self.h, kind, layer, arr.ctypes.data_as(F32P), rows, cols)
                assert rc == 0, self.L.accel_llama_last_error()
        self.bpe = LlamaBpe(self.L, C.c_void_p(self.h))
        if tokenizer:
            self.bpe.load(TOKENIZER_JSON)

    def close(self):
        self.L.accel_llama_destroy(self.h)

    def error(self):
        return self.L.accel_llama_last_error().decode()

    def complete(self, prompt, max_new, eos=-1, temperature=0.0, seed=0, top_k=0, stream=True, text_cap=1 << 16,
                 ids_cap=None, prompt_tokens=True):
        data = prompt.encode("utf-8") if isinstance(prompt, str) else prompt
        ids_cap = max_new if ids_cap is None else ids_cap
        text = C.create_string_buffer(max(text_cap, 1))
        text_len = C.c_int32(-1)
        ids = np.full(max(ids_cap, 1), -1, np.int32)
        count = C.c_int32(-1)
        ptok = C.c_int32(-1)
        seen = []
        if stream:
            cb = TOKEN_FN(lambda tok, user: seen.append(int(tok)))
            rc = self.L.accel_llama_complete_stream(self.h, data, len(data), max_new, eos, temperature, seed, top_k,
                                                    text, text_cap, C.byref(text_len), ids.ctypes.data_as(I32P),
                                                    ids_cap, C.byref(count), C.byref(ptok) if prompt_tokens else None,
                                                    C.cast(cb, C.c_void_p), None)
        else:
            rc = self.L.accel_llama_complete(self.h, data, len(data), max_new, eos, temperature, seed, top_k, text,
                                             text_cap, C.byref(text_len), ids.ctypes.data_as(I32P), ids_cap,
                                             C.byref(count), C.byref(ptok) if prompt_tokens else None)
        if rc != 0:
            raise TokenizerError(self.error())
        return dict(ids=ids[: count.value].tolist(), stream_ids=seen, text=text.raw[: text_len.value].decode("utf-8"),
                    prompt_tokens=ptok.value)

    def generate(self, prompt_ids, max_new, eos=-1, temperature=0.0, seed=0, top_k=0):
        p = np.ascontiguousarray(prompt_ids, np.int32)
        ids = np.zeros(max(max_new, 1), np.int32)
        count = C.c_int32()
        rc = self.L.accel_llama_generate(self.h, p.ctypes.data_as(I32P), p.size, max_new, eos, temperature, seed,
                                         top_k, ids.ctypes.data_as(I32P), C.byref(count))
        assert rc == 0, self.error()
        return ids[: count.value].tolist()


@pytest.fixture(scope="module")
def orc():
    return Bpe(TOKENIZER_JSON)


@pytest.fixture(params=[False, True], ids=["fast", "exact"])
def products(request):
    L = lib()
    check(L.accel_hip_set_exact_products(1 if request.param else 0))
    yield request.param
    check(L.accel_hip_set_exact_products(0))


def test_golden_matches_the_tokenizer_fixture():
    g = _golden()
    assert g["config"] == complete_config() and g["weight_seed"] == COMPLETE_WEIGHT_SEED
    assert g["tokenizer"] == TOKENIZER_JSON.name
    assert cases()["vocab_size"] == complete_config()["vocab"]


def test_encode_decode_on_a_model(orc):
    m = Model(weights=False)
    try:
        data = cases()
        for c in data["encode"]:
            print(f"encode {c['text']!r}", flush=True)
            assert m.bpe.encode(c["text"]) == c["ids"]
            assert m.bpe.decode(c["ids"]) == c["decoded"]
        for c in data["decode"]:
            for skip in (True, False):
                assert m.bpe.decode(c["ids"], skip) == orc.decode(c["ids"], skip), c["ids"]
        for text in random_texts(200, 31):
            assert m.bpe.encode(text) == orc.encode(text), repr(text)
        for ids in random_ids(200, 32, complete_config()["vocab"]):
            assert m.bpe.decode(ids, False) == orc.decode(ids, False), ids
    finally:
        m.close()


@pytest.mark.parametrize("weights", ["float", "int8"])
def test_complete_matches_the_reference(weights, products, orc):
    m = Model(quant=(weights == "int8"))
    try:
        for c in _golden()["cases"]:
            print(f"complete {c['name']} weights={weights} exact={products}", flush=True)
            m.L.accel_sim_reset_stats()
            got = m.complete(c["prompt"], c["max_new"], c["eos"], c["temperature"], c["seed"], c["top_k"])
            counters = dict(matmuls=m.L.accel_sim_matmuls(), bytes_to_device=m.L.accel_sim_bytes_to_device(),
                            bytes_to_host=m.L.accel_sim_bytes_to_host())
            assert counters == c["counters"]  # the reference's accel_sim_* over the same call
            assert got["ids"] == c["ids"]
            assert got["stream_ids"] == c["stream_ids"] == c["ids"]
            assert got["text"] == c["text"] == orc.decode(c["ids"], True)
            assert got["prompt_tokens"] == c["prompt_tokens"] == len(orc.encode(c["prompt"]))
            plain = m.complete(c["prompt"], c["max_new"], c["eos"], c["temperature"], c["seed"], c["top_k"],
                               stream=False)
            assert plain["ids"] == c["ids"] and plain["text"] == c["text"] and plain["stream_ids"] == []
    finally:
        m.close()


def test_complete_is_generate_of_the_encoded_prompt(orc):
    m = Model(quant=True)
    try:
        for prompt, kw in [("The capital of France is", dict(temperature=0.0)),
                           ("memory stream graph", dict(temperature=0.9, seed=5, top_k=30)),
                           ("x<|endoftext|>y 42", dict(temperature=0.7, seed=9, top_k=0))]:
            got = m.complete(prompt, 12, **kw)
            assert got["ids"] == m.generate(m.bpe.encode(prompt), 12, **kw)
            assert got["text"] == m.bpe.decode(got["ids"], True) == orc.decode(got["ids"], True)
    finally:
        m.close()


def test_complete_copies_only_the_prompt_ids_the_ids_and_the_text():
    L = lib()
    m = Model(quant=True)
    try:
        m.complete("warm up", 4)
        L.accel_hip_reset_stats()
        got = m.complete("The capital of France is", 8)
        st = Stats()
        L.accel_hip_get_stats(C.byref(st))
        assert st.bytes_to_device == got["prompt_tokens"] * 4
        assert st.bytes_to_host == len(got["text"].encode("utf-8")) + len(got["ids"]) * 4
    finally:
        m.close()


def test_errors():
    m = Model(tokenizer=False)
    try:
        with pytest.raises(TokenizerError, match="tokenizer is not loaded"):
            m.complete("hi", 2)
        with pytest.raises(TokenizerError, match="tokenizer is not loaded"):
            m.bpe.encode("hi")
        with pytest.raises(TokenizerError, match="invalid tokenizer"):
            m.bpe.load("")
        with pytest.raises(TokenizerError):
            m.bpe.load("/nonexistent/tokenizer.json")
        m.bpe.load(TOKENIZER_JSON)
        ctx = m.cfg["context"]
        with pytest.raises(TokenizerError, match="prompt encoded to no tokens"):
            m.complete("\x04\x00", 2)
        with pytest.raises(TokenizerError, match="prompt encoded to no tokens"):
            m.complete("", 2)
        with pytest.raises(TokenizerError, match="prompt exceeds context"):
            m.complete(" ".join(["hello world"] * ctx), 2)
        with pytest.raises(TokenizerError, match="prompt is not utf-8"):
            m.complete(b"ab\xff", 2)
        with pytest.raises(TokenizerError, match="invalid complete"):
            m.complete("hi", 4, ids_cap=3)
        with pytest.raises(TokenizerError, match="invalid complete"):
            m.complete("hi", 2, prompt_tokens=False)
        with pytest.raises(TokenizerError, match="invalid complete"):
            m.complete("hi", -1)
        with pytest.raises(TokenizerError, match="completion text buffer is too small"):
            m.complete("The capital of France is", 8, text_cap=1)
        with pytest.raises(TokenizerError, match="encode buffer is too small"):
            m.bpe.encode("The capital of France is", cap=2)
        with pytest.raises(TokenizerError, match="decode buffer is too small"):
            m.bpe.decode(m.bpe.encode("The capital of France is"), cap=3)
        with pytest.raises(TokenizerError, match="outside the vocabulary"):
            m.bpe.decode([m.cfg["vocab"]])
        text = C.create_string_buffer(8)
        n = C.c_int32()
        assert m.L.accel_llama_decode(m.h, None, 0, 1, None, 8, C.byref(n)) == 1
        assert m.error() == "invalid decode"
        assert m.L.accel_llama_decode(m.h, None, 0, 1, text, 8, C.byref(n)) == 0 and n.value == 0
    finally:
        m.close()
    bare = Model(weights=False)
    try:
        with pytest.raises(TokenizerError, match="llama weights are incomplete"):
            bare.complete("hi", 2)
    finally:
        bare.close()
