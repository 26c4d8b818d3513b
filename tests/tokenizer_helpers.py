"""Bindings and inputs shared by the tokenizer tests.

* HostBpe: the library's tokenizer (accelep_amd/csrc/tokenizer.cc) through
  tests/cpp/bin/libbpe_host.so, a test-only C shim with no model and no GPU.
* RefBpe: the compiled reference (oracle/_ref/libaccel_ref.so) through its own
  accel_llama_create / tokenizer / encode / decode on a tiny simulated model; None when the
  reference was not built.
* LlamaBpe: any accel_llama_* library's encode / decode on a model handle.
* random_texts / random_ids: seeded inputs over the character classes the pattern tells apart.
"""

from __future__ import annotations

import ctypes as C
import json
import random
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
TOKENIZER_JSON = GOLDEN / "tokenizer_small.json"
CASES_JSON = GOLDEN / "tokenizer_cases.json"
HOST_SO = ROOT / "tests" / "cpp" / "bin" / "libbpe_host.so"
REF_SO = ROOT / "oracle" / "_ref" / "libaccel_ref.so"
I32P = C.POINTER(C.c_int32)


def cases():
    return json.loads(CASES_JSON.read_text(encoding="utf-8"))


class TokenizerError(RuntimeError):
    pass


class _Calls:
    """encode/decode over functions with accel_llama_encode / decode's arguments."""

    def __init__(self, handle, encode, decode, error):
        self.h = handle
        self._encode = encode
        self._decode = decode
        self._error = error

    def encode(self, text, cap=1 << 16):
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        out = (C.c_int32 * max(cap, 1))()
        count = C.c_int32(-1)
        if self._encode(self.h, data, len(data), out, cap, C.byref(count)) != 0:
            raise TokenizerError(self._error().decode())
        return list(out[: count.value])

    def decode(self, ids, skip_special=True, cap=1 << 18):
        arr = (C.c_int32 * max(len(ids), 1))(*ids)
        buf = C.create_string_buffer(max(cap, 1))
        n = C.c_int32(-1)
        if self._decode(self.h, arr, len(ids), int(skip_special), buf, cap, C.byref(n)) != 0:
            raise TokenizerError(self._error().decode())
        return buf.raw[: n.value].decode("utf-8")


def _sign(lib, prefix):
    getattr(lib, prefix + "encode").argtypes = [C.c_void_p, C.c_char_p, C.c_int32, I32P, C.c_int32, I32P]
    getattr(lib, prefix + "decode").argtypes = [C.c_void_p, I32P, C.c_int32, C.c_int32, C.c_char_p, C.c_int32, I32P]


class HostBpe(_Calls):
    def __init__(self, path=TOKENIZER_JSON):
        if not HOST_SO.exists():
            raise RuntimeError(f"{HOST_SO} is not built (run __graft_entry__.build())")
        lib = C.CDLL(str(HOST_SO))
        lib.bpe_host_create.restype = C.c_void_p
        lib.bpe_host_destroy.argtypes = [C.c_void_p]
        lib.bpe_host_load.argtypes = [C.c_void_p, C.c_char_p]
        lib.bpe_host_error.restype = C.c_char_p
        lib.bpe_host_vocab_size.argtypes = [C.c_void_p]
        _sign(lib, "bpe_host_")
        self.lib = lib
        super().__init__(C.c_void_p(lib.bpe_host_create()), lib.bpe_host_encode, lib.bpe_host_decode,
                         lib.bpe_host_error)
        if path is not None:
            self.load(path)

    def load(self, path):
        if self.lib.bpe_host_load(self.h, str(path).encode()) != 0:
            raise TokenizerError(self.lib.bpe_host_error().decode())

    def vocab_size(self):
        return self.lib.bpe_host_vocab_size(self.h)

    def close(self):
        self.lib.bpe_host_destroy(self.h)


class LlamaBpe(_Calls):
    """encode/decode of an accel_llama_* library on an existing model handle."""

    def __init__(self, lib, handle):
        _sign(lib, "accel_llama_")
        lib.accel_llama_tokenizer.argtypes = [C.c_void_p, C.c_char_p]
        lib.accel_llama_last_error.restype = C.c_char_p
        self.lib = lib
        super().__init__(handle, lib.accel_llama_encode, lib.accel_llama_decode, lib.accel_llama_last_error)

    def load(self, path):
        if self.lib.accel_llama_tokenizer(self.h, str(path).encode()) != 0:
            raise TokenizerError(self.lib.accel_llama_last_error().decode())


class _RefConfig(C.Structure):
    """AccelLlamaConfig (include/accel/sim_api.h:44-54)."""

    _fields_ = [(n, C.c_int32) for n in ("vocab", "hidden", "layers", "heads", "kv_heads", "intermediate",
                                         "context")] + [("eps", C.c_float), ("rope_theta", C.c_float)]


class RefBpe(LlamaBpe):
    """The reference's tokenizer on a tiny simulated model (no weights needed to encode)."""

    def __init__(self, path=TOKENIZER_JSON):
        lib = C.CDLL(str(REF_SO))
        lib.accel_llama_create.argtypes = [C.POINTER(_RefConfig)]
        lib.accel_llama_create.restype = C.c_void_p
        lib.accel_llama_destroy.argtypes = [C.c_void_p]
        cfg = _RefConfig(vocab=8, hidden=8, layers=1, heads=1, kv_heads=1, intermediate=8, context=8, eps=1e-5,
                         rope_theta=10000.0)
        handle = lib.accel_llama_create(C.byref(cfg))
        assert handle, lib.accel_llama_last_error()
        super().__init__(lib, C.c_void_p(handle))
        if path is not None:
            self.load(path)

    def unicode_ranges(self, which):
        """The reference's class table (src/unicode_cats.inc): [(first, last), ...]."""
        self.lib.ref_unicode_ranges.argtypes = [C.c_int32, C.POINTER(C.POINTER(C.c_uint32)), I32P]
        pairs = C.POINTER(C.c_uint32)()
        count = C.c_int32()
        assert self.lib.ref_unicode_ranges(which, C.byref(pairs), C.byref(count)) == 0
        return [(pairs[2 * i], pairs[2 * i + 1]) for i in range(count.value)]

    def close(self):
        self.lib.accel_llama_destroy(self.h)


def reference_bpe(path=TOKENIZER_JSON):
    return RefBpe(path) if REF_SO.exists() else None


# ---- seeded inputs -----------------------------------------------------------------------

POOLS = {
    "lower": "abcdefghijklmnopqrstuvwxyz",
    "upper": "ABCDEFGHIJKLMNOPQRSTUVWXYZ",
    "digit": "0123456789",
    "number": "٣٤०१①②²³½ⅫⅣ¼",
    "letter": "éüßçñøÆΩλπжщ中文日本語한국어אבعربहि",
    "space": " \t\n\r\x0b\x0c\x85\xa0        　",
    "punct": ".,;:!?-_/\\()[]{}<>@#$%^&*+=~`|\"",
    "quote": "'",
    "emoji": "😀🎉👍🏽🚀∑√€£¥—…«»",
    "control": "\x00\x01\x04\x07\x08\x0e\x11\x19\x1a\x1b\x1f\x7f",
    "contraction": ["'s", "'t", "'re", "'ve", "'m", "'ll", "'d", "'S", "'Re"],
    "word": ["the", "capital", "France", "hello", "world", "model", "stream", "tokenizer", "byte"],
    "special": ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|im_start", "|>"],
}


def random_texts(count, seed, max_parts=24, special=True):
    r = random.Random(seed)
    names = [n for n in POOLS if special or n != "special"]
    out = []
    for _ in range(count):
        parts = []
        for _ in range(r.randint(0, max_parts)):
            pool = POOLS[r.choice(names)]
            parts.append(r.choice(pool) * (r.randint(1, 3) if r.random() < 0.2 else 1))
        out.append("".join(parts))
    return out


def random_ids(count, seed, vocab, max_len=40):
    r = random.Random(seed)
    return [[r.randrange(vocab) for _ in range(r.randint(0, max_len))] for _ in range(count)]
