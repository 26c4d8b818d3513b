"""ctypes bindings for the CPU oracle: oracle/liboracle.so (the C restatement) and
oracle/_ref/libaccel_ref.so (the reference's own sources, compiled; present only where
the reference tree was available at build time).

Test infrastructure only. Product code never imports this module.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libaccel_ref.so"

F32P = C.POINTER(C.c_float)
I32P = C.POINTER(C.c_int32)
I64P = C.POINTER(C.c_int64)
I8P = C.POINTER(C.c_int8)
U32P = C.POINTER(C.c_uint32)
i64 = C.c_int64


class QuantPlane(C.Structure):
    """OrcQuantPlane (oracle/oracle.h) == RefPlane (oracle/ref_shim.cc)."""

    _fields_ = [
        ("q", I8P),
        ("scale", F32P),
        ("zero", I8P),
        ("rank", C.c_int32),
        ("shape", C.c_int64 * 8),
        ("axis", C.c_int64),
        ("offset", C.c_int64),
    ]


def fptr(a):
    return None if a is None else a.ctypes.data_as(F32P)


def make_plane(q, scale, zero, shape, axis, offset=0):
    """Returns (plane, keepalive). q int8, scale f32, zero int8 or None."""
    plane = QuantPlane()
    plane.q = q.ctypes.data_as(I8P)
    plane.scale = scale.ctypes.data_as(F32P)
    plane.zero = zero.ctypes.data_as(I8P) if zero is not None else None
    plane.rank = len(shape)
    for i, d in enumerate(shape):
        plane.shape[i] = int(d)
    plane.axis = int(axis)
    plane.offset = int(offset)
    return plane, (q, scale, zero)


class _Lib:
    """Shared signatures: the oracle's orc_* and the shim's ref_* take the same arguments."""

    def __init__(self, path: Path, prefix: str):
        self.path = path
        self.prefix = prefix
        self.lib = C.CDLL(str(path))
        p = prefix
        L = self.lib
        getattr(L, f"{p}_reference_matmul").argtypes = [F32P, F32P, F32P, i64, i64, i64]
        mq = getattr(L, f"{p}_matmul_quantized")
        mq.argtypes = [F32P, C.POINTER(QuantPlane), F32P, C.POINTER(QuantPlane), F32P, i64, i64, i64]
        mq.restype = C.c_int
        ep = getattr(L, f"{p}_gemm_epilogue")
        ep.argtypes = [F32P, i64, i64, C.c_float, F32P, C.c_int32, I64P, C.c_float, C.c_int32]
        ep.restype = None if p == "orc" else C.c_int
        getattr(L, f"{p}_rmsnorm").argtypes = [F32P, F32P, F32P, i64, i64, C.c_float, i64]
        em = getattr(L, f"{p}_embed")
        em.argtypes = [I32P, i64, F32P, F32P, i64, i64, i64]
        em.restype = C.c_int
        getattr(L, f"{p}_rope").argtypes = [F32P, F32P, F32P, i64, i64, i64, i64]
        getattr(L, f"{p}_append_cache").argtypes = [F32P, F32P, i64, i64, i64, i64]
        getattr(L, f"{p}_attention").argtypes = [F32P, F32P, F32P, F32P, F32P, i64, i64, i64, i64, i64]
        getattr(L, f"{p}_silu_mul").argtypes = [F32P, F32P, i64]
        getattr(L, f"{p}_add").argtypes = [F32P, F32P, i64]
        getattr(L, f"{p}_sample_token").argtypes = [F32P, I32P, i64, i64, C.c_float, U32P, C.c_int32]

    def _f(self, name):
        return getattr(self.lib, f"{self.prefix}_{name}")

    # ---- numpy-level wrappers -------------------------------------------------
    def reference_matmul(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        m, k = a.shape
        n = b.shape[1]
        c = np.full((m, n), 7.0, np.float32)
        self._f("reference_matmul")(fptr(a), fptr(b), fptr(c), m, k, n)
        return c

    def matmul_quantized(self, a, aplane, b, bplane, m, k, n):
        c = np.full((m, n), 3.0, np.float32)
        rc = self._f("matmul_quantized")(
            fptr(a), C.byref(aplane) if aplane is not None else None,
            fptr(b), C.byref(bplane) if bplane is not None else None, fptr(c), m, k, n)
        if rc != 0:
            raise ValueError(f"{self.prefix}_matmul_quantized failed")
        return c

    def gemm_epilogue(self, c, alpha, bias, bias_shape, beta, act):
        c = np.ascontiguousarray(c, np.float32).copy()
        m, n = c.shape
        shape = (C.c_int64 * 8)(*([int(d) for d in bias_shape] + [0] * (8 - len(bias_shape))))
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        rc = self._f("gemm_epilogue")(fptr(c), m, n, alpha, fptr(b), len(bias_shape), shape, beta, act)
        if rc not in (None, 0):
            raise ValueError("gemm_epilogue failed")
        return c

    def rmsnorm(self, x, w, rows, dim, eps, row_offset=0):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        y = np.full((rows, dim), 42.0, np.float32)
        self._f("rmsnorm")(fptr(x), fptr(w), fptr(y), rows, dim, eps, row_offset)
        return y

    def embed(self, ids, id_offset, table, seq):
        ids = np.ascontiguousarray(ids, np.int32)
        table = np.ascontiguousarray(table, np.float32)
        vocab, hidden = table.shape
        out = np.zeros((seq, hidden), np.float32)
        rc = self._f("embed")(ids.ctypes.data_as(I32P), id_offset, fptr(table), fptr(out), seq, hidden, vocab)
        return rc, out

    def rope(self, states, cos, sin, seq, heads, head_dim, position):
        s = np.ascontiguousarray(states, np.float32).copy()
        self._f("rope")(fptr(s), fptr(np.ascontiguousarray(cos, np.float32)),
                        fptr(np.ascontiguousarray(sin, np.float32)), seq, heads, head_dim, position)
        return s

    def append_cache(self, src, cache, seq, position, heads, head_dim):
        cache = np.ascontiguousarray(cache, np.float32).copy()
        self._f("append_cache")(fptr(np.ascontiguousarray(src, np.float32)), fptr(cache), seq, position, heads,
                                head_dim)
        return cache

    def attention(self, q, k, v, seq, position, heads, kv_heads, head_dim):
        out = np.zeros((seq, heads, head_dim), np.float32)
        scores = np.zeros(position + seq, np.float32)
        self._f("attention")(fptr(np.ascontiguousarray(q, np.float32)), fptr(np.ascontiguousarray(k, np.float32)),
                             fptr(np.ascontiguousarray(v, np.float32)), fptr(scores), fptr(out), seq, position,
                             heads, kv_heads, head_dim)
        return out

    def silu_mul(self, gate, up):
        g = np.ascontiguousarray(gate, np.float32).copy()
        self._f("silu_mul")(fptr(g), fptr(np.ascontiguousarray(up, np.float32)), g.size)
        return g

    def add(self, dest, extra):
        d = np.ascontiguousarray(dest, np.float32).copy()
        self._f("add")(fptr(d), fptr(np.ascontiguousarray(extra, np.float32)), d.size)
        return d

    def sample_token(self, logits, temperature, rng, top_k, index=0):
        logits = np.ascontiguousarray(logits, np.float32)
        chosen = np.full(index + 1, -1, np.int32)
        state = C.c_uint32(rng)
        self._f("sample_token")(fptr(logits), chosen.ctypes.data_as(I32P), index, logits.size, temperature,
                                C.byref(state), top_k)
        return int(chosen[index]), int(state.value)


class Oracle(_Lib):
    def __init__(self):
        super().__init__(ORACLE_SO, "orc")
        L = self.lib
        L.orc_dequant_at.argtypes = [C.POINTER(QuantPlane), i64]
        L.orc_dequant_at.restype = C.c_float
        L.orc_rope_tables.argtypes = [C.c_int32, C.c_int32, C.c_float, F32P, F32P]
        L.orc_llama_create.argtypes = [C.POINTER(LlamaConfig)]
        L.orc_llama_create.restype = C.c_void_p
        L.orc_llama_destroy.argtypes = [C.c_void_p]
        L.orc_llama_weight.argtypes = [C.c_void_p, C.c_int32, C.c_int32, F32P, i64, i64]
        L.orc_llama_generate.argtypes = [C.c_void_p, I32P, C.c_int32, C.c_int32, C.c_int32, C.c_float, C.c_uint32,
                                         C.c_int32, I32P, I32P]
        L.orc_llama_forward_ids.argtypes = [C.c_void_p, I32P, C.c_int32, C.c_int32]
        L.orc_llama_logits.argtypes = [C.c_void_p, F32P, C.c_int32]

    def rope_tables(self, context, head_dim, theta):
        cos = np.zeros((context, head_dim), np.float32)
        sin = np.zeros((context, head_dim), np.float32)
        self.lib.orc_rope_tables(context, head_dim, theta, fptr(cos), fptr(sin))
        return cos, sin


class Reference(_Lib):
    def __init__(self):
        super().__init__(REF_SO, "ref")
        L = self.lib
        L.ref_device_matmul.argtypes = [F32P, F32P, F32P, i64, i64, i64]
        L.ref_device_matmul.restype = C.c_int
        L.accel_llama_create.argtypes = [C.POINTER(LlamaConfig)]
        L.accel_llama_create.restype = C.c_void_p
        L.accel_llama_destroy.argtypes = [C.c_void_p]
        L.accel_llama_weight.argtypes = [C.c_void_p, C.c_int32, C.c_int32, F32P, i64, i64]
        L.accel_llama_generate.argtypes = [C.c_void_p, I32P, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                           C.c_uint32, C.c_int32, I32P, I32P]
        L.accel_llama_forward_ids.argtypes = [C.c_void_p, I32P, C.c_int32, C.c_int32]
        L.accel_llama_logit_max_abs.argtypes = [C.c_void_p, F32P, C.c_int32, F32P]
        L.accel_llama_last_error.restype = C.c_char_p

    def device_matmul(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        m, k = a.shape
        n = b.shape[1]
        c = np.full((m, n), 5.0, np.float32)
        assert self.lib.ref_device_matmul(fptr(a), fptr(b), fptr(c), m, k, n) == 0
        return c


class LlamaConfig(C.Structure):
    """AccelLlamaConfig (include/accel/sim_api.h:44-54) == OrcLlamaConfig."""

    _fields_ = [(name, C.c_int32) for name in ("vocab", "hidden", "layers", "heads", "kv_heads", "intermediate",
                                               "context")] + [("eps", C.c_float), ("rope_theta", C.c_float)]


_oracle = None
_reference = None


def oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def reference():
    """The compiled reference, or None when it was not built (no reference tree)."""
    global _reference
    if _reference is None and REF_SO.exists():
        _reference = Reference()
    return _reference


# ---- the reference tests' own input generators --------------------------------

def fill_lcg(count, seed):
    """FillLcg, tests/test_runtime.cc:225-232. Returns (values, next_seed)."""
    out = np.empty(count, np.float32)
    s = seed & 0xFFFFFFFF
    for i in range(count):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(float((s % 10007) - 5003) * 0.1)
    return out, s


def lcg_int8(count, seed):
    """q fill of tests/test_runtime.cc:335-338: (seed % 251) - 125."""
    out = np.empty(count, np.int8)
    s = seed & 0xFFFFFFFF
    for i in range(count):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (s % 251) - 125
    return out, s


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def from_bits(u):
    return np.asarray(u, np.uint32).view(np.float32)
