"""ctypes binding of include/accel_hip.h (libaccel_hip.so, built in-tree).

There is no fallback: if the library is missing or cannot be loaded, `lib()` raises.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libaccel_hip.so"

ACCEL_HIP_OK = 0
STATUS_NAMES = {1: "invalid_argument", 2: "overflow_error", 3: "logic_error", 4: "bad_alloc", 5: "runtime_error"}
ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2

F32P = C.POINTER(C.c_float)
I8P = C.POINTER(C.c_int8)
I32P = C.POINTER(C.c_int32)
I64P = C.POINTER(C.c_int64)
U32P = C.POINTER(C.c_uint32)
i64 = C.c_int64


class Buffer(C.Structure):
    """AccelHipBuffer == accel::DeviceBuffer."""

    _fields_ = [("data", C.c_void_p), ("bytes", C.c_size_t), ("id", C.c_uint64)]


class QuantPlane(C.Structure):
    """AccelHipQuantPlane == accel::QuantPlane with the shape inline."""

    _fields_ = [("q", C.c_void_p), ("scale", C.c_void_p), ("zero", C.c_void_p), ("rank", C.c_int32),
                ("shape", C.c_int64 * 8), ("axis", C.c_int64), ("offset", C.c_int64)]


class Stats(C.Structure):
    _fields_ = [(n, C.c_int64) for n in ("matmul_ops", "gemm_ops", "kernel_matmuls", "relu_epilogues",
                                         "gelu_epilogues", "add_epilogues", "device_transposes", "bytes_to_device",
                                         "bytes_to_host")]


class Epilogue(C.Structure):
    _fields_ = [("alpha", C.c_float), ("beta", C.c_float), ("bias", C.c_void_p), ("bias_rank", C.c_int32),
                ("bias_shape", C.c_int64 * 2), ("activation", C.c_int32), ("residual", C.c_void_p),
                ("rms_weight", C.c_void_p), ("rms_eps", C.c_float), ("rms_out", C.c_void_p)]


WORK_FN = C.CFUNCTYPE(C.c_int, C.c_void_p)

# name -> (restype, argtypes)
SIGNATURES = {
    "accel_hip_last_error": (C.c_char_p, []),
    "accel_hip_init": (C.c_int, []),
    "accel_hip_synchronize": (C.c_int, []),
    "accel_hip_device_arch": (C.c_char_p, []),
    "accel_hip_set_exact_products": (C.c_int, [C.c_int32]),
    "accel_hip_exact_products": (C.c_int32, []),
    "accel_hip_allocate": (C.c_int, [C.c_size_t, C.POINTER(Buffer)]),
    "accel_hip_free": (C.c_int, [Buffer]),
    "accel_hip_copy_h2d": (C.c_int, [Buffer, C.c_void_p, C.c_size_t]),
    "accel_hip_copy_d2h": (C.c_int, [C.c_void_p, Buffer, C.c_size_t]),
    "accel_hip_peek": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "accel_hip_poke": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "accel_hip_live_allocs": (C.c_int64, []),
    "accel_hip_trim": (C.c_int, []),
    "accel_hip_get_stats": (None, [C.POINTER(Stats)]),
    "accel_hip_reset_stats": (None, []),
    "accel_hip_packed_matmul_calls": (C.c_int64, []),
    "accel_hip_packed_k_trips": (C.c_int64, []),
    "accel_hip_reset_packed_probes": (None, []),
    "accel_hip_matmul": (C.c_int, [Buffer, Buffer, Buffer, i64, i64, i64]),
    "accel_hip_matmul_quantized": (C.c_int, [C.c_void_p, C.POINTER(QuantPlane), C.c_void_p, C.POINTER(QuantPlane),
                                             C.c_void_p, i64, i64, i64]),
    "accel_hip_matmul_fused": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, i64, i64, i64, C.POINTER(Epilogue)]),
    "accel_hip_matmul_quantized_fused": (C.c_int, [C.c_void_p, C.POINTER(QuantPlane), C.c_void_p,
                                                   C.POINTER(QuantPlane), C.c_void_p, i64, i64, i64,
                                                   C.POINTER(Epilogue)]),
    "accel_hip_matmul_quantized_fused_noalloc": (C.c_int, [C.c_void_p, C.POINTER(QuantPlane), C.c_void_p,
                                                           C.POINTER(QuantPlane), C.c_void_p, i64, i64, i64,
                                                           C.POINTER(Epilogue)]),
    "accel_hip_prepare_quantized": (C.c_int, [C.POINTER(QuantPlane), i64, i64, C.c_uint32,
                                              C.POINTER(C.c_uint32)]),
    "accel_hip_transpose": (C.c_int, [Buffer, Buffer, i64, i64]),
    "accel_hip_gemm_epilogue": (C.c_int, [Buffer, i64, i64, C.c_float, C.POINTER(Buffer), C.c_int32, I64P,
                                          C.c_float, C.c_int32]),
    "accel_hip_embedding": (C.c_int, [Buffer, i64, Buffer, Buffer, i64, i64, i64]),
    "accel_hip_embedding_q8": (C.c_int, [Buffer, i64, C.c_void_p, C.c_void_p, Buffer, i64, i64, i64]),
    "accel_hip_rms_norm": (C.c_int, [Buffer, Buffer, Buffer, i64, i64, C.c_float, i64]),
    "accel_hip_rope": (C.c_int, [Buffer, Buffer, Buffer, i64, i64, i64, i64]),
    "accel_hip_append_cache": (C.c_int, [Buffer, Buffer, i64, i64, i64, i64]),
    "accel_hip_attention": (C.c_int, [Buffer, Buffer, Buffer, Buffer, Buffer, i64, i64, i64, i64, i64]),
    "accel_hip_silu_mul": (C.c_int, [Buffer, Buffer, i64]),
    "accel_hip_residual_add": (C.c_int, [Buffer, Buffer, i64]),
    "accel_hip_sample_token": (C.c_int, [Buffer, Buffer, i64, i64, C.c_float, U32P, C.c_int32]),
    "accel_hip_time_ms": (C.c_double, [WORK_FN, C.c_void_p, C.c_int32]),
    "accel_hip_event_record": (C.c_int, [C.c_int32]),
    "accel_hip_event_elapsed_ms": (C.c_double, [C.c_int32, C.c_int32]),
    "accel_hip_capture_begin": (C.c_int, []),
    "accel_hip_capture_end": (C.c_int, [C.POINTER(C.c_void_p)]),
    "accel_hip_graph_launch": (C.c_int, [C.c_void_p, C.c_int32]),
    "accel_hip_graph_destroy": (C.c_int, [C.c_void_p]),
}

_lib = None


class HipError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.kind = STATUS_NAMES.get(code, str(code))
        self.message = message


class LlamaConfig(C.Structure):
    """AccelLlamaConfig (include/accel_llama.h)."""

    _fields_ = [("vocab", C.c_int32), ("hidden", C.c_int32), ("layers", C.c_int32), ("heads", C.c_int32),
                ("kv_heads", C.c_int32), ("intermediate", C.c_int32), ("context", C.c_int32), ("eps", C.c_float),
                ("rope_theta", C.c_float)]


# include/accel_llama.h
LLAMA_SIGNATURES = {
    "accel_llama_create": (C.c_void_p, [C.POINTER(LlamaConfig)]),
    "accel_llama_destroy": (None, [C.c_void_p]),
    "accel_llama_weight": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, F32P, i64, i64]),
    "accel_llama_weight_q8": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, I8P, F32P, i64, i64]),
    "accel_llama_generate": (C.c_int, [C.c_void_p, I32P, C.c_int32, C.c_int32, C.c_int32, C.c_float, C.c_uint32,
                                       C.c_int32, I32P, I32P]),
    "accel_llama_tokenizer": (C.c_int, [C.c_void_p, C.c_char_p]),
    "accel_llama_encode": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int32, I32P, C.c_int32, I32P]),
    "accel_llama_decode": (C.c_int, [C.c_void_p, I32P, C.c_int32, C.c_int32, C.c_char_p, C.c_int32, I32P]),
    "accel_llama_complete": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.c_int32, C.c_float, C.c_uint32,
                                       C.c_int32, C.c_char_p, C.c_int32, I32P, I32P, C.c_int32, I32P, I32P]),
    "accel_llama_complete_stream": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                              C.c_uint32, C.c_int32, C.c_char_p, C.c_int32, I32P, I32P, C.c_int32,
                                              I32P, I32P, C.c_void_p, C.c_void_p]),
    "accel_llama_forward_ids": (C.c_int, [C.c_void_p, I32P, C.c_int32, C.c_int32]),
    "accel_llama_logit_max_abs": (C.c_int, [C.c_void_p, F32P, C.c_int32, F32P]),
    "accel_llama_logits": (C.c_int, [C.c_void_p, F32P, C.c_int32]),
    "accel_llama_set_fused_inputs": (C.c_int, [C.c_void_p, C.c_int32]),
    "accel_llama_reset": (None, [C.c_void_p]),
    "accel_llama_last_error": (C.c_char_p, []),
}

# include/accel_sim.h
SIM_SIGNATURES = {
    "accel_sim_create": (C.c_void_p, []),
    "accel_sim_destroy": (None, [C.c_void_p]),
    "accel_sim_upload": (C.c_void_p, [C.c_void_p, F32P, i64]),
    "accel_sim_release": (None, [C.c_void_p, C.c_void_p]),
    "accel_sim_matmul": (C.c_int, [C.c_void_p, F32P, i64, i64, C.c_void_p, i64, F32P]),
    "accel_sim_reset_stats": (None, []),
    "accel_sim_matmuls": (C.c_int64, []),
    "accel_sim_bytes_to_device": (C.c_int64, []),
    "accel_sim_bytes_to_host": (C.c_int64, []),
    "accel_sim_last_error": (C.c_char_p, []),
}


# AccelLlamaTokenFn: void (*)(int32_t token_id, void* user)
TOKEN_FN = C.CFUNCTYPE(None, C.c_int32, C.c_void_p)


def lib() -> C.CDLL:
    """Loads libaccel_hip.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m accelep_amd.build`")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in {**SIGNATURES, **LLAMA_SIGNATURES, **SIM_SIGNATURES}.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int):
    if rc != ACCEL_HIP_OK:
        raise HipError(rc, lib().accel_hip_last_error().decode())
