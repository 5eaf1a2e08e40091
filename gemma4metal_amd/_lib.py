"""ctypes binding of ``libturboquant_hip.so`` (the C ABI in include/tq_c_api.h).

The library must be built (``python -m gemma4metal_amd._build`` or
``__graft_entry__.build()``); importing never falls back to anything else --
a missing library raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libturboquant_hip.so")

TQ_F32, TQ_F16, TQ_BF16 = 0, 1, 2
TQ_QUANT_MLX, TQ_QUANT_MINMAX = 0, 1

STATUS = {0: "TQ_OK", 1: "TQ_ERR_INVALID", 2: "TQ_ERR_UNSUPPORTED", 3: "TQ_ERR_HIP",
          4: "TQ_ERR_WORKSPACE"}

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float
SZ = ctypes.c_size_t

# name -> (restype, argtypes); every symbol declared in include/tq_c_api.h
SIGNATURES = {
    "tq_version": (I, []),
    "tq_last_error": (ctypes.c_char_p, []),
    "tq_device_count": (I, [P]),
    "tq_set_device": (I, [I]),
    "tq_malloc": (I, [P, SZ]),
    "tq_free": (I, [P]),
    "tq_memcpy_h2d": (I, [P, P, SZ]),
    "tq_memcpy_d2h": (I, [P, P, SZ]),
    "tq_memset": (I, [P, I, SZ]),
    "tq_sync": (I, []),
    "tq_stream_read": (I, [P, SZ, P, I, P]),
    "tq_stream_read_tiles": (I, [P, SZ, P, I, I, I, I, I, P]),
    "tq_sdpa_int4_workspace_size": (SZ, [I, I, I, I, I]),
    "tq_sdpa_int4_plan": (I, [I, I, I, I, I, I, I, I, P, P, P, SZ]),
    "tq_sdpa_int4_noalloc": (I, [P, I, P, P, P, P, P, P, I, P, I, I, I, I, I, I, F, I, P]),
    "tq_reload_options": (I, []),
    "tq_sdpa_int4": (I, [P, I, P, P, P, P, P, P, I, P, I, I, I, I, I, I, F, I, P, SZ, P]),
    "tq_sdpa_int4_ragged": (I, [P, I, P, P, P, P, P, P, I, P, I, I, I, I, I, P, P, I, I, F, I,
                                P, SZ, P]),
    "tq_sdpa_int4_prefill": (I, [P, I, P, P, P, P, P, P, I, P, I, I, I, I, I, I, I, F, I, P, SZ,
                                 P]),
    "tq_quantize_int4": (I, [P, I, I64, I, I, I, I, P, P, P, I, P]),
    "tq_kv_append_int4": (I, [P, P, I, P, P, P, P, P, P, I, I, I, I, I, P, I, I, P]),
    "tq_kv_append_int4_ring": (I, [P, P, I, P, P, P, P, P, P, I, I, I, I, I, P, I, I, P]),
    "tq_dequantize_int4": (I, [P, P, P, I, I64, I, P, P]),
    "tq_polar_quantize": (I, [P, P, P, P, I64, I, I, P, P, P, P, P, P]),
    "tq_polar_quantize_packed": (I, [P, P, P, P, I64, I, I, P, P, P, P, P, P]),
    "tq_polar_dequantize": (I, [P, P, P, P, P, P, P, P, I64, I, I, P, P]),
    "tq_polar_dequantize_packed": (I, [P, P, P, P, P, P, P, P, I64, I, I, P, P]),
    "tq_compressed_score": (I, [P, I, P, P, P, P, P, P, P, I, I, I, I, F, P, P]),
    "tq_compressed_score_packed": (I, [P, I, P, P, P, P, P, P, P, I, I, I, I, F, P, P]),
    "tq_compressed_sdpa_workspace_size": (SZ, [I, I, I, I]),
    "tq_compressed_sdpa": (I, [P, I, P, P, P, P, P, P, P, P, I, I, I, I, F, P, P, SZ, P]),
    "tq_polar_rotate": (I, [P, P, I64, I, P, P]),
    "tq_qjl_query": (I, [P, P, I, P, P]),
    "tq_polar7_encode": (I, [P, P, P, P, P, I64, P, P, P, P]),
    "tq_polar7_kv_append": (I, [P, P, P, P, P, P, P, P, I, I, I, P, I, P]),
    "tq_polar7_prepare_query": (I, [P, P, P, P, I, P, P, P, P]),
    "tq_polar7_sketch_precondition": (I, [P, P, P, P]),
    "tq_polar7_prepare_query_sp": (I, [P, P, P, P, I, P, P, P, P]),
    "tq_polar7_score": (I, [P, P, P, P, P, I, I, I, I, F, P, P]),
    "tq_polar7_score_q": (I, [P, P, P, P, P, P, P, I, I, I, I, F, P, P]),
    "tq_polar7_sdpa_workspace_size": (SZ, [I, I, I]),
    "tq_polar7_sdpa_int4v": (I, [P, P, P, P, P, P, P, P, I, P, I, I, I, I, F, I, P, SZ, P]),
    "tq_polar7_sdpa_int4v_q": (I, [P, P, P, P, P, P, P, P, P, P, I, P, I, I, I, I, F, I, P, SZ, P]),
}


class TQError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero tq_status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} -> {STATUS.get(status, status)}: {msg}")
        self.status = status


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m gemma4metal_amd._build` "
                "(or __graft_entry__.build()) first -- there is no fallback path")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


_fns: dict = {}


def call(name: str, *args) -> int:
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    st = fn(*args)
    if st != 0:
        raise TQError(name, st, load().tq_last_error().decode())
    return st


def last_error() -> str:
    return load().tq_last_error().decode()
