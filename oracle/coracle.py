"""ctypes wrapper and build recipe for ``oracle/tq_oracle.c``.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "tq_oracle.c")
LIB = os.path.join(HERE, "libtq_oracle.so")

_lib = None


def build(force: bool = True) -> str:
    """Compile the C restatement with gcc (no fused multiply-add, OpenMP)."""
    if force or not os.path.exists(LIB):
        tmp = LIB + ".tmp"
        subprocess.check_call([
            "gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
            "-fno-fast-math", "-std=c11", SRC, "-o", tmp, "-lm"])
        os.replace(tmp, LIB)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build(force=True)
        L = ctypes.CDLL(LIB)
        P = ctypes.c_void_p
        I = ctypes.c_int
        L.tqo_quantize_int4.argtypes = [P, ctypes.c_int64, I, I, P, P, P]
        L.tqo_quantize_int4.restype = None
        L.tqo_sdpa_int4_f64.argtypes = [P] * 7 + [I] * 6 + [ctypes.c_float, I, P]
        L.tqo_sdpa_int4_f64.restype = None
        L.tqo_sdpa_dequant_f32.argtypes = [P] * 7 + [I] * 6 + [ctypes.c_float, I, P, P, P, I]
        L.tqo_sdpa_dequant_f32.restype = None
        L.tqo_num_threads.argtypes = []
        L.tqo_num_threads.restype = I
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize_int4(x: np.ndarray, mode: int = 0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.size // D
    wq = np.empty(x.shape[:-1] + (D // 8,), np.uint32)
    s = np.empty(x.shape[:-1] + (D // 64,), np.float32)
    b = np.empty_like(s)
    lib().tqo_quantize_int4(_p(x), rows, D, mode, _p(wq), _p(s), _p(b))
    return wq, s, b


def _f32(a):
    return np.ascontiguousarray(np.asarray(a).astype(np.float32))


def sdpa_int4_f64(q, kq, ks, kb, vq, vs, vb, gqa, scale=1.0, window=0, kv_len=None):
    q = _f32(q)
    Hq, D = q.shape
    Hkv, cap = kq.shape[0], kq.shape[1]
    n = cap if kv_len is None else kv_len
    out = np.empty((Hq, D), np.float64)
    args = [np.ascontiguousarray(kq, np.uint32), _f32(ks), _f32(kb),
            np.ascontiguousarray(vq, np.uint32), _f32(vs), _f32(vb)]
    lib().tqo_sdpa_int4_f64(_p(q), *[_p(a) for a in args], Hq, Hkv, D, cap, n, gqa,
                            float(scale), window, _p(out))
    return out


class DequantSdpaBaseline:
    """The CPU baseline: fp32 dequantize + fp32 attention (OpenMP)."""

    def __init__(self, q, kq, ks, kb, vq, vs, vb, gqa, scale=1.0, window=0,
                 kv_len=None, threads=0):
        self.q = _f32(q)
        self.Hq, self.D = self.q.shape
        self.Hkv, self.cap = kq.shape[0], kq.shape[1]
        self.n = self.cap if kv_len is None else kv_len
        self.gqa, self.scale, self.window, self.threads = gqa, float(scale), window, threads
        self.args = [np.ascontiguousarray(kq, np.uint32), _f32(ks), _f32(kb),
                     np.ascontiguousarray(vq, np.uint32), _f32(vs), _f32(vb)]
        lo = max(0, self.n - window) if window > 0 else 0
        L = self.n - lo
        self.kdq = np.empty((self.Hkv, max(L, 1), self.D), np.float32)
        self.vdq = np.empty_like(self.kdq)
        self.out = np.empty((self.Hq, self.D), np.float32)

    def __call__(self):
        lib().tqo_sdpa_dequant_f32(_p(self.q), *[_p(a) for a in self.args], self.Hq,
                                   self.Hkv, self.D, self.cap, self.n, self.gqa,
                                   self.scale, self.window, _p(self.kdq), _p(self.vdq),
                                   _p(self.out), self.threads)
        return self.out


def num_threads() -> int:
    return lib().tqo_num_threads()
