"""CPU: the C-ABI library loads, exports every function include/tq_c_api.h
declares, and rejects bad arguments on the host before any GPU call."""
import ctypes
import os
import re

import pytest

from gemma4metal_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NULL = ctypes.c_void_p(0)
FAKE = ctypes.c_void_p(0x10000)  # aligned, never dereferenced: validation fails first


def declared_functions():
    names = set()
    for hdr in os.listdir(os.path.join(ROOT, "include")):
        if not hdr.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", hdr)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tq_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared_functions()
    assert "tq_sdpa_int4" in names and "tq_kv_append_int4" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_error_string():
    lib = _lib.load()
    assert lib.tq_version() == 100
    assert isinstance(lib.tq_last_error(), bytes)


def sdpa(**over):
    a = dict(q=FAKE, q_dtype=_lib.TQ_BF16, kq=FAKE, ks=FAKE, kb=FAKE, vq=FAKE, vs=FAKE, vb=FAKE,
             sb=_lib.TQ_F16, out=FAKE, Hq=32, Hkv=16, D=256, n=128, cap=128, gqa=2, scale=1.0,
             W=0, ws=NULL, wsb=0)
    a.update(over)
    lib = _lib.load()
    st = lib.tq_sdpa_int4(a["q"], a["q_dtype"], a["kq"], a["ks"], a["kb"], a["vq"], a["vs"],
                          a["vb"], a["sb"], a["out"], a["Hq"], a["Hkv"], a["D"], a["n"], a["cap"],
                          a["gqa"], a["scale"], a["W"], a["ws"], a["wsb"], NULL)
    return st, lib.tq_last_error().decode()


@pytest.mark.parametrize("over,status,needle", [
    (dict(D=100), 2, "head_dim"),
    (dict(Hq=30), 1, "num_heads"),
    (dict(n=200), 1, "kv_len"),
    (dict(W=-1), 1, "sliding_window"),
    (dict(q=NULL), 1, "null"),
    (dict(q_dtype=7), 1, "q_dtype"),
    (dict(sb=_lib.TQ_BF16), 1, "sb_dtype"),
    (dict(kq=ctypes.c_void_p(0x10004)), 1, "aligned"),
    (dict(scale=float("inf")), 1, "scale"),
    (dict(n=4096, cap=4096), 4, "workspace"),
    (dict(n=4096, cap=4096, ws=ctypes.c_void_p(0x10008), wsb=1 << 30), 1, "workspace must be 16-byte"),
])
def test_sdpa_rejects_bad_arguments_on_host(over, status, needle):
    st, msg = sdpa(**over)
    assert st == status, msg
    assert needle in msg.lower()


def test_quantize_rejects_bad_arguments_on_host():
    lib = _lib.load()
    st = lib.tq_quantize_int4(FAKE, _lib.TQ_F32, 4, 256, 32, 4, 0, FAKE, FAKE, FAKE, _lib.TQ_F16, NULL)
    assert st == 1 and "group_size" in lib.tq_last_error().decode()
    st = lib.tq_quantize_int4(FAKE, _lib.TQ_F32, 4, 100, 64, 4, 0, FAKE, FAKE, FAKE, _lib.TQ_F16, NULL)
    assert st == 1 and "dim" in lib.tq_last_error().decode()
    st = lib.tq_quantize_int4(FAKE, _lib.TQ_F32, 0, 256, 64, 4, 0, NULL, NULL, NULL, _lib.TQ_F16, NULL)
    assert st == 0  # zero rows is a no-op
    st = lib.tq_kv_append_int4(FAKE, FAKE, _lib.TQ_F32, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                               _lib.TQ_F16, 2, 16, 256, 64, NULL, 1, 0, NULL)
    assert st == 1 and "null" in lib.tq_last_error().decode().lower()


def test_workspace_size_bounds_every_length():
    lib = _lib.load()
    prev = 0
    for L in (1, 64, 786, 1024, 4000, 4100, 32768, 262144):
        ws = lib.tq_sdpa_int4_workspace_size(1, 32, 16, 256, L)
        assert ws >= prev
        prev = ws
    assert lib.tq_sdpa_int4_workspace_size(0, 32, 16, 256, 10) == 0
