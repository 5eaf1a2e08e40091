"""The no-allocation decode entry point tq_sdpa_int4_noalloc (library-owned
static scratch), called through the C ABI, against tq_sdpa_int4 with a
caller workspace: bit-identical outputs on consecutive calls, the second one
smaller, and both within the parity bar of the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from gemma4metal_amd import _lib
from oracle import oracle as O
from tests.gpu_util import assert_close, dev, host, queries


def _call_both(tq, qd, cache, Hq, Hkv, D, n, W, sb):
    out_ws = torch.full((Hq, D), float("nan"), dtype=torch.float32, device="cuda")
    out_na = torch.full((Hq, D), float("nan"), dtype=torch.float32, device="cuda")
    cap = cache[0].shape[1]
    qdt = tq._DT[qd.dtype]
    sbt = tq._DT[cache[1].dtype]
    nbytes = _lib.load().tq_sdpa_int4_workspace_size(1, Hq, Hkv, D, n)
    ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = [t.data_ptr() for t in cache]
    _lib.call("tq_sdpa_int4", qd.data_ptr(), qdt, ptrs[0], ptrs[1], ptrs[2], ptrs[3], ptrs[4],
              ptrs[5], sbt, out_ws.data_ptr(), Hq, Hkv, D, n, cap, Hq // Hkv, 1.0, W,
              ws.data_ptr(), ws.numel(), stream)
    _lib.call("tq_sdpa_int4_noalloc", qd.data_ptr(), qdt, ptrs[0], ptrs[1], ptrs[2], ptrs[3],
              ptrs[4], ptrs[5], sbt, out_na.data_ptr(), Hq, Hkv, D, n, cap, Hq // Hkv, 1.0, W,
              stream)
    torch.cuda.synchronize()
    return host(out_ws), host(out_na)


@pytest.mark.gpu
@pytest.mark.parametrize("sb", ["f16", "f32"])
def test_noalloc_matches_workspace_entry_point(gpu, sb):
    rng = np.random.default_rng(2027)
    # two calls in a row, the second with a smaller input
    for Hq, Hkv, D, L, W in ((32, 16, 256, 20000, 0), (32, 16, 256, 3000, 1024)):
        qd, qv = queries(rng, (Hq, D), "bf16")
        k = O.rms_norm(rng.standard_normal((Hkv, L, D)).astype(np.float32))
        v = rng.standard_normal((Hkv, L, D)).astype(np.float32)
        c = O.quantize_int4(k, sb) + O.quantize_int4(v, sb)
        cache = [dev(a) for a in c]
        a, b = _call_both(gpu, qd, cache, Hq, Hkv, D, L, W, sb)
        assert np.array_equal(a, b), f"L={L}: noalloc differs from the workspace call"
        assert_close(b, O.sdpa_int4(qv, *c, Hq // Hkv, 1.0, W), f"noalloc L={L}")


@pytest.mark.gpu
def test_noalloc_global_layer_and_tiny(gpu):
    """The D 512 heads-as-columns path (with its separate merge kernel) and a
    single-split call share the same scratch one after the other."""
    rng = np.random.default_rng(2028)
    for Hq, Hkv, D, L in ((32, 4, 512, 9000), (2, 1, 128, 33)):
        qd, qv = queries(rng, (Hq, D), "bf16")
        k = O.rms_norm(rng.standard_normal((Hkv, L, D)).astype(np.float32))
        v = rng.standard_normal((Hkv, L, D)).astype(np.float32)
        c = O.quantize_int4(k, "f16") + O.quantize_int4(v, "f16")
        a, b = _call_both(gpu, qd, [dev(x) for x in c], Hq, Hkv, D, L, 0, "f16")
        assert np.array_equal(a, b)
        assert_close(b, O.sdpa_int4(qv, *c, Hq // Hkv), f"noalloc D{D} L{L}")


def test_noalloc_rejects_shapes_beyond_the_scratch(tq_env):
    """A shape whose split-K workspace exceeds the static 8 MiB is refused
    on the host, before any device call (so this runs without a GPU)."""
    tq_env("TQ_SDPA_CHUNK", "128")  # 256 splits: 32 heads x 256 x 1 KiB of partials
    lib = _lib.load()
    assert lib.tq_sdpa_int4_workspace_size(1, 32, 16, 256, 32768) > 8 << 20
    # Fake pointers, and a k_quant that is not 16-byte aligned: whichever
    # host check runs first refuses the call, so no kernel ever sees them.
    f = ctypes.c_void_p(0x10000)
    kq = ctypes.c_void_p(0x10008)
    st = lib.tq_sdpa_int4_noalloc(f, _lib.TQ_BF16, kq, f, f, f, f, f, _lib.TQ_F16, f, 32,
                                  16, 256, 32768, 32768, 2, 1.0, 0, None)
    assert st == 2  # TQ_ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error()
