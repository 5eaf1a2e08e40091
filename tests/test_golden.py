"""The committed fixtures of tests/golden/ (written by make_golden.py): the
oracle reproduces them bit for bit (CPU), and the HIP path matches them
(GPU: bit-exact for quantize/encode, the parity tolerances otherwise)."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from oracle import polar as PQ

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    if a.dtype.kind == "f":
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    else:
        assert np.array_equal(a, b)


# ---------------------------------------------------------------- oracle ----

@pytest.mark.parametrize("name,sb,mode", [("quant_f32", "f32", "mlx"), ("quant_f16", "f16", "mlx"),
                                          ("quant_minmax_f16", "f16", "minmax")])
def test_oracle_reproduces_quant_fixture(name, sb, mode):
    g = load(name)
    for got, want in zip(O.quantize_int4(g["x"], sb, mode=mode), (g["wq"], g["scales"], g["biases"])):
        same(got, want)


def test_oracle_reproduces_sdpa_fixture():
    g = load("sdpa_tiny")
    o = O.sdpa_int4(g["q"], g["kq"], g["ks"], g["kb"], g["vq"], g["vs"], g["vb"], 2, 1.0, 0)
    assert np.max(np.abs(o - g["out"])) < 1e-12


def test_oracle_reproduces_polar_fixtures():
    g = load("polar16")
    cbs = [g["cb1"], g["cb2"], g["cb3"], g["cb4"]]
    for got, want in zip(PQ.polar_quantize(g["x"], g["P"], cbs), (g["i1"], g["i2"], g["i3"], g["i4"], g["radii"])):
        same(got, want)
    g = load("polar7")
    for got, want in zip(PQ.polar7_encode(g["x"].reshape(-1, 128), g["P"], g["S"]),
                         (g["angles"], g["norms"], g["qjl"])):
        same(got, want)


# ------------------------------------------------------------------- GPU ----

@pytest.mark.gpu
def test_gpu_matches_quant_fixtures(gpu):
    from tests.gpu_util import dev, host
    import torch
    for name, sdt, mode in (("quant_f32", torch.float32, "mlx"), ("quant_f16", torch.float16, "mlx"),
                            ("quant_minmax_f16", torch.float16, "minmax")):
        g = load(name)
        wq, s, b = gpu.quantize(dev(g["x"]), scale_dtype=sdt, mode=mode)
        same(host(wq), g["wq"])
        same(host(s), g["scales"])
        same(host(b), g["biases"])


@pytest.mark.gpu
def test_gpu_matches_sdpa_fixture(gpu):
    from tests.gpu_util import assert_close, dev, host
    g = load("sdpa_tiny")
    out = gpu.sdpa_int4(dev(g["q"]), *[dev(g[k]) for k in ("kq", "ks", "kb", "vq", "vs", "vb")], 2, 1.0, 0)
    assert_close(host(out), g["out"], "golden tiny decode")


@pytest.mark.gpu
def test_gpu_matches_polar_fixtures(gpu):
    from gemma4metal_amd import polar as pq
    from tests.gpu_util import dev, host
    g = load("polar16")
    cbs = [dev(g[f"cb{i}"]) for i in range(1, 5)]
    got = pq.polar_quantize(dev(g["x"]), dev(g["P"]), *cbs)
    for a, k in zip(got, ("i1", "i2", "i3", "i4", "radii")):
        same(host(a), g[k])
    got = pq.polar_quantize_packed(dev(g["x"]), dev(g["P"]), *cbs)
    for a, k in zip(got, ("p1", "p2", "p3", "p4", "radii")):
        same(host(a).astype(g[k].dtype) if k != "radii" else host(a), g[k])
    g = load("polar7")
    codec = pq.Polar7Codec(dev(g["P"]), dev(g["S"]))
    ang, nrm, qj = (host(t) for t in codec.encode(dev(g["x"].reshape(-1, 128))))
    same(ang, g["angles"])
    n16 = g["norms"].view(np.uint16).astype(np.uint32)
    same(nrm, n16[:, 0] | (n16[:, 1] << 16))
    same(qj, g["qjl"])
    tab = codec.prepare_query(dev(g["q"]))
    d = [t.reshape(2, 30, -1) if t.dim() == 2 else t.reshape(2, 30) for t in codec.encode(dev(g["x"].reshape(-1, 128)))]
    sc = host(codec.score(tab, *d))
    assert np.max(np.abs(sc - g["scores"])) < 1e-3
