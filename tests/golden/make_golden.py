"""Writes the committed fixtures of tests/golden/ (inputs and expected
outputs, .npz without pickles) from the oracle.  The reference has no golden
vectors of its own for this path (its test draws unseeded random inputs,
tests/test_sdpa_int4.cpp:20-22) and its implementation cannot run here
(Metal + MLX), so these are this build's regression anchors: the CPU tests
check that the oracle still reproduces them bit for bit, the GPU tests check
the HIP path against them.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from oracle import polar as PQ  # noqa: E402

f32 = np.float32


def quant_inputs():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((24, 128)).astype(f32)
    x[0, :64] = 0.75                      # constant group
    x[1, :64] = np.linspace(-1, 1, 64)    # contains exact zero crossing
    x[2, :64] = np.arange(64) / 4.0       # exact quarter steps (rint ties)
    x[3, :64] = -np.arange(64) / 8.0
    x[4, 64:] = 1e-9 * rng.standard_normal(64)  # below the eps clamp
    return x


def make():
    out = {}
    x = quant_inputs()
    for sb in ("f32", "f16"):
        wq, s, b = O.quantize_int4(x, sb)
        out[f"quant_{sb}"] = dict(x=x, wq=wq, scales=s, biases=b)
    wq, s, b = O.quantize_int4(x, "f16", mode="minmax")
    out["quant_minmax_f16"] = dict(x=x, wq=wq, scales=s, biases=b)

    # tiny decode: Hq 2, Hkv 1, D 128, L 33, RMS-normed q/k, scale 1
    rng = np.random.default_rng(20260)
    q = O.rms_norm(rng.standard_normal((2, 128)).astype(f32))
    k = O.rms_norm(rng.standard_normal((1, 33, 128)).astype(f32))
    v = rng.standard_normal((1, 33, 128)).astype(f32)
    kq, ks, kb = O.quantize_int4(k, "f16")
    vq, vs, vb = O.quantize_int4(v, "f16")
    o = O.sdpa_int4(q, kq, ks, kb, vq, vs, vb, 2, 1.0, 0)
    out["sdpa_tiny"] = dict(q=q, kq=kq, ks=ks, kb=kb, vq=vq, vs=vs, vb=vb, out=o)

    # reference polar layouts, D 64 with a preconditioner
    rng = np.random.default_rng(31)
    xv = rng.standard_normal((40, 64)).astype(f32)
    P = np.linalg.qr(rng.standard_normal((64, 64)))[0].astype(f32)
    cbs = [np.sort(rng.uniform(0, 2 * np.pi, 16)).astype(f32)] + \
          [np.sort(rng.uniform(0, np.pi / 2, 4)).astype(f32) for _ in range(3)]
    i1, i2, i3, i4, rad = PQ.polar_quantize(xv, P, cbs)
    p1, p2, p3, p4 = PQ.pack_ref([i1, i2, i3, i4])
    out["polar16"] = dict(x=xv, P=P, cb1=cbs[0], cb2=cbs[1], cb3=cbs[2], cb4=cbs[3],
                          i1=i1, i2=i2, i3=i3, i4=i4, radii=rad, p1=p1, p2=p2, p3=p3, p4=p4)

    # polar7 layout: 7 levels + QJL, and scores of 2 query heads
    rng = np.random.default_rng(47)
    xk = rng.standard_normal((2, 30, 128)).astype(f32)
    P = np.linalg.qr(rng.standard_normal((128, 128)))[0].astype(f32)
    S = rng.standard_normal((128, 128)).astype(f32)
    ang, nrm, qj = PQ.polar7_encode(xk.reshape(-1, 128), P, S)
    qh = rng.standard_normal((4, 128)).astype(f32)
    qp = (qh.astype(np.float64) @ P.astype(np.float64).T).astype(f32)
    qs = PQ.qjl_query(qp, S).astype(f32)
    sc = PQ.polar7_scores(qp, qs, ang.reshape(2, 30, 12), nrm.reshape(2, 30, 2),
                          qj.reshape(2, 30, 4), 2)
    out["polar7"] = dict(x=xk, P=P, S=S, angles=ang, norms=nrm, qjl=qj, q=qh, q_rot=qp,
                         q_sketch=qs, scores=sc)
    return out


def main():
    for name, arrays in make().items():
        np.savez(os.path.join(HERE, name + ".npz"), **arrays)
        print("wrote", name)


if __name__ == "__main__":
    main()
