"""Pins the PolarQuant / QJL oracle (oracle/polar.py) with checks that do not
restate its formulas: float64 library values, exact-hit round trips,
invariants, closed forms, bit-position known answers, Monte-Carlo
unbiasedness, and a planted mutant."""
import math

import numpy as np
import pytest

from oracle import polar as PQ

f32 = np.float32


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- atan2 ----

def test_atan2_matches_float64_library():
    r = rng(1)
    y = r.standard_normal(100000).astype(f32) * f32(10) ** r.integers(-3, 4, 100000).astype(f32)
    x = r.standard_normal(100000).astype(f32) * f32(10) ** r.integers(-3, 4, 100000).astype(f32)
    a = PQ.atan2_f32(y, x).astype(np.float64)
    ref = np.arctan2(y.astype(np.float64), x.astype(np.float64))
    assert np.max(np.abs(a - ref)) < 5e-7


@pytest.mark.parametrize("y,x,expect", [
    (0.0, 0.0, 0.0), (-0.0, 0.0, -0.0), (0.0, -0.0, math.pi), (-0.0, -0.0, -math.pi),
    (1.0, 0.0, math.pi / 2), (-1.0, 0.0, -math.pi / 2), (0.0, -1.0, math.pi),
    (-0.0, -1.0, -math.pi), (1.0, 1.0, math.pi / 4), (-1.0, -1.0, -3 * math.pi / 4),
    (3.0, -4.0, math.atan2(3, -4)),
])
def test_atan2_special_cases(y, x, expect):
    a = PQ.atan2_f32(f32(y), f32(x))
    assert abs(float(a) - expect) < 4e-7
    assert np.signbit(a) == np.signbit(f32(expect)) or expect == 0.0 and y >= 0


def test_nearest_first_minimum_wins():
    cb = np.array([0.0, 1.0, 1.0, 2.0], dtype=f32)
    assert PQ.nearest_index(f32(1.0), cb) == 1        # duplicate entries: first
    assert PQ.nearest_index(f32(0.5), cb) == 0        # exact tie 0 vs 1: first
    assert PQ.nearest_index(f32(1.6), cb) == 3


# ------------------------------------------------------- encode / decode ----

def _tree_from_indices(idx_levels, R, cbs):
    """Builds y (float64) whose polar encoding is exactly the given indices."""
    v = np.array([R], dtype=np.float64)
    for lvl in range(len(idx_levels) - 1, -1, -1):
        th = np.asarray(cbs[lvl], dtype=f32).astype(np.float64)[idx_levels[lvl]]
        out = np.empty(2 * v.shape[0])
        out[0::2] = v * np.cos(th)
        out[1::2] = v * np.sin(th)
        v = out
    return v


def test_exact_codebook_hits_round_trip_polar7():
    cb1, cb2 = PQ.polar7_codebooks()
    cbs = [cb1] + [cb2] * 6
    r = rng(2)
    for _ in range(20):
        idx = [r.integers(0, 16, 64)] + [r.integers(0, 4, 64 >> l) for l in range(1, 7)]
        R = float(np.float16(r.uniform(1, 20)))
        y = _tree_from_indices(idx, R, cbs).astype(f32)
        got, rad = PQ.encode_blocks(y[None], cbs)
        for l in range(7):
            assert np.array_equal(got[l][0], idx[l]), l
        yh = PQ.decode_blocks(got, rad, cbs)[0]
        assert np.max(np.abs(yh - y)) < 2e-5 * R


def test_indices_are_nearest_of_exact_angle_away_from_boundaries():
    cb1, cb2 = PQ.polar7_codebooks()
    cbs = [cb1] + [cb2] * 6
    y = rng(3).standard_normal((400, 128)).astype(f32)
    idx, _ = PQ.encode_blocks(y, cbs)
    r = y.astype(np.float64)
    checked = 0
    for lvl in range(7):
        a, b = r[:, 0::2], r[:, 1::2]
        th = np.arctan2(b, a)
        if lvl == 0:
            th = np.where(th < 0, th + 2 * np.pi, th)
        c = np.asarray(cbs[lvl], dtype=np.float64)
        d = np.abs(th[..., None] - c)
        best = np.argmin(d, axis=-1)
        srt = np.sort(d, axis=-1)
        clear = (srt[..., 1] - srt[..., 0]) > 2e-5   # not within 1e-5 rad of a boundary
        assert np.array_equal(idx[lvl][clear], best[clear]), lvl
        checked += clear.sum()
        r = np.sqrt(a * a + b * b)
    assert checked > 0.99 * 400 * 127


def test_decoded_norm_equals_radius_and_radius_is_norm():
    x = rng(4).standard_normal((50, 128)).astype(f32)
    S = rng(5).standard_normal((128, 128)).astype(f32)
    ang, norms, _ = PQ.polar7_encode(x, None, S)
    yh = PQ.polar7_decode(ang, norms)
    R = norms[:, 0].astype(np.float64)
    # the fp32 (cos, sin) tables satisfy cos^2 + sin^2 = 1 to ~1e-7 per level
    assert np.allclose(np.linalg.norm(yh, axis=1), R, rtol=2e-6)
    assert np.allclose(R, np.linalg.norm(x.astype(np.float64), axis=1), rtol=1e-3)


def test_recursive_contraction_equals_decode_dot():
    """The GPU scores by contracting q' bottom-up with the angle tree; that
    must equal <q', decode(k)>."""
    cb1, cb2 = PQ.polar7_codebooks()
    cst = [PQ.cs_table(cb1)] + [PQ.cs_table(cb2)] * 6
    x = rng(6).standard_normal((30, 128)).astype(f32)
    q = rng(7).standard_normal(128)
    ang, norms, _ = PQ.polar7_encode(x, None, rng(8).standard_normal((128, 128)).astype(f32))
    idx = PQ.unpack_polar7(ang)
    yh = PQ.polar7_decode(ang, norms)
    for n in range(30):
        c = q.copy()
        for lvl in range(7):
            cs = cst[lvl].astype(np.float64)[idx[lvl][n]]
            c = c[0::2] * cs[:, 0] + c[1::2] * cs[:, 1]
        assert abs(float(norms[n, 0]) * c[0] - yh[n] @ q) < 1e-9 * (1 + abs(yh[n] @ q))


def test_rotation_matches_float64_matmul():
    x = rng(9).standard_normal((20, 128)).astype(f32)
    P = np.linalg.qr(rng(10).standard_normal((128, 128)))[0].astype(f32)
    y = PQ.rotate_f32(x, P)
    ref = x.astype(np.float64) @ P.astype(np.float64).T
    assert np.max(np.abs(y - ref)) < 1e-5


# ------------------------------------------------------------- packing ----

def test_polar7_pack_known_bits():
    idx = [np.arange(64)[None] % 16] + [np.full((1, 64 >> l), l % 4) for l in range(1, 7)]
    w = PQ.pack_polar7(idx)[0]
    assert w[0] == 0x76543210 and w[1] == 0xFEDCBA98 and w[7] == 0xFEDCBA98
    assert w[8] == 0x55555555 and w[9] == 0x55555555          # level 2 = 1
    assert w[10] == 0xAAAAAAAA                                 # level 3 = 2
    # word 11: level 4 = 3 (bits 0-15), level 5 = 0, level 6 = 1, level 7 = 2
    assert w[11] == (0xFFFF | (0x0 << 16) | (0x5 << 24) | (0x2 << 28))
    back = PQ.unpack_polar7(PQ.pack_polar7(idx))
    for a, b in zip(back, idx):
        assert np.array_equal(a, b)


def test_ref_pack_known_bits_and_round_trip():
    i1 = np.arange(8, dtype=np.uint8)           # one block
    i2 = np.array([3, 2, 1, 0], dtype=np.uint8)
    i3 = np.array([1, 2], dtype=np.uint8)
    i4 = np.array([3], dtype=np.uint8)
    p1, p2, p3, p4 = PQ.pack_ref([i1, i2, i3, i4])
    assert p1[0] == 0x76543210 and p2[0] == 0b00011011 and p3[0] == 0b1001 and p4[0] == 3
    r = rng(11)
    lv = [r.integers(0, 16, 80), r.integers(0, 4, 40), r.integers(0, 4, 20), r.integers(0, 4, 10)]
    back = PQ.unpack_ref(*PQ.pack_ref(lv))
    for a, b in zip(back, lv):
        assert np.array_equal(a, b)


# ---------------------------------------------------------------- QJL ----

def test_qjl_sign_bits_closed_form():
    S = rng(12).standard_normal((128, 128)).astype(f32)
    r = np.zeros(128, dtype=f32)
    r[5] = 2.0
    bits = (PQ.sketch_f32(S, r[None])[0] >= 0)
    assert np.array_equal(bits, S[:, 5] >= 0)


def test_qjl_estimator_is_unbiased():
    """E_S[sqrt(pi/2)/m ||r|| <S q, sign(S r)>] = <q, r> (Monte Carlo)."""
    r0 = rng(13)
    q = r0.standard_normal(128)
    r = r0.standard_normal(128) * 0.3
    est = []
    for s in range(3000):
        S = np.random.default_rng(1000 + s).standard_normal((128, 128))
        est.append(math.sqrt(math.pi / 2) / 128 * np.linalg.norm(r) * ((S @ q) @ np.sign(S @ r)))
    est = np.array(est)
    se = est.std() / math.sqrt(len(est))
    assert abs(est.mean() - q @ r) < 4 * se


def test_qjl_corrects_polar_bias_on_average():
    """Over many sketch matrices the polar+QJL score is unbiased for <q', y>."""
    x = rng(14).standard_normal((1, 128)).astype(f32)
    qp = rng(15).standard_normal((1, 128)).astype(f32)
    true = float(qp[0].astype(np.float64) @ x[0].astype(np.float64))
    polar_only, full = [], []
    for s in range(400):
        S = np.random.default_rng(5000 + s).standard_normal((128, 128)).astype(f32)
        ang, norms, qj = PQ.polar7_encode(x, None, S)
        qs = PQ.qjl_query(qp, S)
        full.append(PQ.polar7_scores(qp, qs, ang[None], norms[None], qj[None], 1)[0, 0])
        polar_only.append(float(PQ.polar7_decode(ang, norms)[0] @ qp[0]))
    full = np.array(full)
    se = full.std() / math.sqrt(len(full))
    # the fp16 norms leave a tiny bias; the estimator is otherwise unbiased
    assert abs(full.mean() - true) < 4 * se + 1e-2 * abs(true) + 1e-3


# ------------------------------------------------------------ attention ----

def _ref16_setup(seed, Hkv, N, D):
    r = rng(seed)
    cbs = [np.sort(r.uniform(0, 2 * np.pi, 16)).astype(f32)] + \
          [np.sort(r.uniform(0, np.pi / 2, 4)).astype(f32) for _ in range(3)]
    k = r.standard_normal((Hkv * N, D)).astype(f32)
    out = PQ.polar_quantize(k, None, cbs)
    return cbs, k, out


def test_compressed_sdpa_single_key_returns_value():
    cbs, _, (i1, i2, i3, i4, rad) = _ref16_setup(16, 2, 1, 64)
    v = rng(17).standard_normal((2, 64)).astype(f32)
    q = rng(18).standard_normal((2, 64)).astype(f32)
    out = PQ.compressed_sdpa(q, i1, i2, i3, i4, rad, cbs, v, 0.125)
    assert np.allclose(out, v.astype(np.float64) / (1 + 1e-8), atol=1e-12)


def test_compressed_sdpa_identical_keys_average_values():
    cbs, k, _ = _ref16_setup(19, 1, 1, 64)
    kk = np.repeat(k, 7, axis=0)
    i1, i2, i3, i4, rad = PQ.polar_quantize(kk, None, cbs)
    v = rng(20).standard_normal((7, 64)).astype(f32)
    q = rng(21).standard_normal((1, 64)).astype(f32)
    out = PQ.compressed_sdpa(q, i1, i2, i3, i4, rad, cbs, v, 0.3)
    assert np.allclose(out[0], v.astype(np.float64).mean(0) / (1 + 1e-8 / 7), atol=1e-9)


def test_compressed_score_is_dot_with_decoded_keys():
    cbs, k, (i1, i2, i3, i4, rad) = _ref16_setup(22, 2, 9, 128)
    q = rng(23).standard_normal((4, 128)).astype(f32)
    s = PQ.compressed_score(q, i1, i2, i3, i4, rad, cbs, 9, 0.5, gqa=2)
    kh = PQ.polar_dequantize(i1, i2, i3, i4, rad, None, cbs, 128).reshape(2, 9, 128)
    for h in range(4):
        assert np.allclose(s[h], 0.5 * kh[h // 2] @ q[h].astype(np.float64), atol=1e-9)


def test_polar_dequantize_with_preconditioner_inverts_rotation():
    """Exact codebook hits encoded after rotation decode back to x."""
    P = np.linalg.qr(rng(24).standard_normal((64, 64)))[0].astype(f32)
    cbs = [((np.arange(16) + 0.5) * 2 * np.pi / 16).astype(f32)] + \
          [((np.arange(4) + 0.5) * np.pi / 8).astype(f32)] * 3
    r = rng(25)
    y = np.concatenate([_tree_from_indices([r.integers(0, 16, 8)] +
                                           [r.integers(0, 4, 8 >> l) for l in range(1, 4)],
                                           float(np.float16(2.0)), cbs) for _ in range(4)])
    x = (y @ P.astype(np.float64)).astype(f32)[None]  # y = x P^T  <=>  x = y P
    i1, i2, i3, i4, rad = PQ.polar_quantize(x, P, cbs)
    back = PQ.polar_dequantize(i1, i2, i3, i4, rad, P, cbs, 64)
    assert np.max(np.abs(back - x)) < 1e-4


def test_polar7_sdpa_closed_forms():
    cb1, cb2 = PQ.polar7_codebooks()
    from oracle import oracle as O
    x = rng(26).standard_normal((1, 5, 128)).astype(f32)
    S = rng(27).standard_normal((128, 128)).astype(f32)
    ang, norms, qj = PQ.polar7_encode(x.reshape(-1, 128), None, S)
    ang, norms, qj = ang.reshape(1, 5, 12), norms.reshape(1, 5, 2), qj.reshape(1, 5, 4)
    v = rng(28).standard_normal((1, 5, 128)).astype(f32)
    vq, vs, vb = O.quantize_int4(v.reshape(-1, 128))
    vq, vs, vb = vq.reshape(1, 5, 16), vs.reshape(1, 5, 2), vb.reshape(1, 5, 2)
    qp = rng(29).standard_normal((2, 128)).astype(f32)
    qs = PQ.qjl_query(qp, S)
    vdq = O.dequantize(vq, vs, vb)[0]
    # window 1 keeps only the last key -> its value row
    out = PQ.polar7_sdpa_int4v(qp, qs, ang, norms, qj, vq, vs, vb, gqa=2, window=1)
    assert np.allclose(out, vdq[4][None], atol=1e-12)
    # kv_len 0 -> zeros
    assert not PQ.polar7_sdpa_int4v(qp, qs, ang, norms, qj, vq, vs, vb, gqa=2, kv_len=0).any()
    # scale 0 -> uniform average of the attended values
    out = PQ.polar7_sdpa_int4v(qp, qs, ang, norms, qj, vq, vs, vb, gqa=2, scale=0.0)
    assert np.allclose(out, vdq.mean(0)[None], atol=1e-12)


def test_planted_mutant_swapping_cos_sin_is_caught():
    """A decoder that swaps cos and sin still preserves the norm but breaks
    the exact-hit round trip, which the tests above would flag."""
    cb1, cb2 = PQ.polar7_codebooks()
    cbs = [cb1] + [cb2] * 6
    r = rng(30)
    idx = [r.integers(0, 16, 64)] + [r.integers(0, 4, 64 >> l) for l in range(1, 7)]
    y = _tree_from_indices(idx, 4.0, cbs)
    bad = [np.asarray(c, dtype=np.float64)[::-1] * 0 + (np.pi / 2 - np.asarray(c, dtype=np.float64))
           for c in cbs]                                   # cos <-> sin
    ybad = _tree_from_indices(idx, 4.0, bad)
    assert abs(np.linalg.norm(ybad) - np.linalg.norm(y)) < 1e-9
    assert np.max(np.abs(ybad - y)) > 0.1
