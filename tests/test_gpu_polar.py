"""GPU parity of the PolarQuant / QJL path against oracle/polar.py.

Encoders (indices, packed words, fp16 radii/norms, sketch bits): bit-exact.
Decoders: 1e-5 relative to the vector norm.  Scores: max-abs 1e-3.
Attention: the parity tolerance (2e-3 abs / 1e-3 rel)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import polar as PQ
from tests.gpu_util import assert_close, dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32
SCORE_ATOL = 1e-3


@pytest.fixture(scope="module")
def pq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from gemma4metal_amd import polar
    return polar


def rand_codebooks(rng, packed):
    n1 = 16 if packed else 24
    n2 = 4 if packed else 7
    cb1 = np.sort(rng.uniform(0, 2 * np.pi, n1)).astype(f32)
    rest = [np.sort(rng.uniform(0, np.pi / 2, n2)).astype(f32) for _ in range(3)]
    return [cb1] + rest


def special_rows(D):
    """zeros, signed zeros, axis-aligned and tied pairs."""
    z = np.zeros((4, D), dtype=f32)
    z[1, :] = -0.0
    z[2, ::2] = 1.0
    z[3, :] = 1.0
    z[3, 1::4] = -1.0
    return z


def ortho(rng, D):
    return np.linalg.qr(rng.standard_normal((D, D)))[0].astype(f32)


# ------------------------------------------------------------ encode ---------

@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("rot", [False, True])
def test_polar_quantize_bit_exact(pq, D, packed, rot):
    rng = np.random.default_rng(D * 10 + packed * 3 + rot)
    x = np.concatenate([rng.standard_normal((300, D)).astype(f32), special_rows(D)])
    P = ortho(rng, D) if rot else None
    cbs = rand_codebooks(rng, packed)
    ref = PQ.polar_quantize(x, P, cbs)
    dcb = [dev(c) for c in cbs]
    dP = dev(P) if rot else None
    if packed:
        got = pq.polar_quantize_packed(dev(x), dP, *dcb)
        want = list(PQ.pack_ref(ref[:4])) + [ref[4]]
    else:
        got = pq.polar_quantize(dev(x), dP, *dcb)
        want = list(ref)
    for i, (g, w) in enumerate(zip(got, want)):
        g = host(g)
        if w.dtype == np.float16:
            g, w = g.view(np.uint16), w.view(np.uint16)
        mism = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
        assert mism.size == 0, f"output {i}: {mism.size} mismatches, first at {mism[:5]}"


# ------------------------------------------------------------ decode ---------

@pytest.mark.parametrize("D", [64, 128])
def test_polar_dequantize_variants(pq, D):
    rng = np.random.default_rng(40 + D)
    x = rng.standard_normal((200, D)).astype(f32)
    P = ortho(rng, D)
    cbs = rand_codebooks(rng, packed=True)
    i1, i2, i3, i4, rad = PQ.polar_quantize(x, P, cbs)
    dcb = [dev(c) for c in cbs]
    di = [dev(a) for a in (i1, i2, i3, i4, rad)]
    norm = np.linalg.norm(x, axis=1, keepdims=True)

    y_ref = PQ.polar_dequantize(i1, i2, i3, i4, rad, None, cbs, D)
    x_ref = PQ.polar_dequantize(i1, i2, i3, i4, rad, P, cbs, D)
    y = host(pq.polar_dequantize_fast(*di, *dcb, D))
    xx = host(pq.polar_dequantize(*di, dev(P), *dcb))
    assert np.max(np.abs(y - y_ref) / norm) < 1e-5
    assert np.max(np.abs(xx - x_ref) / norm) < 1e-5

    packed = [dev(a) for a in PQ.pack_ref([i1, i2, i3, i4])] + [di[4]]
    yp = host(pq.polar_dequantize_packed(*packed, *dcb, D))
    cs = [pq.cos_sin_table(c) for c in dcb]
    ypf = host(pq.polar_dequantize_packed_fast(*packed, *cs, D))
    assert np.max(np.abs(yp - y_ref) / norm) < 1e-5
    assert np.max(np.abs(ypf - y_ref) / norm) < 1e-5


# ------------------------------------------------- reference scores / sdpa ----

@pytest.mark.parametrize("D,Hq,Hkv,N", [(128, 4, 4, 300), (128, 8, 4, 1500), (64, 2, 1, 77),
                                        (256, 16, 2, 700)])
def test_compressed_score(pq, D, Hq, Hkv, N):
    rng = np.random.default_rng(D + Hq + N)
    cbs = rand_codebooks(rng, packed=False)
    k = rng.standard_normal((Hkv * N, D)).astype(f32)
    q = rng.standard_normal((Hq, D)).astype(f32)
    idx = PQ.polar_quantize(k, None, cbs)
    scale = 1.0 / np.sqrt(D)
    ref = PQ.compressed_score(q, *idx, cbs, N, scale, gqa=Hq // Hkv)
    got = host(pq.compressed_score(dev(q), *[dev(a) for a in idx], *[dev(c) for c in cbs], N,
                                   scale=scale, num_kv_heads=Hkv))
    assert np.max(np.abs(got - ref)) < SCORE_ATOL
    # packed layout (codebooks within 16/4 entries)
    cbs_p = rand_codebooks(rng, packed=True)
    idx = PQ.polar_quantize(k, None, cbs_p)
    ref = PQ.compressed_score(q, *idx, cbs_p, N, scale, gqa=Hq // Hkv)
    packed = [dev(a) for a in PQ.pack_ref(idx[:4])] + [dev(idx[4])]
    got = host(pq.compressed_score_packed(dev(q), *packed, *[dev(c) for c in cbs_p], N,
                                          scale=scale, num_kv_heads=Hkv))
    assert np.max(np.abs(got - ref)) < SCORE_ATOL


@pytest.mark.parametrize("D,Hq,Hkv,N", [(128, 1, 1, 1), (128, 4, 4, 300), (128, 8, 2, 5000),
                                        (64, 2, 2, 2000), (256, 4, 1, 900)])
def test_compressed_sdpa(pq, D, Hq, Hkv, N):
    rng = np.random.default_rng(7 * D + Hq + N)
    cbs = rand_codebooks(rng, packed=False)
    k = rng.standard_normal((Hkv * N, D)).astype(f32)
    v = rng.standard_normal((Hkv * N, D)).astype(f32)
    q = rng.standard_normal((Hq, D)).astype(f32)
    idx = PQ.polar_quantize(k, None, cbs)
    scale = 0.0884
    ref = PQ.compressed_sdpa(q, *idx, cbs, v, scale, gqa=Hq // Hkv)
    got = host(pq.compressed_sdpa(dev(q), *[dev(a) for a in idx], *[dev(c) for c in cbs], dev(v),
                                  scale=scale, num_kv_heads=Hkv))
    assert_close(got, ref, f"compressed_sdpa D{D} Hq{Hq} Hkv{Hkv} N{N}")


# --------------------------------------------------------------- polar7 --------

def p7_inputs(seed, n, rot=True):
    rng = np.random.default_rng(seed)
    x = np.concatenate([rng.standard_normal((n, 128)).astype(f32), special_rows(128)])
    P = ortho(rng, 128) if rot else None
    S = rng.standard_normal((128, 128)).astype(f32)
    return rng, x, P, S


@pytest.mark.parametrize("n,rot", [(1, True), (500, True), (777, False)])
def test_polar7_encode_bit_exact(pq, n, rot):
    rng, x, P, S = p7_inputs(100 + n, n, rot)
    ang, norms, qjl = PQ.polar7_encode(x, P, S)
    codec = pq.Polar7Codec(dev(P) if rot else None, dev(S))
    ga, gn, gq = (host(t) for t in codec.encode(dev(x)))
    nrm16 = norms.view(np.uint16).astype(np.uint32)
    want_n = nrm16[:, 0] | (nrm16[:, 1] << 16)
    for name, g, w in (("angles", ga, ang), ("norms", gn, want_n), ("qjl", gq, qjl)):
        mism = np.flatnonzero((g != w).reshape(g.shape[0], -1).any(axis=1))
        assert mism.size == 0, f"{name}: rows {mism[:8]} differ ({mism.size} rows)"


def test_polar7_kv_append_positions(pq):
    rng, x, P, S = p7_inputs(5, 0)
    B, Hkv, T, cap = 3, 2, 4, 10
    k_new = rng.standard_normal((B, Hkv, T, 128)).astype(f32)
    codec = pq.Polar7Codec(dev(P), dev(S))
    caches = codec.new_cache(Hkv, cap, batch=B)
    pos = np.array([0, 8, -2], dtype=np.int32)       # row 8: 2 fit; -2: rows 0, 1 fit
    codec.append(dev(k_new), *caches, dev(pos))
    ang, norms, qjl = PQ.polar7_encode(k_new.reshape(-1, 128), P, S)
    ang = ang.reshape(B, Hkv, T, 12)
    ga = host(caches[0])
    for b in range(B):
        for h in range(Hkv):
            for t in range(T):
                r = pos[b] + t
                if 0 <= r < cap:
                    assert np.array_equal(ga[b, h, r], ang[b, h, t]), (b, h, t)
    written = np.zeros((B, cap), bool)
    for b in range(B):
        for t in range(T):
            if 0 <= pos[b] + t < cap:
                written[b, pos[b] + t] = True
    assert not ga[~written[:, None, :].repeat(Hkv, 1)].any()


def test_prepare_query(pq):
    rng, _, P, S = p7_inputs(6, 0)
    q = rng.standard_normal((32, 128)).astype(f32)
    codec = pq.Polar7Codec(dev(P), dev(S))
    tab, qp, qs = (host(t) for t in codec.prepare_query(dev(q), with_vectors=True))
    qp_ref = q.astype(np.float64) @ P.astype(np.float64).T
    qs_ref = qp_ref @ S.astype(np.float64).T
    assert np.max(np.abs(qp - qp_ref)) < 1e-4
    assert np.max(np.abs(qs - qs_ref)) < 1e-3
    # tables: level-1 dot products, QJL byte subset sums, sum of S q'
    cb1, _ = PQ.polar7_codebooks()
    cs1 = PQ.cs_table(cb1).astype(np.float64)
    t1 = qp_ref[:, 0::2, None] * cs1[:, 0] + qp_ref[:, 1::2, None] * cs1[:, 1]
    assert np.max(np.abs(tab[:, :1024].reshape(32, 64, 16) - t1)) < 1e-4
    bits = (np.arange(256)[:, None] >> np.arange(8)) & 1
    tq = np.einsum("hpi,bi->hpb", qs_ref.reshape(32, 16, 8), bits)
    assert np.max(np.abs(tab[:, 1024:5120].reshape(32, 16, 256) - tq)) < 1e-3
    # sum of S q' as four partial sums, then zero padding
    assert np.max(np.abs(tab[:, 5120:5124].sum(1) - qs_ref.sum(1))) < 1e-2
    assert not tab[:, 5124:].any()


@pytest.mark.parametrize("rot", [True, False])
def test_prepare_query_entry_points_agree(pq, rot):
    """tq_polar7_prepare_query (S applied to q') and tq_polar7_prepare_query_sp
    (S P applied to q, the codec's path) give the same tables up to fp32
    rounding, and S P from tq_polar7_sketch_precondition is S P."""
    import ctypes
    from gemma4metal_amd._lib import call
    rng, _, P, S = p7_inputs(8, 0)
    q = rng.standard_normal((32, 128)).astype(f32)
    codec = pq.Polar7Codec(dev(P) if rot else None, dev(S))
    sp_ref = S.astype(np.float64) @ (P.astype(np.float64) if rot else np.eye(128))
    assert np.max(np.abs(host(codec.SP) - sp_ref)) < 1e-4
    qd = dev(q)
    tab_sp = host(codec.prepare_query(qd))
    tab = torch.empty((32, pq.P7_QTAB), dtype=torch.float32, device="cuda")
    ptr = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)
    call("tq_polar7_prepare_query", ptr(qd), ptr(codec.P), ptr(codec.S), ptr(codec.cs), 32,
         ptr(tab), ptr(None), ptr(None), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    tab = host(tab)
    assert np.max(np.abs(tab[:, :5120] - tab_sp[:, :5120])) < 1e-3
    assert np.max(np.abs(tab[:, 5120:5124].sum(1) - tab_sp[:, 5120:5124].sum(1))) < 1e-2


def p7_cache_on_gpu(pq, seed, Hkv, L, rot=True):
    """Keys encoded on the GPU (the encoder is checked bit-exact separately),
    int4 V from the oracle quantizer; returns device + host copies."""
    rng = np.random.default_rng(seed)
    P = ortho(rng, 128) if rot else None
    S = rng.standard_normal((128, 128)).astype(f32)
    codec = pq.Polar7Codec(dev(P) if rot else None, dev(S))
    k = torch.from_numpy(rng.standard_normal((Hkv, L, 128)).astype(f32)).cuda()
    dk = codec.encode(k)
    v = rng.standard_normal((Hkv, L, 128)).astype(f32)
    return rng, codec, P, S, dk, [host(t) for t in dk], v


def host_norms(n):
    """(.., 2) float16 view of the packed norms word."""
    return n.view(np.uint16).reshape(n.shape + (2,)).view(np.float16)


@pytest.mark.parametrize("Hq,Hkv,L,scale", [(32, 16, 2000, 1.0), (4, 4, 333, 0.3), (16, 2, 1200, 1.0),
                                            (8, 8, 70, 1.0),
                                            (32, 16, 5000, 1.0),   # 3 blocks of 2048, partial last
                                            (8, 2, 4096, 0.5)])    # exactly two blocks
def test_polar7_score(pq, Hq, Hkv, L, scale):
    rng, codec, P, S, dk, hk, _ = p7_cache_on_gpu(pq, Hq + L, Hkv, L)
    q = rng.standard_normal((Hq, 128)).astype(f32)
    tab, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    got = host(codec.score(tab, *dk, scale))
    ref = PQ.polar7_scores(host(qp), host(qs), hk[0], host_norms(hk[1]), hk[2], Hq // Hkv, scale)
    err = np.abs(got - ref)
    assert err.max() < SCORE_ATOL, f"max score err {err.max():.3e}"


@pytest.mark.parametrize("Hq,Hkv,L,scale,rot", [(32, 16, 5000, 1.0, True), (4, 4, 333, 0.3, False),
                                                (16, 2, 1200, 1.0, True), (8, 8, 70, 1.0, True),
                                                (8, 2, 4096, 0.5, False)])
def test_polar7_score_q(pq, Hq, Hkv, L, scale, rot):
    """Scores straight from q (query tables built in each workgroup):
    against the oracle and against the two-launch path."""
    rng, codec, P, S, dk, hk, _ = p7_cache_on_gpu(pq, 7 * Hq + L, Hkv, L, rot=rot)
    q = rng.standard_normal((Hq, 128)).astype(f32)
    got = host(codec.score_q(dev(q), *dk, scale))
    tab, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    two = host(codec.score(tab, *dk, scale))
    assert np.max(np.abs(got - two)) < 1e-4, f"fused vs two-launch {np.max(np.abs(got - two)):.3e}"
    ref = PQ.polar7_scores(host(qp), host(qs), hk[0], host_norms(hk[1]), hk[2], Hq // Hkv, scale)
    err = np.abs(got - ref)
    assert err.max() < SCORE_ATOL, f"max score err {err.max():.3e}"
    assert codec.score_q(dev(q), *dk, scale, kv_len=0).shape == (Hq, 0)


@pytest.mark.parametrize("Hq,Hkv,L,W,sb", [
    (32, 16, 786, 0, "f16"), (32, 16, 3000, 1024, "f16"), (4, 4, 1, 0, "f32"),
    (8, 1, 5000, 0, "f16"), (16, 2, 20000, 0, "f16"), (2, 2, 400, 0, "f32")])
def test_polar7_sdpa_int4v(pq, Hq, Hkv, L, W, sb):
    rng, codec, P, S, dk, hk, v = p7_cache_on_gpu(pq, 3 * Hq + L + W, Hkv, L)
    vq, vs, vb = O.quantize_int4(v, sb)
    q = rng.standard_normal((Hq, 128)).astype(f32)
    tab, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    got = host(codec.sdpa_int4v(tab, *dk, dev(vq), dev(vs), dev(vb), 1.0, W))
    ref = PQ.polar7_sdpa_int4v(host(qp), host(qs), hk[0], host_norms(hk[1]), hk[2], vq, vs, vb,
                               Hq // Hkv, 1.0, W)
    assert_close(got, ref, f"polar7 sdpa Hq{Hq} Hkv{Hkv} L{L} W{W} {sb}")


@pytest.mark.parametrize("Hq,Hkv,L,W,sb,rot", [
    (32, 16, 3000, 0, "f16", True), (32, 16, 3000, 1024, "f16", True), (4, 4, 1, 0, "f32", True),
    (8, 1, 5000, 0, "f16", False), (16, 2, 20000, 0, "f32", True), (2, 2, 400, 0, "f16", False)])
def test_polar7_sdpa_int4v_q(pq, Hq, Hkv, L, W, sb, rot):
    """Attention straight from q (query tables built in each workgroup):
    against the oracle, and against the two-launch path on the same
    inputs (same tables up to the order of the fp32 sums of q' and S q':
    the scores then differ in the last bits, and so may the bf16 hi/lo split
    of a weight, ~2^-17 of it)."""
    rng, codec, P, S, dk, hk, v = p7_cache_on_gpu(pq, 5 * Hq + L + W, Hkv, L, rot=rot)
    vq, vs, vb = O.quantize_int4(v, sb)
    q = rng.standard_normal((Hq, 128)).astype(f32)
    d = [dev(vq), dev(vs), dev(vb)]
    got = host(codec.sdpa_int4v_q(dev(q), *dk, *d, 1.0, W))
    tab, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    two = host(codec.sdpa_int4v(tab, *dk, *d, 1.0, W))
    assert np.max(np.abs(got - two)) < 1e-4, f"fused vs two-launch {np.max(np.abs(got - two)):.3e}"
    ref = PQ.polar7_sdpa_int4v(host(qp), host(qs), hk[0], host_norms(hk[1]), hk[2], vq, vs, vb,
                               Hq // Hkv, 1.0, W)
    assert_close(got, ref, f"polar7 fused sdpa Hq{Hq} Hkv{Hkv} L{L} W{W} {sb} rot{rot}")


def test_polar7_sdpa_int4v_q_empty_and_prefix(pq):
    rng, codec, P, S, dk, hk, v = p7_cache_on_gpu(pq, 78, 2, 300)
    vq, vs, vb = O.quantize_int4(v)
    q = rng.standard_normal((4, 128)).astype(f32)
    d = [dev(vq), dev(vs), dev(vb)]
    assert not host(codec.sdpa_int4v_q(dev(q), *dk, *d, kv_len=0)).any()
    got = host(codec.sdpa_int4v_q(dev(q), *dk, *d, kv_len=123))
    _, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    ref = PQ.polar7_sdpa_int4v(host(qp), host(qs), hk[0], host_norms(hk[1]), hk[2], vq, vs, vb, 2,
                               kv_len=123)
    assert_close(got, ref, "fused prefix 123")


def test_polar7_sdpa_empty_and_prefix(pq):
    rng, codec, P, S, dk, hk, v = p7_cache_on_gpu(pq, 77, 2, 300)
    vq, vs, vb = O.quantize_int4(v)
    q = rng.standard_normal((4, 128)).astype(f32)
    tab, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    d = [dev(vq), dev(vs), dev(vb)]
    z = host(codec.sdpa_int4v(tab, *dk, *d, kv_len=0))
    assert not z.any()
    got = host(codec.sdpa_int4v(tab, *dk, *d, kv_len=123))
    ref = PQ.polar7_sdpa_int4v(host(qp), host(qs), hk[0], host_norms(hk[1]), hk[2], vq, vs, vb, 2,
                               kv_len=123)
    assert_close(got, ref, "prefix 123")


def test_polar7_full_size_two_heads(pq):
    """The polar7 decode shape (Hq 32, Hkv 16, L 32768): the whole launch,
    checked against the oracle on two kv heads' outputs."""
    Hq, Hkv, L = 32, 16, 32768
    rng, codec, P, S, dk, hk, v = p7_cache_on_gpu(pq, 2026, Hkv, L)
    vq, vs, vb = O.quantize_int4(v)
    q = rng.standard_normal((Hq, 128)).astype(f32)
    tab, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    got = host(codec.sdpa_int4v(tab, *dk, dev(vq), dev(vs), dev(vb)))
    fused = host(codec.sdpa_int4v_q(dev(q), *dk, dev(vq), dev(vs), dev(vb)))
    assert np.max(np.abs(fused - got)) < 1e-4, f"fused vs two-launch {np.max(np.abs(fused - got)):.3e}"
    hqp, hqs = host(qp), host(qs)
    for kvh in (0, 11):
        sl = slice(kvh, kvh + 1)
        ref = PQ.polar7_sdpa_int4v(hqp[2 * kvh:2 * kvh + 2], hqs[2 * kvh:2 * kvh + 2], hk[0][sl],
                                   host_norms(hk[1][sl]), hk[2][sl], vq[sl], vs[sl], vb[sl], 2)
        assert_close(got[2 * kvh:2 * kvh + 2], ref, f"kv head {kvh}")
        assert_close(fused[2 * kvh:2 * kvh + 2], ref, f"fused, kv head {kvh}")


def test_polar7_score_full_size_two_heads(pq):
    """The score-only launch at the configs[4] shape (Hq 32, Hkv 16,
    L 32768: 16 blocks of 2048 keys per head), checked on two kv heads."""
    Hq, Hkv, L = 32, 16, 32768
    rng, codec, P, S, dk, hk, _ = p7_cache_on_gpu(pq, 4242, Hkv, L)
    q = rng.standard_normal((Hq, 128)).astype(f32)
    tab, qp, qs = codec.prepare_query(dev(q), with_vectors=True)
    got = host(codec.score(tab, *dk))
    hqp, hqs = host(qp), host(qs)
    for kvh in (0, 13):
        sl = slice(kvh, kvh + 1)
        ref = PQ.polar7_scores(hqp[2 * kvh:2 * kvh + 2], hqs[2 * kvh:2 * kvh + 2], hk[0][sl],
                               host_norms(hk[1][sl]), hk[2][sl], 2)
        err = np.abs(got[2 * kvh:2 * kvh + 2] - ref)
        assert err.max() < SCORE_ATOL, f"kv head {kvh}: max score err {err.max():.3e}"
