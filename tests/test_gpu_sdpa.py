"""GPU parity: fused int4 decode attention vs the oracle (2e-3 abs / 1e-3 rel)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import assert_close, dev, host, queries

pytestmark = pytest.mark.gpu


def host_cache(rng, Hkv, cap, D, sb="f16"):
    k = O.rms_norm(rng.standard_normal((Hkv, cap, D)).astype(np.float32))
    v = rng.standard_normal((Hkv, cap, D)).astype(np.float32)
    return O.quantize_int4(k, sb) + O.quantize_int4(v, sb)


@pytest.mark.parametrize("Hq,Hkv,D,L,W,qdt,sb,scale", [
    (2, 1, 128, 33, 0, "f32", "f32", 1.0),        # tiny decode (the reference test shape)
    (2, 1, 128, 33, 0, "f32", "f16", 1.0),
    (16, 16, 256, 10, 0, "f32", "f32", 1.0),      # reference test shape
    (32, 16, 256, 786, 1024, "bf16", "f16", 1.0), # Gemma sliding layer at L 786
    (32, 16, 256, 1500, 1024, "bf16", "f16", 1.0),  # window active
    (32, 4, 512, 300, 0, "bf16", "f16", 1.0),     # Gemma global layer (GQA 8, D 512)
    (8, 1, 512, 129, 0, "f16", "f32", 0.0625),
    (12, 4, 128, 1000, 0, "bf16", "f16", 1.0),    # GQA 3 -> head subgroups of 1
    (24, 4, 256, 640, 100, "bf16", "f16", 1.0),   # GQA 6 -> subgroups of 2
    (16, 4, 128, 5000, 0, "bf16", "f16", 1.0),    # GQA 4
    (4, 4, 256, 1, 0, "bf16", "f16", 1.0),        # single key
    (32, 16, 256, 8192, 0, "bf16", "f16", 1.0),   # many splits
])
def test_sdpa_matches_oracle(gpu, Hq, Hkv, D, L, W, qdt, sb, scale):
    rng = np.random.default_rng(Hq * 7919 + L * 31 + D)
    qd, qv = queries(rng, (Hq, D), qdt)
    c = host_cache(rng, Hkv, L, D, sb)
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], Hq // Hkv, scale, W)
    ref = O.sdpa_int4(qv, *c, Hq // Hkv, scale, W)
    assert_close(host(out), ref, f"Hq{Hq} Hkv{Hkv} D{D} L{L} W{W}")


@pytest.mark.parametrize("Hq,Hkv,D,L,W", [
    (32, 16, 256, 3000, 0),    # Gemma sliding layer shape, packed columns
    (32, 16, 256, 1500, 1024), # window active
    (2, 1, 128, 33, 0),        # the reference test shape
    (32, 4, 256, 1500, 0),     # GQA 8 at D 256: two 4-head subgroups per kv head
    (12, 4, 512, 2000, 0),     # D 512, GQA 3: one-head subgroups
    (8, 8, 512, 700, 0),       # D 512, GQA 1
    (16, 2, 128, 2100, 0),     # D 128, GQA 8: all 16 columns
])
def test_f32_scales_on_matrix_cores(gpu, Hq, Hkv, D, L, W):
    """fp32 scale/bias, the reference's cache dtype (lib/turboquant.h:199,
    fed by quantize at engine/gemma4_multilayer.cpp:228), runs on the
    matrix-core kernel and matches the oracle."""
    assert gpu.sdpa_plan(Hq, Hkv, D, L, sb_dtype=torch.float32,
                         sliding_window=W)["kernel"] == "sdpa_int4_mfma_kernel"
    rng = np.random.default_rng(Hq * 17 + L + D)
    qd, qv = queries(rng, (Hq, D), "bf16")
    c = host_cache(rng, Hkv, L, D, "f32")
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], Hq // Hkv, 1.0, W)
    assert_close(host(out), O.sdpa_int4(qv, *c, Hq // Hkv, 1.0, W), f"f32 s/b Hq{Hq} Hkv{Hkv} D{D}")


def test_gqa8_d256_fp16(gpu):
    rng = np.random.default_rng(88)
    Hq, Hkv, D, L = 32, 4, 256, 2500
    assert gpu.sdpa_plan(Hq, Hkv, D, L)["kernel"] == "sdpa_int4_mfma_kernel"
    qd, qv = queries(rng, (Hq, D), "bf16")
    c = host_cache(rng, Hkv, L, D, "f16")
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], 8)
    assert_close(host(out), O.sdpa_int4(qv, *c, 8), "GQA 8 D 256")


def test_sdpa_prefix_of_capacity_and_repeat_calls(gpu):
    rng = np.random.default_rng(3)
    Hq, Hkv, D, cap = 32, 16, 256, 3000
    qd, qv = queries(rng, (Hq, D), "bf16")
    c = host_cache(rng, Hkv, cap, D)
    cd = [dev(a) for a in c]
    for n in (2999, 1, 64, 65, 1234, 3000):
        out = gpu.sdpa_int4(qd, *cd, 2, 1.0, 0, kv_len=n)
        assert_close(host(out), O.sdpa_int4(qv, *c, 2, 1.0, 0, kv_len=n), f"kv_len {n}")
    # repeated identical calls are bit-identical (workspace counters reset)
    a = host(gpu.sdpa_int4(qd, *cd, 2, kv_len=2500))
    b = host(gpu.sdpa_int4(qd, *cd, 2, kv_len=2500))
    assert np.array_equal(a, b)


def test_sdpa_empty_keys_zero(gpu):
    rng = np.random.default_rng(4)
    qd, qv = queries(rng, (4, 128), "bf16")
    c = host_cache(rng, 2, 8, 128)
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], 2, kv_len=0)
    assert np.all(host(out) == 0)


def test_sdpa_full_context_split_k(gpu):
    """The context sweep's largest size (L=262144): cache built on the GPU
    by the (separately bit-exact) quantize kernel, checked against the C oracle
    on the heads of two kv heads."""
    from oracle import coracle
    Hq, Hkv, D, L = 32, 16, 256, 262144
    g = torch.Generator(device="cuda").manual_seed(1234)
    kq = torch.empty((Hkv, L, D // 8), dtype=torch.uint32, device="cuda")
    vq = torch.empty_like(kq)
    ks = torch.empty((Hkv, L, D // 64), dtype=torch.float16, device="cuda")
    kb, vs, vb = torch.empty_like(ks), torch.empty_like(ks), torch.empty_like(ks)
    for h in range(Hkv):
        k = torch.randn((L, D), generator=g, device="cuda")
        k = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-6)
        v = torch.randn((L, D), generator=g, device="cuda")
        kq[h], ks[h], kb[h] = gpu.quantize(k, scale_dtype=torch.float16)
        vq[h], vs[h], vb[h] = gpu.quantize(v, scale_dtype=torch.float16)
    rng = np.random.default_rng(77)
    qd, qv = queries(rng, (Hq, D), "bf16")
    out = host(gpu.sdpa_int4(qd, kq, ks, kb, vq, vs, vb, 2))
    for kvh in (0, 15):
        sl = slice(kvh, kvh + 1)
        c = [host(t[sl]) for t in (kq, ks, kb, vq, vs, vb)]
        ref = coracle.sdpa_int4_f64(qv[2 * kvh:2 * kvh + 2], *c, 2)
        assert_close(out[2 * kvh:2 * kvh + 2], ref, f"L=262144 kv head {kvh}")


@pytest.mark.parametrize("sb", ["f16", "f32"])
def test_ragged_batch_matches_oracle(gpu, sb):
    rng = np.random.default_rng(21)
    B, Hq, Hkv, D, cap = 9, 32, 16, 256, 2100
    lens = np.array([2100, 0, 1, 513, 1024, 1025, 64, 2000, 777], np.int32)
    wins = np.array([1024, 0, 1024, 0, 1024, 1024, 0, 5, 1024], np.int32)
    qd, qv = queries(rng, (B, Hq, D), "bf16")
    k = O.rms_norm(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32))
    v = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    c = O.quantize_int4(k, sb) + O.quantize_int4(v, sb)
    out = gpu.sdpa_int4_ragged(qd, *[dev(a) for a in c], dev(lens), 2, windows=dev(wins))
    ref = O.sdpa_int4_ragged(qv, *c, lens, wins, 2)
    assert_close(host(out), ref, "ragged")


@pytest.mark.parametrize("long_len,W", [(20000, 0), (9000, 4096)])
def test_ragged_skewed_batch(gpu, long_len, W):
    """One long sequence among 63 short ones: the device chooses its own
    chunk for the batch (the long sequence split, the short ones whole)
    and runs the jobs longest first; every sequence matches the oracle.
    The cache is quantized on the GPU, row range by row range."""
    from oracle import coracle
    rng = np.random.default_rng(long_len + W)
    B, Hq, Hkv, D = 64, 32, 16, 256
    cap = long_len + 1
    lens = np.concatenate([[long_len], rng.integers(1, 600, size=B - 1)]).astype(np.int32)
    wins = np.full(B, W, np.int32)
    g = torch.Generator(device="cuda").manual_seed(long_len)
    kq = torch.zeros((B, Hkv, cap, D // 8), dtype=torch.uint32, device="cuda")
    vq = torch.zeros_like(kq)
    ks = torch.zeros((B, Hkv, cap, D // 64), dtype=torch.float16, device="cuda")
    kb, vs, vb = torch.zeros_like(ks), torch.zeros_like(ks), torch.zeros_like(ks)
    for b in range(B):
        n = int(lens[b])
        for h in range(Hkv):
            k = torch.randn((n, D), generator=g, device="cuda")
            k = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-6)
            v = torch.randn((n, D), generator=g, device="cuda")
            kq[b, h, :n], ks[b, h, :n], kb[b, h, :n] = gpu.quantize(k, scale_dtype=torch.float16)
            vq[b, h, :n], vs[b, h, :n], vb[b, h, :n] = gpu.quantize(v, scale_dtype=torch.float16)
    qd, qv = queries(rng, (B, Hq, D), "bf16")
    out = host(gpu.sdpa_int4_ragged(qd, kq, ks, kb, vq, vs, vb, dev(lens), Hq // Hkv,
                                    windows=dev(wins)))
    for b in range(B):
        n = int(lens[b])
        cb = [host(x[b, :, :n]) for x in (kq, ks, kb, vq, vs, vb)]
        ref = coracle.sdpa_int4_f64(qv[b], *cb, Hq // Hkv, 1.0, W)
        assert_close(out[b], ref, f"sequence {b} (L={n})")


def test_append_then_attend_round_trip(gpu):
    """Config-4 step at reduced size: quantize+append one fp32 token per
    sequence, then ragged decode over the grown caches."""
    rng = np.random.default_rng(31)
    B, Hq, Hkv, D, cap = 6, 32, 16, 256, 1200
    lens0 = np.array([1000, 10, 1100, 512, 700, 1199], np.int32)
    wins = np.array([1024, 0] * 3, np.int32)
    cache = gpu.Int4KVCache(B, Hkv, cap, D, "cuda")
    k0 = O.rms_norm(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32))
    v0 = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    hc = O.quantize_int4(k0) + O.quantize_int4(v0)
    for t, a in zip(cache.tensors(), hc):
        t.copy_(dev(a))
    cache.lengths.copy_(dev(lens0))
    kn = O.rms_norm(rng.standard_normal((B, Hkv, 1, D)).astype(np.float32))
    vn = rng.standard_normal((B, Hkv, 1, D)).astype(np.float32)
    cache.append(dev(kn), dev(vn))
    qd, qv = queries(rng, (B, Hq, D), "bf16")
    out = cache.attend(qd, 2, windows=dev(wins))
    ref_cache = dict(zip(["kq", "ks", "kb", "vq", "vs", "vb"], [a.copy() for a in hc]))
    O.kv_append_int4(ref_cache, kn, vn, lens0)
    ref = O.sdpa_int4_ragged(qv, *ref_cache.values(), lens0 + 1, wins, 2)
    assert_close(host(out), ref, "append+attend")


def test_workspace_reuse_across_shapes(gpu):
    """Regression: split counters must be back at zero after every call, so
    calls with different shapes / split counts sharing one workspace stay
    correct in any order."""
    rng = np.random.default_rng(41)
    cases = []
    # the last case has batch * heads = 2560 > 2048, so its split counters
    # are closer than one line apart (stride 25 ints instead of 32)
    many = rng.integers(1, 49, size=80).tolist()
    for (B, cap, lens, wins) in [(2, 900, [900, 513], [0, 0]), (3, 1500, [1500, 7, 1025], [1024, 0, 0]),
                                 (1, 4000, [4000], [0]), (4, 700, [1, 700, 650, 129], [0, 64, 0, 0]),
                                 (80, 48, many, [0] * 80)]:
        qd, qv = queries(rng, (B, 32, 256), "bf16")
        k = O.rms_norm(rng.standard_normal((B, 16, cap, 256)).astype(np.float32))
        v = rng.standard_normal((B, 16, cap, 256)).astype(np.float32)
        c = O.quantize_int4(k) + O.quantize_int4(v)
        ref = O.sdpa_int4_ragged(qv, *c, np.array(lens), np.array(wins), 2)
        cases.append((qd, [dev(a) for a in c], dev(np.array(lens, np.int32)),
                      dev(np.array(wins, np.int32)), ref))
    for rep in range(3):
        for i in (0, 2, 4, 1, 3, 4, 2, 0):
            qd, cd, ld, wd, ref = cases[i]
            out = gpu.sdpa_int4_ragged(qd, *cd, ld, 2, windows=wd)
            assert_close(host(out), ref, f"rep {rep} case {i}")


def test_workspace_shared_by_both_merge_forms(gpu):
    """One workspace serving, in turn, D=512 calls (split partials merged by
    a second launch) and calls whose last workgroup merges them (D=256
    decode, a ragged batch, D=128): the partial slots overlap, and whatever
    one form leaves there must not leak into the other's results."""
    rng = np.random.default_rng(77)
    q512, v512 = queries(rng, (32, 512), "bf16")
    c512 = host_cache(rng, 4, 5000, 512)
    r512 = O.sdpa_int4(v512, *c512, 8, 1.0, 0)
    q256, v256 = queries(rng, (32, 256), "bf16")
    c256 = host_cache(rng, 16, 4000, 256)
    r256 = O.sdpa_int4(v256, *c256, 2, 1.0, 0)
    q128, v128 = queries(rng, (8, 128), "f32")
    c128 = host_cache(rng, 4, 3000, 128)
    r128 = O.sdpa_int4(v128, *c128, 2, 1.0, 0)
    lens, wins = [3000, 1, 2100], [0, 0, 1024]
    qr, vr = queries(rng, (3, 32, 256), "bf16")
    k = O.rms_norm(rng.standard_normal((3, 16, 3000, 256)).astype(np.float32))
    v = rng.standard_normal((3, 16, 3000, 256)).astype(np.float32)
    cr = O.quantize_int4(k) + O.quantize_int4(v)
    rr = O.sdpa_int4_ragged(vr, *cr, np.array(lens), np.array(wins), 2)
    d512, d256, d128, dr = ([dev(a) for a in c] for c in (c512, c256, c128, cr))
    ld, wd = dev(np.array(lens, np.int32)), dev(np.array(wins, np.int32))
    assert gpu.sdpa_plan(32, 4, 512, 5000)["kernel"] == "sdpa_int4_hc2_kernel"
    for rep in range(3):
        for what in ("512", "256", "512", "ragged", "128", "512", "512", "256"):
            if what == "512":
                got, ref = gpu.sdpa_int4(q512, *d512, 8, 1.0, 0), r512
            elif what == "256":
                got, ref = gpu.sdpa_int4(q256, *d256, 2, 1.0, 0), r256
            elif what == "128":
                got, ref = gpu.sdpa_int4(q128, *d128, 2, 1.0, 0), r128
            else:
                got, ref = gpu.sdpa_int4_ragged(qr, *dr, ld, 2, windows=wd), rr
            assert_close(host(got), ref, f"rep {rep} {what}")


@pytest.mark.parametrize("Hq,Hkv,L,W,qdt", [
    (32, 4, 5000, 0, "bf16"),     # Gemma global layer: many splits, partial last iteration
    (32, 4, 3001, 1024, "bf16"),  # window active
    (32, 2, 2100, 0, "f16"),      # GQA 16: two 8-head subgroups per kv head
    (8, 1, 1, 0, "f32"),          # single key
    (16, 2, 129, 0, "bf16"),
])
def test_sdpa_d512_gqa8(gpu, Hq, Hkv, L, W, qdt):
    """D=512 with 8 query heads per kv head (the heads-as-columns kernel)."""
    rng = np.random.default_rng(Hq * 131 + L * 7 + W)
    qd, qv = queries(rng, (Hq, 512), qdt)
    c = host_cache(rng, Hkv, L, 512, "f16")
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], Hq // Hkv, 1.0, W)
    ref = O.sdpa_int4(qv, *c, Hq // Hkv, 1.0, W)
    assert_close(host(out), ref, f"D512 Hq{Hq} Hkv{Hkv} L{L} W{W}")


@pytest.mark.parametrize("Hq,Hkv,L,W,qdt", [
    (32, 4, 5000, 0, "bf16"),     # Gemma global layer, fp32 scale/bias (the reference's cache)
    (32, 4, 3001, 1024, "bf16"),  # window active
    (32, 2, 2100, 0, "f16"),      # GQA 16: two 8-head subgroups per kv head
    (8, 1, 1, 0, "f32"),          # single key
    (16, 2, 129, 0, "bf16"),      # one split, odd step count
    (16, 2, 257, 0, "bf16"),
])
def test_sdpa_d512_gqa8_f32_scales(gpu, Hq, Hkv, L, W, qdt):
    """fp32 scale/bias (lib/turboquant.h:199) on the wave-specialised
    heads-as-columns kernel."""
    assert gpu.sdpa_plan(Hq, Hkv, 512, L, sb_dtype=torch.float32,
                         sliding_window=W)["kernel"] == "sdpa_int4_hc2_kernel"
    rng = np.random.default_rng(Hq * 113 + L * 5 + W)
    qd, qv = queries(rng, (Hq, 512), qdt)
    c = host_cache(rng, Hkv, L, 512, "f32")
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], Hq // Hkv, 1.0, W)
    ref = O.sdpa_int4(qv, *c, Hq // Hkv, 1.0, W)
    assert_close(host(out), ref, f"f32 s/b D512 Hq{Hq} Hkv{Hkv} L{L} W{W}")


def test_sdpa_d512_gqa8_f32_scales_ragged(gpu):
    rng = np.random.default_rng(52)
    B, Hq, Hkv, D, cap = 3, 32, 4, 512, 1500
    lens = np.array([1500, 1, 700], np.int32)
    wins = np.array([0, 1024, 100], np.int32)
    qd, qv = queries(rng, (B, Hq, D), "bf16")
    k = O.rms_norm(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32))
    v = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    c = O.quantize_int4(k, "f32") + O.quantize_int4(v, "f32")
    out = gpu.sdpa_int4_ragged(qd, *[dev(a) for a in c], dev(lens), 8, windows=dev(wins))
    ref = O.sdpa_int4_ragged(qv, *c, lens, wins, 8)
    assert_close(host(out), ref, "D512 f32 ragged")


@pytest.mark.parametrize("L", [2, 31, 32, 33, 100, 127, 128, 129, 255, 257, 383, 640, 1000])
def test_sdpa_d512_gqa8_lengths(gpu, L):
    """The wave-specialised D=512 kernel at lengths that give one split with
    odd / even step counts and key streams with no keys."""
    rng = np.random.default_rng(4000 + L)
    Hq, Hkv = 16, 2
    qd, qv = queries(rng, (Hq, 512), "bf16")
    c = host_cache(rng, Hkv, L, 512, "f16")
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], 8)
    assert_close(host(out), O.sdpa_int4(qv, *c, 8), f"D512 L{L}")


def test_sdpa_d512_gqa8_ragged(gpu):
    rng = np.random.default_rng(51)
    B, Hq, Hkv, D, cap = 3, 32, 4, 512, 1500
    lens = np.array([1500, 1, 700], np.int32)
    wins = np.array([0, 1024, 100], np.int32)
    qd, qv = queries(rng, (B, Hq, D), "bf16")
    k = O.rms_norm(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32))
    v = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    c = O.quantize_int4(k, "f16") + O.quantize_int4(v, "f16")
    out = gpu.sdpa_int4_ragged(qd, *[dev(a) for a in c], dev(lens), 8, windows=dev(wins))
    ref = O.sdpa_int4_ragged(qv, *c, lens, wins, 8)
    assert_close(host(out), ref, "D512 ragged")


@pytest.mark.parametrize("Hq,Hkv,D", [(32, 16, 256), (32, 4, 512), (8, 2, 128), (8, 4, 512)])
def test_sdpa_large_value_range(gpu, Hq, Hkv, D):
    """V of magnitude ~1e3 (fp16 scales ~1e2): the matrix-core P.V weights
    p * s_v must not overflow.  Tolerance scaled by the value magnitude."""
    rng = np.random.default_rng(D + Hq)
    mag = 300.0
    qd, qv = queries(rng, (Hq, D), "bf16")
    k = O.rms_norm(rng.standard_normal((Hkv, 700, D)).astype(np.float32))
    v = (rng.standard_normal((Hkv, 700, D)) * mag).astype(np.float32)
    c = O.quantize_int4(k, "f16") + O.quantize_int4(v, "f16")
    got = np.asarray(host(gpu.sdpa_int4(qd, *[dev(a) for a in c], Hq // Hkv)), np.float64)
    ref = np.asarray(O.sdpa_int4(qv, *c, Hq // Hkv), np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    d = np.abs(got - ref)
    assert d.max() <= 2e-3 * mag, d.max()
    assert np.linalg.norm(d) / np.linalg.norm(ref) <= 1e-3


def ramp_inputs(rng, Hq, Hkv, S, cap, D, qdt, sign):
    """K rows sign * r_t * u + small noise, u a unit direction per kv head and
    r_t = slope * t; queries along u (norm sqrt(D)).  A query's scores then
    rise (sign 1) or fall (sign -1) by ~0.1 log2 units per key, so the online
    softmax's running max moves past any threshold again and again along a
    wave's keys (or never moves after its first keys)."""
    slope = 0.1 / np.log2(np.e) / np.sqrt(D)
    u = rng.standard_normal((Hkv, 1, D))
    u /= np.linalg.norm(u, axis=-1, keepdims=True)
    t = np.arange(cap, dtype=np.float64)[None, :, None]
    k = (sign * slope * t * u + 0.05 * rng.standard_normal((Hkv, cap, D))).astype(np.float32)
    v = rng.standard_normal((Hkv, cap, D)).astype(np.float32)
    cache = O.quantize_int4(k, "f16") + O.quantize_int4(v, "f16")
    g = Hq // Hkv
    q = np.repeat(u[:, 0, :], g, axis=0) * np.sqrt(D) + 0.1 * rng.standard_normal((S, Hq, D))
    q = q.astype(np.float32)
    if qdt == "bf16":
        bits = O.f32_to_bf16_bits(q)
        qd = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
        q = O.bf16_bits_to_f32(bits)
    else:
        qd = torch.from_numpy(q).cuda()
    return qd, q, cache


@pytest.mark.parametrize("Hq,Hkv,D,L", [
    (32, 16, 256, 3000),  # matrix-core kernel, D 256
    (8, 2, 128, 2000),    # matrix-core kernel, D 128
    (32, 4, 512, 3000),   # heads-as-columns kernel (D 512, GQA 8)
    (8, 4, 512, 1500),    # matrix-core kernel, D 512 GQA 2
])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_sdpa_rising_and_falling_scores(gpu, Hq, Hkv, D, L, sign):
    """Scores that climb (or fall) steadily along the context exercise the
    online softmax's rescale on every batch of keys (or on none after the
    first)."""
    rng = np.random.default_rng(D + L + int(sign > 0))
    qd, qv, c = ramp_inputs(rng, Hq, Hkv, 1, L, D, "bf16", sign)
    qd, qv = qd[0], qv[0]
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], Hq // Hkv)
    ref = O.sdpa_int4(qv, *c, Hq // Hkv)
    assert_close(host(out), ref, f"ramp {sign:+.0f} Hq{Hq} Hkv{Hkv} D{D} L{L}")


@pytest.mark.parametrize("Hq,Hkv,D,S,prior", [
    (32, 16, 256, 128, 900),  # tile kernel
    (32, 4, 512, 96, 700),    # tile kernel, D 512
    (32, 4, 512, 40, 500),    # split-K prefill on the heads-as-columns kernel
])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_sdpa_prefill_rising_and_falling_scores(gpu, Hq, Hkv, D, S, prior, sign):
    rng = np.random.default_rng(D + S + int(sign > 0))
    qd, qv, c = ramp_inputs(rng, Hq, Hkv, S, prior + S, D, "bf16", sign)
    out = gpu.sdpa_int4_prefill(qd, *[dev(a) for a in c], prior, Hq // Hkv, 1.0, 0)
    ref = O.sdpa_int4_prefill(qv, *c, prior, Hq // Hkv, 1.0, 0)
    assert_close(host(out), ref, f"prefill ramp {sign:+.0f} D{D} S{S}")


def test_sdpa_global_layer_full_context(gpu):
    """Gemma global layer at 32k (Hq 32, Hkv 4, D 512): cache built on the GPU
    by the (separately bit-exact) quantize kernel, two kv heads checked
    against the C oracle."""
    from oracle import coracle
    Hq, Hkv, D, L = 32, 4, 512, 32768
    g = torch.Generator(device="cuda").manual_seed(512)
    kq = torch.empty((Hkv, L, D // 8), dtype=torch.uint32, device="cuda")
    vq = torch.empty_like(kq)
    ks = torch.empty((Hkv, L, D // 64), dtype=torch.float16, device="cuda")
    kb, vs, vb = torch.empty_like(ks), torch.empty_like(ks), torch.empty_like(ks)
    for h in range(Hkv):
        k = torch.randn((L, D), generator=g, device="cuda")
        k = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-6)
        v = torch.randn((L, D), generator=g, device="cuda")
        kq[h], ks[h], kb[h] = gpu.quantize(k, scale_dtype=torch.float16)
        vq[h], vs[h], vb[h] = gpu.quantize(v, scale_dtype=torch.float16)
    rng = np.random.default_rng(78)
    qd, qv = queries(rng, (Hq, D), "bf16")
    out = host(gpu.sdpa_int4(qd, kq, ks, kb, vq, vs, vb, 8))
    for kvh in (0, 3):
        sl = slice(kvh, kvh + 1)
        c = [host(t[sl]) for t in (kq, ks, kb, vq, vs, vb)]
        ref = coracle.sdpa_int4_f64(qv[8 * kvh:8 * kvh + 8], *c, 8)
        assert_close(out[8 * kvh:8 * kvh + 8], ref, f"global L=32768 kv head {kvh}")


def test_ring_cache_equals_window_rule(gpu):
    """Sliding-window eviction by a ring of capacity W: after appends that
    wrap the ring (a prefill longer than W, single tokens, a 3-token step),
    attention over the ring (window 0) equals the reference window rule W
    over the full history (lib/turboquant.metal:779)."""
    rng = np.random.default_rng(61)
    B, Hq, Hkv, D, W = 2, 32, 16, 256, 64
    ring = gpu.Int4KVCache(B, Hkv, W, D, "cuda", ring=True)
    hist_k = np.zeros((B, Hkv, 0, D), np.float32)
    hist_v = np.zeros((B, Hkv, 0, D), np.float32)
    for T in (70, 1, 1, 3, 1):
        k = O.rms_norm(rng.standard_normal((B, Hkv, T, D)).astype(np.float32))
        v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
        ring.append(dev(k), dev(v))
        hist_k = np.concatenate([hist_k, k], axis=2)
        hist_v = np.concatenate([hist_v, v], axis=2)
        qd, qv = queries(rng, (B, Hq, D), "bf16")
        out = ring.attend(qd, Hq // Hkv)
        n = hist_k.shape[2]
        c = O.quantize_int4(hist_k) + O.quantize_int4(hist_v)
        ref = O.sdpa_int4_ragged(qv, *c, np.full(B, n, np.int32), np.full(B, W, np.int32), Hq // Hkv)
        assert_close(host(out), ref, f"ring after {n} tokens")
    assert np.all(host(ring.lengths) == hist_k.shape[2])


def test_prompt_cache_file_round_trip(gpu, tmp_path):
    """save_kv_cache / load_kv_cache (reference prompt-cache layout) with GPU
    caches: a global (linear) and a sliding (ring) layer reload into fresh
    caches whose attention output is bit-identical."""
    from gemma4metal_amd import kvcache_io as IO
    rng = np.random.default_rng(71)
    Hq, Hkv, D = 32, 16, 256
    lin = gpu.Int4KVCache(1, Hkv, 300, D, "cuda")
    ring = gpu.Int4KVCache(1, Hkv, 128, D, "cuda", ring=True)
    for T in (150, 1, 2):
        k = dev(O.rms_norm(rng.standard_normal((1, Hkv, T, D)).astype(np.float32)))
        v = dev(rng.standard_normal((1, Hkv, T, D)).astype(np.float32))
        lin.append(k, v)
        ring.append(k, v)
    p = str(tmp_path / "kv.safetensors")
    IO.save_kv_cache(p, [lin, ring], cache_offset=153)
    lin2 = gpu.Int4KVCache(1, Hkv, 300, D, "cuda")
    ring2 = gpu.Int4KVCache(1, Hkv, 128, D, "cuda", ring=True)
    assert IO.load_kv_cache(p, [lin2, ring2]) == 153
    qd, _ = queries(rng, (1, Hq, D), "bf16")
    for a, b in ((lin, lin2), (ring, ring2)):
        assert np.array_equal(host(a.attend(qd, 2)), host(b.attend(qd, 2)))


@pytest.mark.parametrize("Hq,Hkv,D,S,prior,W,qdt", [
    (32, 16, 256, 100, 0, 0, "bf16"),      # first prefill chunk, causal only
    (32, 16, 256, 64, 700, 128, "bf16"),   # chunk after a cached prefix, sliding window
    (32, 4, 512, 48, 300, 0, "bf16"),      # Gemma global layer (heads-as-columns kernel)
    (8, 2, 128, 33, 5, 16, "f32"),
    (4, 4, 256, 1, 90, 0, "f16"),          # a single query = decode
    (16, 8, 128, 37, 20, 5, "bf16"),       # 4 queries per workgroup, partial last group, window 5
    (4, 4, 256, 7, 0, 0, "f32"),           # GQA 1: 4 queries per workgroup
    (8, 4, 512, 9, 30, 0, "bf16"),         # D 512, GQA 2
    (32, 16, 256, 300, 1200, 256, "bf16"),  # long prefix, window, many groups
])
def test_sdpa_prefill_matches_oracle(gpu, Hq, Hkv, D, S, prior, W, qdt):
    """Multi-query attention with the engine fallback's causal + window mask
    (engine/gemma4_multilayer.cpp:343-364)."""
    rng = np.random.default_rng(S * 13 + prior + D)
    cap = prior + S + 7
    qd, qv = queries(rng, (S, Hq, D), qdt)
    c = host_cache(rng, Hkv, cap, D, "f16")
    out = gpu.sdpa_int4_prefill(qd, *[dev(a) for a in c], prior, Hq // Hkv, 1.0, W)
    ref = O.sdpa_int4_prefill(qv, *c, prior, Hq // Hkv, 1.0, W)
    assert_close(host(out), ref, f"prefill S{S} prior{prior} W{W} D{D}")


@pytest.mark.parametrize("Hq,Hkv,D,S,prior,W,qdt", [
    (32, 16, 256, 200, 0, 0, "bf16"),      # GQA 2: 32 queries x 2 heads per workgroup
    (32, 16, 256, 128, 900, 256, "bf16"),  # cached prefix + window
    (16, 2, 128, 70, 33, 0, "f16"),        # GQA 8: 8 queries x 8 heads, partial last group
    (8, 8, 128, 65, 10, 16, "f32"),        # GQA 1: 64 queries per workgroup, tiny window
    (4, 1, 256, 96, 2000, 0, "bf16"),      # GQA 4, long prefix
    (32, 4, 512, 100, 300, 0, "bf16"),     # Gemma global layer: 8 queries x 8 heads
    (8, 1, 512, 70, 40, 64, "f16"),        # D 512 with a window, partial last group
    (16, 8, 512, 64, 10, 0, "f32"),        # D 512 GQA 2: 32 queries x 2 heads
])
@pytest.mark.parametrize("sb", ["f16", "f32"])
def test_sdpa_prefill_tile_kernel(gpu, Hq, Hkv, D, S, prior, W, qdt, sb):
    """Prefills of >= 64 queries at D 128 / 256 / 512 run the K/V-tile kernel
    (fp16 / bf16 hi-lo matrix-core products), for fp16 and fp32 (the
    reference's cache dtype) scale/bias."""
    plan = gpu.sdpa_plan(Hq, Hkv, D, prior + S, mode="prefill", batch=S, sliding_window=W,
                         sb_dtype=torch.float32 if sb == "f32" else torch.float16)
    assert plan["kernel"] == ("prefill_int4_kernel" if D == 512 else "prefill_int4_ws_kernel")
    rng = np.random.default_rng(S * 7 + prior + Hq)
    cap = prior + S + 3
    qd, qv = queries(rng, (S, Hq, D), qdt)
    c = host_cache(rng, Hkv, cap, D, sb)
    out = gpu.sdpa_int4_prefill(qd, *[dev(a) for a in c], prior, Hq // Hkv, 1.0, W)
    ref = O.sdpa_int4_prefill(qv, *c, prior, Hq // Hkv, 1.0, W)
    assert_close(host(out), ref, f"tiles S{S} prior{prior} W{W} D{D} gqa{Hq // Hkv}")


@pytest.mark.parametrize("Hq,Hkv,L,W", [(32, 4, 5000, 0), (32, 4, 3001, 1024), (16, 2, 129, 0)])
def test_d512_one_wave_and_wave_specialised_kernels_agree(gpu, tq_env, Hq, Hkv, L, W):
    """The two D=512 GQA-8 kernels (TQ_HC_IMPL=1 selects the one-wave one)
    compute the same products: outputs agree to fp32 rounding."""
    rng = np.random.default_rng(L + W)
    qd, qv = queries(rng, (Hq, 512), "bf16")
    c = host_cache(rng, Hkv, L, 512, "f16")
    cd = [dev(a) for a in c]
    two = host(gpu.sdpa_int4(qd, *cd, Hq // Hkv, 1.0, W))
    tq_env("TQ_HC_IMPL", "1")
    one = host(gpu.sdpa_int4(qd, *cd, Hq // Hkv, 1.0, W))
    assert np.abs(two - one).max() < 1e-4
    assert_close(one, O.sdpa_int4(qv, *c, Hq // Hkv, 1.0, W), "one-wave D512")


@pytest.mark.parametrize("D,gqa", [(256, 2), (128, 8)])
def test_prefill_tile_kernels_agree(gpu, tq_env, D, gqa):
    """The wave-specialised and one-role tile kernels (TQ_PREFILL_WS=0)
    compute the same products in the same order: bit-identical outputs."""
    rng = np.random.default_rng(D + gqa)
    Hkv, S, prior, W = 4, 130, 400, 256
    qd, qv = queries(rng, (S, Hkv * gqa, D), "bf16")
    c = host_cache(rng, Hkv, prior + S, D, "f16")
    cd = [dev(a) for a in c]
    ws = host(gpu.sdpa_int4_prefill(qd, *cd, prior, gqa, 1.0, W))
    tq_env("TQ_PREFILL_WS", "0")
    one = host(gpu.sdpa_int4_prefill(qd, *cd, prior, gqa, 1.0, W))
    assert np.array_equal(ws, one)
    assert_close(ws, O.sdpa_int4_prefill(qv, *c, prior, gqa, 1.0, W), f"ws prefill D{D}")


@pytest.mark.parametrize("Hq,Hkv,D,L", [(32, 16, 256, 3000), (8, 2, 128, 1500), (8, 4, 512, 700)])
def test_valu_kernel_forced_matches_oracle(gpu, tq_env, Hq, Hkv, D, L):
    """TQ_SDPA_IMPL=valu runs the VALU kernel for fp16 caches too."""
    rng = np.random.default_rng(D + L)
    qd, qv = queries(rng, (Hq, D), "bf16")
    c = host_cache(rng, Hkv, L, D, "f16")
    tq_env("TQ_SDPA_IMPL", "valu")
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], Hq // Hkv)
    assert_close(host(out), O.sdpa_int4(qv, *c, Hq // Hkv), f"valu D{D} L{L}")


@pytest.mark.parametrize("chunk", [128, 384, 4096])
def test_forced_chunk_matches_oracle(gpu, tq_env, chunk):
    """TQ_SDPA_CHUNK overrides the split planner (more or fewer splits)."""
    rng = np.random.default_rng(chunk)
    Hq, Hkv, D, L = 32, 16, 256, 6000
    qd, qv = queries(rng, (Hq, D), "bf16")
    c = host_cache(rng, Hkv, L, D, "f16")
    tq_env("TQ_SDPA_CHUNK", str(chunk))
    out = gpu.sdpa_int4(qd, *[dev(a) for a in c], 2)
    assert_close(host(out), O.sdpa_int4(qv, *c, 2), f"chunk {chunk}")


def test_sdpa_prefill_tile_and_split_paths_agree(gpu, tq_env):
    rng = np.random.default_rng(91)
    Hq, Hkv, D, S, prior, W = 32, 16, 256, 160, 500, 300
    qd, _ = queries(rng, (S, Hq, D), "bf16")
    cd = [dev(a) for a in host_cache(rng, Hkv, prior + S, D, "f16")]
    tiles = host(gpu.sdpa_int4_prefill(qd, *cd, prior, 2, 1.0, W))
    tq_env("TQ_PREFILL_IMPL", "splitk")
    split = host(gpu.sdpa_int4_prefill(qd, *cd, prior, 2, 1.0, W))
    assert np.abs(tiles - split).max() < 1e-3


def test_fresh_workspace_on_non_default_streams(gpu):
    """Calls on non-default streams, each getting a fresh workspace on its
    first call: the zero-fill is ordered on the call's stream, and two
    streams never share counters.  Decode and ragged, interleaved on two
    streams without synchronisation between them, match the default-stream
    results bit for bit."""
    rng = np.random.default_rng(515)
    Hq, Hkv, D, L = 32, 16, 256, 9000
    qd, qv = queries(rng, (Hq, D), "bf16")
    cd = [dev(a) for a in host_cache(rng, Hkv, L, D)]
    B, cap = 3, 2000
    lens = np.array([2000, 17, 1500], np.int32)
    qr, _ = queries(rng, (B, Hq, D), "bf16")
    k = O.rms_norm(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32))
    v = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    cr = [dev(a) for a in (O.quantize_int4(k) + O.quantize_int4(v))]
    ld = dev(lens)
    ref_d = host(gpu.sdpa_int4(qd, *cd, 2))
    ref_r = host(gpu.sdpa_int4_ragged(qr, *cr, ld, 2))
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(4):
        for s in (s1, s2):
            with torch.cuda.stream(s):
                outs.append(("d", gpu.sdpa_int4(qd, *cd, 2, stream=s)))
                outs.append(("r", gpu.sdpa_int4_ragged(qr, *cr, ld, 2, stream=s)))
    torch.cuda.synchronize()
    for kind, o in outs:
        assert np.array_equal(host(o), ref_d if kind == "d" else ref_r), kind


def _poison_tail(c, n_valid, sb):
    """Returns device copies of cache c whose rows from n_valid on hold
    non-finite scales and biases (rows past the sequence, never written by
    an append): K scale +Inf, K bias NaN, V scale NaN, V bias -Inf."""
    kq, ks, kb, vq, vs, vb = [a.copy() for a in c]
    if sb == "f16":
        nan, inf = np.uint16(0x7E00).view(np.float16), np.float16(np.inf)
    else:
        nan, inf = np.float32(np.nan), np.float32(np.inf)
    ks[..., n_valid:, :] = inf
    kb[..., n_valid:, :] = nan
    vs[..., n_valid:, :] = nan
    vb[..., n_valid:, :] = -inf
    return [dev(a) for a in (kq, ks, kb, vq, vs, vb)]


@pytest.mark.parametrize("sb", ["f16", "f32"])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 16, 256), (8, 4, 128), (8, 4, 512)])
@pytest.mark.parametrize("n", [1, 17, 31])
def test_short_sequence_unwritten_tail(gpu, sb, Hq, Hkv, D, n):
    """A sequence shorter than one 32-key block in a cache of 64 rows: rows
    past it (never written) hold NaN / Inf scales and biases, and the output
    still matches the oracle over the first n rows -- decode (kv_len),
    ragged (seq_lens) and prefill (causal end inside the first block)."""
    rng = np.random.default_rng(900 + n + D)
    cap = 64
    c = host_cache(rng, Hkv, cap, D, sb)
    cd = _poison_tail(c, n, sb)
    qd, qv = queries(rng, (Hq, D), "bf16")
    out = gpu.sdpa_int4(qd, *cd, Hq // Hkv, 1.0, 0, kv_len=n)
    cut = [a[:, :n] for a in c]
    assert_close(host(out), O.sdpa_int4(qv, *cut, Hq // Hkv, 1.0, 0), f"decode n={n}")
    # ragged: every sequence of the batch ends at n (caches (B, Hkv, cap, .))
    B = 2
    cb = [np.stack([a, a]) for a in c]
    cbd = _poison_tail(cb, n, sb)
    lens = np.full(B, n, np.int32)
    qr, qrv = queries(rng, (B, Hq, D), "bf16")
    out_r = gpu.sdpa_int4_ragged(qr, *cbd, dev(lens), Hq // Hkv)
    ref_r = O.sdpa_int4_ragged(qrv, *cb, lens, np.zeros(B, np.int32), Hq // Hkv)
    assert_close(host(out_r), ref_r, f"ragged n={n}")
    # prefill: queries at positions n - S .. n - 1 over rows [0, n)
    S = min(n, 5)
    qp, qpv = queries(rng, (S, Hq, D), "bf16")
    out_p = gpu.sdpa_int4_prefill(qp, *cd, n - S, Hq // Hkv, 1.0, 0)
    ref_p = O.sdpa_int4_prefill(qpv, *c, n - S, Hq // Hkv, 1.0, 0)
    assert_close(host(out_p), ref_p, f"prefill n={n}")
