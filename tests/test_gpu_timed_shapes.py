"""GPU parity at exactly the shapes bench.py times.

Each test builds its inputs the way the bench does (seeded N(0,1) on the GPU,
RMS-normed K, quantized by the separately bit-exact quantize kernel), runs the
same launch, and checks it against the oracle: the C float64 restatement on
the heads or sequences named in each test, or the numpy restatement where it
finishes in seconds.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import assert_close, dev, host, queries

pytestmark = pytest.mark.gpu


def gpu_cache(tq, Hkv, L, D, g, cap=None, sb=torch.float16):
    """bench.py's gen_cache: one int4 KV set built on the GPU."""
    cap = cap or L
    kq = torch.zeros((Hkv, cap, D // 8), dtype=torch.uint32, device="cuda")
    vq = torch.zeros_like(kq)
    ks = torch.zeros((Hkv, cap, D // 64), dtype=sb, device="cuda")
    kb, vs, vb = torch.zeros_like(ks), torch.zeros_like(ks), torch.zeros_like(ks)
    for h in range(Hkv):
        k = torch.randn((L, D), generator=g, device="cuda")
        k = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-6)
        v = torch.randn((L, D), generator=g, device="cuda")
        kq[h, :L], ks[h, :L], kb[h, :L] = tq.quantize(k, scale_dtype=sb)
        vq[h, :L], vs[h, :L], vb[h, :L] = tq.quantize(v, scale_dtype=sb)
    return kq, ks, kb, vq, vs, vb


def check_heads(out, qv, cache, kv_heads, gqa, window=0, kv_len=None, what=""):
    from oracle import coracle
    for kvh in kv_heads:
        sl = slice(kvh, kvh + 1)
        c = [host(t[sl]) for t in cache]
        ref = coracle.sdpa_int4_f64(qv[gqa * kvh:gqa * (kvh + 1)], *c, gqa, 1.0, window, kv_len)
        assert_close(out[gqa * kvh:gqa * (kvh + 1)], ref, f"{what} kv head {kvh}")


@pytest.mark.parametrize("sb", [torch.float16, torch.float32])
def test_headline_launch_32k(gpu, sb):
    """The driver-timed launch: Hq 32, Hkv 16, D 256, L 32768, bf16 q, no
    window -- 16 splits of 2048 keys, non-temporal loads -- on every kv
    head.  fp32 scale/bias is the reference's own cache dtype."""
    from gemma4metal_amd import _lib
    Hq, Hkv, D, L = 32, 16, 256, 32768
    plan = gpu.sdpa_plan(Hq, Hkv, D, L, sb_dtype=sb)
    assert plan == {"kernel": "sdpa_int4_mfma_kernel", "splits": 16, "chunk": 2048}
    g = torch.Generator(device="cuda").manual_seed(32768)
    cache = gpu_cache(gpu, Hkv, L, D, g, sb=sb)
    rng = np.random.default_rng(32768)
    qd, qv = queries(rng, (Hq, D), "bf16")
    out = host(gpu.sdpa_int4(qd, *cache, Hq // Hkv, 1.0, 0))
    check_heads(out, qv, cache, range(Hkv), 2, what="L=32768")
    assert _lib.last_error() == ""


@pytest.mark.parametrize("sb", [torch.float16, torch.float32])
def test_global_launch_32k(gpu, sb):
    """bench.py --workload global: Hq 32, Hkv 4 (GQA 8), D 512, L 32768 on
    the wave-specialised heads-as-columns kernel, for both scale/bias
    dtypes; two kv heads checked against the C oracle."""
    from gemma4metal_amd import _lib
    Hq, Hkv, D, L = 32, 4, 512, 32768
    assert gpu.sdpa_plan(Hq, Hkv, D, L, sb_dtype=sb)["kernel"] == "sdpa_int4_hc2_kernel"
    g = torch.Generator(device="cuda").manual_seed(5120)
    cache = gpu_cache(gpu, Hkv, L, D, g, sb=sb)
    rng = np.random.default_rng(5120)
    qd, qv = queries(rng, (Hq, D), "bf16")
    out = host(gpu.sdpa_int4(qd, *cache, Hq // Hkv, 1.0, 0))
    check_heads(out, qv, cache, (0, 3), 8, what="global L=32768")
    assert _lib.last_error() == ""


@pytest.mark.parametrize("L", [1024, 131072])
def test_sweep_points(gpu, L):
    """Sweep lengths of configs[2] not covered elsewhere (8192 and 262144
    are in test_gpu_sdpa.py)."""
    Hq, Hkv, D = 32, 16, 256
    g = torch.Generator(device="cuda").manual_seed(L)
    cache = gpu_cache(gpu, Hkv, L, D, g)
    rng = np.random.default_rng(L)
    qd, qv = queries(rng, (Hq, D), "bf16")
    out = host(gpu.sdpa_int4(qd, *cache, Hq // Hkv, 1.0, 0))
    heads = range(Hkv) if L <= 8192 else (0, 9, 15)
    check_heads(out, qv, cache, heads, 2, what=f"L={L}")


def test_sliding50_graph_step(gpu):
    """configs[1] as bench.py times it: 50 distinct sliding layers (L 786,
    W 1024) captured in one HIP graph.  Every replay equals the eager calls
    bit for bit (eager work on the same workspace and synchronisations
    between replays), and the layers match the oracle."""
    Hq, Hkv, D, L, W, layers = 32, 16, 256, 786, 1024, 50
    g = torch.Generator(device="cuda").manual_seed(786)
    sets = [gpu_cache(gpu, Hkv, L, D, g) for _ in range(layers)]
    rng = np.random.default_rng(786)
    qd, qv = queries(rng, (Hq, D), "bf16")
    outs = [torch.empty((Hq, D), dtype=torch.float32, device="cuda") for _ in range(layers)]

    def step():
        for s, o in zip(sets, outs):
            gpu.sdpa_int4(qd, *s, Hq // Hkv, 1.0, W, out=o)

    # The eager calls run on the capture stream, so the graph's kernels and
    # the eager calls between replays use that stream's one workspace (it
    # exists before capture, so nothing is allocated while capturing).
    cs = torch.cuda.Stream()
    with torch.cuda.stream(cs):
        step()
    torch.cuda.synchronize()
    eager = [host(o).copy() for o in outs]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cs):
        step()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert np.array_equal(host(o), eager[i]), f"replay {rep} layer {i}"
        # eager work on the graph's workspace between replays
        with torch.cuda.stream(cs):
            gpu.sdpa_int4(qd, *sets[rep], Hq // Hkv, 1.0, W, out=outs[0])
        torch.cuda.synchronize()
    for i in (0, 17, 49):
        ref = O.sdpa_int4(qv, *[host(t) for t in sets[i]], Hq // Hkv, 1.0, W)
        assert_close(eager[i], ref, f"layer {i}")


def test_mixed_layers_graph_step(gpu):
    """A Gemma-like decode step in one HIP graph: sliding layers (D 256,
    last-workgroup merge) around a global layer (D 512, the heads-as-columns
    kernel and the separate merge launch), all on one workspace.  Replays
    equal the eager step bit for bit; the global layer matches the oracle."""
    g = torch.Generator(device="cuda").manual_seed(4512)
    rng = np.random.default_rng(4512)
    slid = [gpu_cache(gpu, 16, 786, 256, g) for _ in range(3)]
    glob = gpu_cache(gpu, 4, 4096, 512, g)
    assert gpu.sdpa_plan(32, 4, 512, 4096)["kernel"] == "sdpa_int4_hc2_kernel"
    assert gpu.sdpa_plan(32, 4, 512, 4096)["splits"] > 1
    qs, _ = queries(rng, (32, 256), "bf16")
    qg, qgv = queries(rng, (32, 512), "bf16")
    outs = [torch.empty((32, 256), dtype=torch.float32, device="cuda") for _ in range(3)]
    outg = torch.empty((32, 512), dtype=torch.float32, device="cuda")

    def step():
        gpu.sdpa_int4(qs, *slid[0], 2, 1.0, 1024, out=outs[0])
        gpu.sdpa_int4(qs, *slid[1], 2, 1.0, 1024, out=outs[1])
        gpu.sdpa_int4(qg, *glob, 8, 1.0, 0, out=outg)
        gpu.sdpa_int4(qs, *slid[2], 2, 1.0, 1024, out=outs[2])

    cs = torch.cuda.Stream()  # eager calls and capture share this stream's workspace
    with torch.cuda.stream(cs):
        step()
    torch.cuda.synchronize()
    eager = [host(o).copy() for o in outs + [outg]]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cs):
        step()
    for rep in range(3):
        for o in outs + [outg]:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs + [outg]):
            assert np.array_equal(host(o), eager[i]), f"replay {rep} output {i}"
        # eager work on the graph's workspace between replays
        with torch.cuda.stream(cs):
            gpu.sdpa_int4(qg, *glob, 8, 1.0, 0, out=outg)
        torch.cuda.synchronize()
    check_heads(eager[3], qgv, glob, (1,), 8, what="global layer in the graph")


def test_ragged_full_size_append_then_attend(gpu):
    """configs[3] at full size, as bench.py times it: B 64, lengths
    U[512, 32768] (seed 4), W 1024 on even sequences, capacity 32769; one
    fp32 token per sequence quantized and appended, then ragged decode.
    The appended rows are bit-exact; eight sequences (the longest, the
    shortest, windowed and not) are checked on every kv head."""
    from oracle import coracle
    B, Hq, Hkv, D, cap = 64, 32, 16, 256, 32768 + 1
    rng = np.random.default_rng(4)
    lens = rng.integers(512, 32768, size=B, endpoint=True).astype(np.int32)
    wins = np.array([1024 if b % 2 == 0 else 0 for b in range(B)], np.int32)
    g = torch.Generator(device="cuda").manual_seed(64)
    cache = gpu.Int4KVCache(B, Hkv, cap, D, "cuda")
    for b in range(B):
        c = gpu_cache(gpu, Hkv, int(lens[b]), D, g)
        for dst, src in zip(cache.tensors(), c):
            dst[b, :, :int(lens[b])] = src
    cache.lengths.copy_(torch.from_numpy(lens).cuda())
    knew = torch.randn((B, Hkv, 1, D), generator=g, device="cuda")
    vnew = torch.randn((B, Hkv, 1, D), generator=g, device="cuda")
    qd, qv = queries(np.random.default_rng(44), (B, Hq, D), "bf16")
    cache.append(knew, vnew)
    out = host(cache.attend(qd, Hq // Hkv, windows=dev(wins), max_kv_len=cap))
    assert np.array_equal(host(cache.lengths), lens + 1)
    # appended rows: bit-exact MLX quantize of the new tokens
    kn, vn = knew.cpu().numpy(), vnew.cpu().numpy()
    for b in range(B):
        row = int(lens[b])
        for src, qt in ((kn, cache.tensors()[:3]), (vn, cache.tensors()[3:])):
            ref = O.quantize_int4(src[b, :, 0], "f16")
            got = [host(t[b, :, row]) for t in qt]
            for r, x in zip(ref, got):
                assert np.array_equal(np.asarray(r).view(np.uint8), np.asarray(x).view(np.uint8)), b
    picks = [int(np.argmax(lens)), int(np.argmin(lens))]
    picks += [b for b in range(B) if b not in picks][:6]
    for b in picks:
        n = int(lens[b]) + 1
        c = [host(t[b, :, :n]) for t in cache.tensors()]
        ref = coracle.sdpa_int4_f64(qv[b], *c, Hq // Hkv, 1.0, int(wins[b]))
        assert_close(out[b], ref, f"sequence {b} (L={n}, W={wins[b]})")
