"""GPU parity: quantize / append / dequantize are bit-exact against the oracle."""
import zlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import dev, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("x_dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("sb", ["f16", "f32"])
@pytest.mark.parametrize("mode", ["mlx", "minmax"])
def test_quantize_bit_exact(gpu, x_dtype, sb, mode):
    rng = np.random.default_rng(zlib.crc32(f"{x_dtype}-{sb}-{mode}".encode()))
    x = (rng.standard_normal((300, 256)) * rng.uniform(0.01, 20, (300, 1))).astype(np.float32)
    x[0] = 0.0
    x[1] = 3.0
    x[2, :64] = np.arange(64) % 16
    x[3, :8] = [0, 15, 7.5, 6.5, 8.5, 0.5, 0, 0]
    if x_dtype == "f16":
        x = x.astype(np.float16).astype(np.float32)
        xd = dev(x.astype(np.float16))
    elif x_dtype == "bf16":
        bits = O.f32_to_bf16_bits(x)
        x = O.bf16_bits_to_f32(bits)
        xd = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
    else:
        xd = dev(x)
    sdt = torch.float16 if sb == "f16" else torch.float32
    wq, s, b = gpu.quantize(xd, scale_dtype=sdt, mode=mode)
    rq, rs, rb = O.quantize_int4(x, sb, mode)
    assert np.array_equal(host(wq), rq)
    assert np.array_equal(host(s).view(np.uint16 if sb == "f16" else np.uint32),
                          rs.view(np.uint16 if sb == "f16" else np.uint32))
    assert np.array_equal(host(b).view(np.uint16 if sb == "f16" else np.uint32),
                          rb.view(np.uint16 if sb == "f16" else np.uint32))


@pytest.mark.parametrize("D", [64, 128, 512, 4096])
def test_quantize_dims(gpu, D):
    rng = np.random.default_rng(D)
    x = rng.standard_normal((37, D)).astype(np.float32)
    wq, s, b = gpu.quantize(dev(x), scale_dtype=torch.float32)
    rq, rs, rb = O.mlx_affine_quantize(x)
    assert np.array_equal(host(wq), rq) and np.array_equal(host(s), rs) and np.array_equal(host(b), rb)


def test_dequantize_matches(gpu):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    wq, s, b = O.quantize_int4(x, "f16")
    out = host(gpu.dequantize(dev(wq), dev(s), dev(b)))
    ref = O.dequantize(wq, s, b)
    np.testing.assert_allclose(out, ref, rtol=2e-7, atol=1e-7)


def test_kv_append_bit_exact_and_bounds(gpu):
    rng = np.random.default_rng(11)
    B, Hkv, cap, D = 4, 3, 40, 256
    cache = gpu.Int4KVCache(B, Hkv, cap, D, "cuda")
    ref = {k: np.zeros(tuple(t.shape), np.uint32 if t.dtype == torch.uint32 else np.float16)
           for k, t in zip(["kq", "ks", "kb", "vq", "vs", "vb"], cache.tensors())}
    start = np.array([0, 5, 38, 39], np.int32)
    cache.lengths.copy_(torch.from_numpy(start))
    pos = start.copy()
    for step, T in enumerate([1, 2, 1]):
        k = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
        v = rng.standard_normal((B, Hkv, T, D)).astype(np.float32)
        cache.append(dev(k), dev(v))
        # oracle: rows past the capacity are dropped (not written)
        for b in range(B):
            T_b = max(0, min(T, cap - pos[b]))
            if T_b:
                sub = {kk: vv[b:b + 1] for kk, vv in ref.items()}
                O.kv_append_int4(sub, k[b:b + 1, :, :T_b], v[b:b + 1, :, :T_b], [pos[b]])
                for kk in ref:
                    ref[kk][b:b + 1] = sub[kk]
        pos += T
    assert np.array_equal(host(cache.lengths), pos)
    for name, t in zip(["kq", "ks", "kb", "vq", "vs", "vb"], cache.tensors()):
        got = host(t)
        if got.dtype == np.float16:
            got, exp = got.view(np.uint16), ref[name].view(np.uint16)
        else:
            exp = ref[name]
        assert np.array_equal(got, exp), name
