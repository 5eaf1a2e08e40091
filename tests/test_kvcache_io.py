"""CPU: prompt-cache files in the reference engine's safetensors layout
(engine/gemma4_multilayer.cpp:113-144) to and from Int4KVCache, linear and
ring.  The container format is checked against the safetensors library in
both directions."""
import numpy as np
import pytest
import torch
from safetensors.numpy import load_file, save_file

from gemma4metal_amd import kvcache_io as IO
from gemma4metal_amd.turboquant import Int4KVCache


def fill_random(cache, rng):
    for t in cache.tensors():
        if t.dtype == torch.uint32:
            a = rng.integers(0, 2**32, size=t.shape, dtype=np.uint64).astype(np.uint32)
            t.view(torch.int32).copy_(torch.from_numpy(a.view(np.int32)))
        else:
            t.copy_(torch.from_numpy(rng.standard_normal(t.shape).astype(np.float16)))


def host(t):
    return IO._host(t)


def test_writer_is_read_by_the_safetensors_library(tmp_path):
    rng = np.random.default_rng(0)
    arrays = {"cache_offset": np.array([7], np.int32),
              "l0.kq": rng.integers(0, 2**32, (1, 2, 5, 16), dtype=np.uint64).astype(np.uint32),
              "l0.ks": rng.standard_normal((1, 2, 5, 2)).astype(np.float16),
              "x": rng.standard_normal((3,)).astype(np.float32)}
    p = str(tmp_path / "a.safetensors")
    IO.write_safetensors(p, arrays, metadata={"format": "mlx"})
    back = load_file(p)
    assert set(back) == set(arrays)
    for k, v in arrays.items():
        assert back[k].dtype == v.dtype and np.array_equal(back[k], v)


def test_reader_reads_the_safetensors_library(tmp_path):
    rng = np.random.default_rng(1)
    arrays = {"cache_offset": np.array([3], np.int32),
              "l3.vq": rng.integers(0, 2**32, (1, 1, 3, 32), dtype=np.uint64).astype(np.uint32),
              "l3.vb": rng.standard_normal((1, 1, 3, 4)).astype(np.float32)}
    p = str(tmp_path / "b.safetensors")
    save_file(arrays, p, metadata={"format": "mlx"})
    back, tags, meta = IO.read_safetensors(p)
    assert meta == {"format": "mlx"}
    assert tags == {"cache_offset": "I32", "l3.vq": "U32", "l3.vb": "F32"}
    for k, v in arrays.items():
        assert np.array_equal(back[k], v)


def reference_style_file(path, rng, offset, layers):
    """A file laid out as the engine writes it: layers {L: N}."""
    arrays = {"cache_offset": np.array([offset], np.int32)}
    for L, n in layers.items():
        for name in ("kq", "vq"):
            arrays[f"l{L}.{name}"] = rng.integers(0, 2**32, (1, 2, n, 16),
                                                  dtype=np.uint64).astype(np.uint32)
        for name in ("ks", "kb", "vs", "vb"):
            arrays[f"l{L}.{name}"] = rng.standard_normal((1, 2, n, 2)).astype(np.float16)
    save_file(arrays, path)
    return arrays


def test_load_reference_layout_into_linear_and_ring(tmp_path):
    rng = np.random.default_rng(2)
    p = str(tmp_path / "ref.safetensors")
    # global layer 0 holds all 12 positions, sliding layer 1 was trimmed to 5
    arrays = reference_style_file(p, rng, 12, {0: 12, 1: 5})
    lin = Int4KVCache(1, 2, 16, 128, "cpu")
    ring = Int4KVCache(1, 2, 4, 128, "cpu", ring=True)
    assert IO.load_kv_cache(p, [lin, ring]) == 12
    assert int(lin.lengths[0]) == 12 and int(ring.lengths[0]) == 12
    assert np.array_equal(host(lin.kq)[:, :, :12], arrays["l0.kq"])
    # the ring keeps positions 8..11 (the newest 4 of the trimmed 7..11) at
    # slots position % 4
    for pos in range(8, 12):
        j = pos - 7  # row of the file (it starts at position 12 - 5)
        assert np.array_equal(host(ring.kq)[0, :, pos % 4], arrays["l1.kq"][0, :, j])
        assert np.array_equal(host(ring.vb)[0, :, pos % 4], arrays["l1.vb"][0, :, j])


@pytest.mark.parametrize("ring,cap,n", [(False, 10, 7), (True, 6, 6), (True, 6, 17), (True, 6, 3)])
def test_round_trip(tmp_path, ring, cap, n):
    rng = np.random.default_rng(cap + n)
    src = Int4KVCache(1, 2, cap, 128, "cpu", ring=ring)
    fill_random(src, rng)
    src.lengths.fill_(n)
    p = str(tmp_path / "c.safetensors")
    IO.save_kv_cache(p, [None, src], cache_offset=n)
    data, tags, _ = IO.read_safetensors(p)
    assert "l0.kq" not in data and tags["l1.kq"] == "U32" and tags["l1.ks"] == "F16"
    kept = min(n, cap)
    order = (np.arange(n - kept, n) % cap) if ring else np.arange(n)
    assert np.array_equal(data["l1.kq"], host(src.kq)[:, :, order])   # oldest first
    dst = Int4KVCache(1, 2, cap, 128, "cpu", ring=ring)
    assert IO.load_kv_cache(p, [None, dst]) == n
    assert int(dst.lengths[0]) == n
    for a, b in zip(src.tensors(), dst.tensors()):
        assert np.array_equal(host(a)[:, :, order], host(b)[:, :, order])
    # a ring file also loads into a linear cache, oldest first
    lin = Int4KVCache(1, 2, cap + n, 128, "cpu")
    IO.load_kv_cache(p, [None, lin])
    assert int(lin.lengths[0]) == kept
    assert np.array_equal(host(lin.vq)[:, :, :kept], host(src.vq)[:, :, order])


def test_load_rejects_mismatches(tmp_path):
    rng = np.random.default_rng(3)
    p = str(tmp_path / "d.safetensors")
    reference_style_file(p, rng, 4, {0: 4})
    with pytest.raises(ValueError, match="shape"):
        IO.load_kv_cache(p, [Int4KVCache(1, 3, 8, 128, "cpu")])       # wrong kv heads
    with pytest.raises(ValueError, match="dtype"):
        IO.load_kv_cache(p, [Int4KVCache(1, 2, 8, 128, "cpu", scale_dtype=torch.float32)])
    with pytest.raises(ValueError, match="capacity"):
        IO.load_kv_cache(p, [Int4KVCache(1, 2, 3, 128, "cpu")])        # linear too small
    with pytest.raises(ValueError, match="batch-1"):
        IO.save_kv_cache(p, [Int4KVCache(2, 2, 3, 128, "cpu")], 0)
    bad = str(tmp_path / "e.safetensors")
    open(bad, "wb").write(b"\x10\x00\x00\x00\x00\x00\x00\x00{}")
    with pytest.raises(ValueError):
        IO.read_safetensors(bad)
