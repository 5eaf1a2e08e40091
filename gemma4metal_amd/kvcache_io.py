"""Int4 KV-cache save / load in the reference engine's prompt-cache format.

The reference writes one safetensors file (``engine/gemma4_multilayer.cpp:
113-129``, read back at ``:131-144``):

* ``cache_offset`` -- int32 [1], the number of positions the cache covers;
* per layer L that has a cache: ``lL.kq``, ``lL.ks``, ``lL.kb``, ``lL.vq``,
  ``lL.vs``, ``lL.vb`` -- uint32 (1, nkv, N, D/8) nibbles and (1, nkv, N, D/64)
  scales / biases, rows oldest first.  N may be smaller than cache_offset
  where the engine trimmed the cache to its window (``:243-248``).

``save_kv_cache`` / ``load_kv_cache`` move such files to and from
``Int4KVCache`` objects (batch 1).  A ring cache is written oldest first and
read back into the ring slots of the same absolute positions, so a file
saved from a ring loads into a linear cache and the other way round.

The safetensors container (8-byte little-endian header length, a JSON header
of ``{name: {dtype, shape, data_offsets}}``, then the raw little-endian
tensor bytes) is written and parsed here directly.
"""
from __future__ import annotations

import json
import struct
from typing import Dict, Optional, Sequence

import numpy as np
import torch

from .turboquant import Int4KVCache

_ARRAYS = ("kq", "ks", "kb", "vq", "vs", "vb")
_NP_OF = {"U32": np.uint32, "I32": np.int32, "F32": np.float32, "F16": np.float16,
          "U16": np.uint16, "BF16": np.uint16, "U8": np.uint8, "I64": np.int64}
_TAG_OF_TORCH = {torch.uint32: "U32", torch.int32: "I32", torch.float32: "F32",
                 torch.float16: "F16", torch.bfloat16: "BF16"}


def write_safetensors(path: str, tensors: Dict[str, np.ndarray],
                      dtags: Optional[Dict[str, str]] = None,
                      metadata: Optional[Dict[str, str]] = None) -> None:
    """Write numpy arrays as one safetensors file.  ``dtags`` overrides the
    dtype tag of a tensor (BF16 data travels as uint16)."""
    dtags = dtags or {}
    header: Dict[str, object] = {}
    if metadata:
        header["__metadata__"] = dict(metadata)
    off = 0
    blobs = []
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        tag = dtags.get(name)
        if tag is None:
            tag = next(t for t, d in _NP_OF.items() if t != "BF16" and np.dtype(d) == a.dtype)
        raw = a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": tag, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * (-len(text) % 8)  # data starts 8-byte aligned
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)


def read_safetensors(path: str):
    """Return ({name: numpy array}, {name: dtype tag}, metadata).  BF16
    tensors come back as their uint16 bit patterns."""
    with open(path, "rb") as f:
        data = f.read()
    if len(data) < 8:
        raise ValueError(f"{path}: not a safetensors file")
    (n,) = struct.unpack("<Q", data[:8])
    if n > len(data) - 8:
        raise ValueError(f"{path}: header length {n} exceeds the file")
    header = json.loads(data[8:8 + n].decode())
    meta = header.pop("__metadata__", {}) or {}
    base = 8 + n
    out, tags = {}, {}
    for name, spec in header.items():
        tag = spec["dtype"]
        if tag not in _NP_OF:
            raise ValueError(f"{path}: tensor {name} has unsupported dtype {tag}")
        b0, b1 = spec["data_offsets"]
        dt = np.dtype(_NP_OF[tag]).newbyteorder("<")
        count = int(np.prod(spec["shape"])) if spec["shape"] else 1
        if b1 - b0 != count * dt.itemsize or base + b1 > len(data):
            raise ValueError(f"{path}: tensor {name} has inconsistent offsets")
        out[name] = np.frombuffer(data, dtype=dt, count=count, offset=base + b0).reshape(
            spec["shape"]).astype(dt.newbyteorder("="))
        tags[name] = tag
    return out, tags, meta


def _host(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.uint32:
        return t.view(torch.int32).cpu().numpy().view(np.uint32)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def _chronological_rows(cache: Int4KVCache, n: int) -> np.ndarray:
    """Rows of the tokens a batch-1 cache holds, oldest first."""
    if not cache.ring:
        if n > cache.cap:
            raise ValueError(f"length {n} exceeds capacity {cache.cap}")
        return np.arange(n)
    kept = min(n, cache.cap)
    return (np.arange(n - kept, n) % cache.cap).astype(np.int64)


def save_kv_cache(path: str, layers: Sequence[Optional[Int4KVCache]], cache_offset: int) -> None:
    """Write the caches of ``layers`` (index = layer; None = no cache) and
    ``cache_offset`` in the reference format."""
    tensors: Dict[str, np.ndarray] = {"cache_offset": np.array([cache_offset], np.int32)}
    tags: Dict[str, str] = {"cache_offset": "I32"}
    for li, cache in enumerate(layers):
        if cache is None:
            continue
        if cache.B != 1:
            raise ValueError("the prompt-cache format holds batch-1 caches")
        n = int(_host(cache.lengths)[0])
        rows = _chronological_rows(cache, n)
        for name, t in zip(_ARRAYS, cache.tensors()):
            a = _host(t)[:, :, rows, :]
            tensors[f"l{li}.{name}"] = a
            tags[f"l{li}.{name}"] = _TAG_OF_TORCH[t.dtype]
    write_safetensors(path, tensors, tags, metadata={"format": "mlx"})


def load_kv_cache(path: str, layers: Sequence[Optional[Int4KVCache]]) -> int:
    """Fill the caches of ``layers`` from a prompt-cache file and return its
    ``cache_offset``.  A layer whose cache is None, or that the file does not
    hold, is left untouched.  A linear cache takes the file's N rows at
    rows 0..N-1 (length N); a ring takes the newest min(N, capacity) of them
    at the slots of their absolute positions cache_offset - N + j (length
    max(cache_offset, N))."""
    data, tags, _ = read_safetensors(path)
    if "cache_offset" not in data:
        raise ValueError(f"{path}: no cache_offset")
    offset = int(data["cache_offset"].reshape(-1)[0])
    for li, cache in enumerate(layers):
        if cache is None or f"l{li}.kq" not in data:
            continue
        if cache.B != 1:
            raise ValueError("the prompt-cache format holds batch-1 caches")
        arrs = [data[f"l{li}.{name}"] for name in _ARRAYS]
        n = arrs[0].shape[2]
        for name, a, t in zip(_ARRAYS, arrs, cache.tensors()):
            want = (1, cache.Hkv, n, t.shape[3])
            if a.shape != want:
                raise ValueError(f"layer {li} {name}: shape {a.shape}, cache needs {want}")
            if tags[f"l{li}.{name}"] != _TAG_OF_TORCH[t.dtype]:
                raise ValueError(f"layer {li} {name}: dtype {tags[f'l{li}.{name}']}, cache holds "
                                 f"{_TAG_OF_TORCH[t.dtype]}")
        if cache.ring:
            total = max(offset, n)
            keep = min(n, cache.cap)
            src = np.arange(n - keep, n)
            dst = (total - n + src) % cache.cap
            length = total
        else:
            if n > cache.cap:
                raise ValueError(f"layer {li}: {n} rows exceed capacity {cache.cap}")
            src = dst = np.arange(n)
            length = n
        for a, t in zip(arrs, cache.tensors()):
            host = _host(t)
            host[0][:, dst, :] = a[0][:, src, :]
            if t.dtype == torch.uint32:
                t.view(torch.int32).copy_(torch.from_numpy(host.view(np.int32)))
            elif t.dtype == torch.bfloat16:
                t.view(torch.int16).copy_(torch.from_numpy(host.view(np.int16)))
            else:
                t.copy_(torch.from_numpy(host))
        cache.lengths.fill_(length)
    return offset
