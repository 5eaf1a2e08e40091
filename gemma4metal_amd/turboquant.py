"""Python mirror of the reference's ``turboquant`` API for the int4-KV path.

Function names, argument order and defaults follow ``lib/turboquant.h`` of the
reference; tensors are torch tensors in GPU memory (torch is only the
device-memory / stream plumbing -- every computation runs in
``libturboquant_hip.so`` through the C ABI, see ``_lib.py``).

Like the reference's ``eval_gpu`` (``lib/turboquant.cpp:372``) these wrappers
allocate their outputs; the split-K workspace is a zero-filled buffer per
(device, stream), grown on demand and reused (the kernels leave it zeroed).
"""
from __future__ import annotations

import ctypes
import functools
from typing import Optional

import torch

from . import _lib
from ._lib import TQ_BF16, TQ_F16, TQ_F32, TQ_QUANT_MINMAX, TQ_QUANT_MLX, call

_DT = {torch.float32: TQ_F32, torch.float16: TQ_F16, torch.bfloat16: TQ_BF16}
_QUANT_DT = (torch.int32, torch.uint32)
_MODES = {"mlx": TQ_QUANT_MLX, "minmax": TQ_QUANT_MINMAX}

_workspaces: dict = {}


# Pointer and stream arguments are passed as plain ints (or None for NULL):
# the C-ABI argtypes convert them, and a decode call's fixed host cost is
# part of a short layer's time.
def _ptr(t: Optional[torch.Tensor]):
    return t.data_ptr() if t is not None else None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(stream) -> int:
    if stream is None:
        if _raw_stream is not None:
            return _raw_stream(torch.cuda.current_device())
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _need(cond: bool, msg: str):
    if not cond:
        raise ValueError(msg)


def _check_cuda(name: str, t: torch.Tensor):
    _need(isinstance(t, torch.Tensor), f"{name} must be a torch.Tensor")
    _need(t.is_cuda, f"{name} must be on a GPU device")
    _need(t.is_contiguous(), f"{name} must be contiguous")


def _sb_dtype(name: str, t: torch.Tensor) -> int:
    _need(t.dtype in (torch.float16, torch.float32), f"{name} must be float16 or float32")
    return _DT[t.dtype]


def workspace(nbytes: int, device: torch.device, stream_handle: int) -> torch.Tensor:
    """Zero-initialised split-K scratch of at least ``nbytes`` for calls on
    one (device, stream) (cached).  Calls on one stream run in order and share
    it; calls on different streams never do.  A new or grown buffer is
    allocated and zero-filled on that stream (torch's allocator then orders
    its reuse after the stream's queued work), so the fill is ordered before
    the kernels that use it, and a replaced buffer is released only behind
    the calls already queued there.  A buffer cannot be created or grown
    under graph capture (the graph would own the allocation): that raises,
    so the caller warms the capture stream up eagerly with the largest shape
    first (``torch.cuda.graph(g, stream=s)`` after a call on ``s``), or uses
    tq_sdpa_int4_noalloc."""
    dev = device.index if device.index is not None else torch.cuda.current_device()
    key = (dev, stream_handle)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        _need(not torch.cuda.is_current_stream_capturing(),
              "the split-K workspace of this (device, stream) must be created or grown, but the "
              "stream is being captured: call once eagerly on the capture stream first "
              "(torch.cuda.graph(g, stream=s)), or use tq_sdpa_int4_noalloc")
        s = torch.cuda.ExternalStream(stream_handle, device=torch.device("cuda", dev))
        with torch.cuda.stream(s):
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


# ---------------------------------------------------------------------------
# fused int4 decode attention
# ---------------------------------------------------------------------------

def sdpa_int4(queries: torch.Tensor,
              k_quant: torch.Tensor, k_scales: torch.Tensor, k_biases: torch.Tensor,
              v_quant: torch.Tensor, v_scales: torch.Tensor, v_biases: torch.Tensor,
              gqa_factor: int, scale: float = 1.0, sliding_window: int = 0, *,
              kv_len: Optional[int] = None, out: Optional[torch.Tensor] = None,
              stream=None) -> torch.Tensor:
    """``turboquant::sdpa_int4`` (reference ``lib/turboquant.h:196-207``).

    queries (num_heads, head_dim) f32|f16|bf16; k_quant/v_quant
    (num_kv_heads, N, head_dim/8) uint32 (or int32 bit patterns); scales and
    biases (num_kv_heads, N, head_dim/64) f16|f32.  ``kv_len`` (default N, as
    the reference's ``N = k_quant.shape(1)``, ``lib/turboquant.cpp:392``)
    lets a preallocated cache of capacity N hold fewer valid rows.
    Returns (num_heads, head_dim) float32.
    """
    for n, t in (("queries", queries), ("k_quant", k_quant), ("k_scales", k_scales),
                 ("k_biases", k_biases), ("v_quant", v_quant), ("v_scales", v_scales),
                 ("v_biases", v_biases)):
        _check_cuda(n, t)
    _need(queries.dim() == 2, "queries must be (num_heads, head_dim)")
    qdt = _DT.get(queries.dtype)
    _need(qdt is not None, "queries must be float32, float16 or bfloat16")
    Hq, D = queries.shape
    _need(k_quant.dim() == 3 and k_quant.dtype in _QUANT_DT, "k_quant must be (Hkv, N, D/8) uint32")
    qshape = k_quant.shape
    Hkv, cap = qshape[0], qshape[1]
    _need(qshape[2] == D // 8, f"k_quant must be ({Hkv}, {cap}, {D // 8}) uint32")
    _need(v_quant.shape == qshape and v_quant.dtype in _QUANT_DT, f"v_quant must be ({Hkv}, {cap}, {D // 8}) uint32")
    sbt = _sb_dtype("k_scales", k_scales)
    sshape = (Hkv, cap, D // 64)
    sdt = k_scales.dtype
    for n, t in (("k_scales", k_scales), ("k_biases", k_biases), ("v_scales", v_scales),
                 ("v_biases", v_biases)):
        _need(t.shape == sshape, f"{n} must be ({Hkv}, {cap}, {D // 64})")
        _need(t.dtype == sdt, "scales and biases must share one dtype")
    n = cap if kv_len is None else int(kv_len)
    if out is None:
        out = torch.empty((Hq, D), dtype=torch.float32, device=queries.device)
    else:
        _check_cuda("out", out)
        _need(out.shape == (Hq, D) and out.dtype == torch.float32, "out must be (Hq, D) float32")
    nbytes = _decode_ws_size(Hq, Hkv, D, n)
    sh = _stream(stream)
    ws = workspace(nbytes, queries.device, sh)
    call("tq_sdpa_int4", queries.data_ptr(), qdt, k_quant.data_ptr(), k_scales.data_ptr(),
         k_biases.data_ptr(), v_quant.data_ptr(), v_scales.data_ptr(), v_biases.data_ptr(), sbt,
         out.data_ptr(), Hq, Hkv, D, n, cap, int(gqa_factor), float(scale), int(sliding_window),
         ws.data_ptr(), ws.numel(), sh)
    return out


_PLAN_MODES = {"decode": 0, "ragged": 1, "prefill": 2}


def sdpa_plan(num_heads: int, num_kv_heads: int, head_dim: int, max_kv_len: int, *,
              sb_dtype: torch.dtype = torch.float16, mode: str = "decode", batch: int = 1,
              sliding_window: int = 0) -> dict:
    """The kernel a call of this shape launches and its split plan
    (``tq_sdpa_int4_plan``; no GPU work): ``{"kernel", "splits", "chunk"}``."""
    _need(sb_dtype in (torch.float16, torch.float32), "sb_dtype must be float16 or float32")
    splits, chunk = ctypes.c_int(0), ctypes.c_int(0)
    name = ctypes.create_string_buffer(64)
    call("tq_sdpa_int4_plan", _PLAN_MODES[mode], int(batch), int(num_heads), int(num_kv_heads),
         int(head_dim), int(max_kv_len), _DT[sb_dtype], int(sliding_window), ctypes.byref(splits),
         ctypes.byref(chunk), name, len(name))
    return {"kernel": name.value.decode(), "splits": splits.value, "chunk": chunk.value}


def reload_options() -> None:
    """Re-read the TQ_* kernel-choice switches from the environment (they
    are read once per process otherwise)."""
    call("tq_reload_options")
    _decode_ws_size.cache_clear()


@functools.lru_cache(maxsize=256)
def _decode_ws_size(Hq: int, Hkv: int, D: int, n: int) -> int:
    """Workspace bytes of one single-sequence decode call (a pure function
    of the shape, cached: the C query costs a call per layer otherwise)."""
    return _lib.load().tq_sdpa_int4_workspace_size(1, Hq, Hkv, D, n)


def sdpa_int4_prefill(queries: torch.Tensor,
                      k_quant: torch.Tensor, k_scales: torch.Tensor, k_biases: torch.Tensor,
                      v_quant: torch.Tensor, v_scales: torch.Tensor, v_biases: torch.Tensor,
                      n_prior: int, gqa_factor: int, scale: float = 1.0,
                      sliding_window: int = 0, *, out: Optional[torch.Tensor] = None,
                      stream=None) -> torch.Tensor:
    """Multi-query (prefill) attention of the reference's fallback path
    (``engine/gemma4_multilayer.cpp:343-364``): queries (n_new, num_heads,
    head_dim) at positions n_prior .. n_prior+n_new-1 over rows
    [0, n_prior + n_new) of the (num_kv_heads, capacity, .) caches (the new
    rows already appended); query i sees key j iff j <= n_prior + i and, with a
    window W > 0, n_prior + i - j < W.  Returns (n_new, num_heads, head_dim)
    float32."""
    for n, t in (("queries", queries), ("k_quant", k_quant), ("k_scales", k_scales),
                 ("k_biases", k_biases), ("v_quant", v_quant), ("v_scales", v_scales),
                 ("v_biases", v_biases)):
        _check_cuda(n, t)
    _need(queries.dim() == 3 and queries.dtype in _DT, "queries must be (n_new, Hq, D)")
    S, Hq, D = queries.shape
    _need(k_quant.dim() == 3 and k_quant.dtype in _QUANT_DT, "k_quant must be (Hkv, cap, D/8) uint32")
    Hkv, cap, _ = k_quant.shape
    for n, t in (("k_quant", k_quant), ("v_quant", v_quant)):
        _need(t.shape == (Hkv, cap, D // 8), f"{n} must be ({Hkv}, {cap}, {D // 8})")
    sbt = _sb_dtype("k_scales", k_scales)
    for n, t in (("k_scales", k_scales), ("k_biases", k_biases), ("v_scales", v_scales),
                 ("v_biases", v_biases)):
        _need(t.shape == (Hkv, cap, D // 64) and _DT.get(t.dtype) == sbt,
              f"{n} must be ({Hkv}, {cap}, {D // 64}) of one scale dtype")
    if out is None:
        out = torch.empty((S, Hq, D), dtype=torch.float32, device=queries.device)
    _check_cuda("out", out)
    _need(out.shape == (S, Hq, D) and out.dtype == torch.float32, "out must be (n_new, Hq, D) f32")
    nbytes = _lib.load().tq_sdpa_int4_workspace_size(max(S, 1), Hq, Hkv, D, int(n_prior) + S)
    sh = _stream(stream)
    ws = workspace(nbytes, queries.device, sh)
    call("tq_sdpa_int4_prefill", _ptr(queries), _DT[queries.dtype], _ptr(k_quant), _ptr(k_scales),
         _ptr(k_biases), _ptr(v_quant), _ptr(v_scales), _ptr(v_biases), sbt, _ptr(out), Hq, Hkv,
         D, int(n_prior), S, cap, int(gqa_factor), float(scale), int(sliding_window), _ptr(ws),
         ws.numel(), sh)
    return out


def sdpa_int4_ragged(queries: torch.Tensor,
                     k_quant: torch.Tensor, k_scales: torch.Tensor, k_biases: torch.Tensor,
                     v_quant: torch.Tensor, v_scales: torch.Tensor, v_biases: torch.Tensor,
                     seq_lens: torch.Tensor, gqa_factor: int, scale: float = 1.0,
                     sliding_window: int = 0, *, windows: Optional[torch.Tensor] = None,
                     max_kv_len: Optional[int] = None, out: Optional[torch.Tensor] = None,
                     stream=None) -> torch.Tensor:
    """Batched ragged decode.  queries (B, Hq, D); caches (B, Hkv, cap, .);
    ``seq_lens`` / ``windows`` int32 device tensors of length B.
    ``max_kv_len`` must bound every length (defaults to the capacity)."""
    _check_cuda("queries", queries)
    _need(queries.dim() == 3 and queries.dtype in _DT, "queries must be (B, Hq, D)")
    B, Hq, D = queries.shape
    _check_cuda("k_quant", k_quant)
    _need(k_quant.dim() == 4 and k_quant.shape[0] == B and k_quant.dtype in _QUANT_DT,
          "k_quant must be (B, Hkv, cap, D/8) uint32")
    _, Hkv, cap, _ = k_quant.shape
    for n, t in (("k_quant", k_quant), ("v_quant", v_quant)):
        _check_cuda(n, t)
        _need(t.shape == (B, Hkv, cap, D // 8), f"{n} must be ({B}, {Hkv}, {cap}, {D // 8})")
    sbt = _sb_dtype("k_scales", k_scales)
    for n, t in (("k_scales", k_scales), ("k_biases", k_biases), ("v_scales", v_scales),
                 ("v_biases", v_biases)):
        _check_cuda(n, t)
        _need(t.shape == (B, Hkv, cap, D // 64) and _DT.get(t.dtype) == sbt,
              f"{n} must be ({B}, {Hkv}, {cap}, {D // 64}) of one scale dtype")
    _check_cuda("seq_lens", seq_lens)
    _need(seq_lens.dtype == torch.int32 and seq_lens.numel() == B, "seq_lens must be int32 [B]")
    if windows is not None:
        _check_cuda("windows", windows)
        _need(windows.dtype == torch.int32 and windows.numel() == B, "windows must be int32 [B]")
    mx = cap if max_kv_len is None else int(max_kv_len)
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float32, device=queries.device)
    nbytes = _lib.load().tq_sdpa_int4_workspace_size(B, Hq, Hkv, D, mx)
    sh = _stream(stream)
    ws = workspace(nbytes, queries.device, sh)
    call("tq_sdpa_int4_ragged", _ptr(queries), _DT[queries.dtype], _ptr(k_quant),
         _ptr(k_scales), _ptr(k_biases), _ptr(v_quant), _ptr(v_scales), _ptr(v_biases), sbt,
         _ptr(out), B, Hq, Hkv, D, cap, _ptr(seq_lens), _ptr(windows), mx, int(gqa_factor),
         float(scale), int(sliding_window), _ptr(ws), ws.numel(), sh)
    return out


# ---------------------------------------------------------------------------
# quantize / dequantize / append
# ---------------------------------------------------------------------------

def quantize(x: torch.Tensor, group_size: int = 64, bits: int = 4, *,
             scale_dtype: Optional[torch.dtype] = None, mode: str = "mlx", stream=None):
    """MLX ``quantize(x, group_size, bits)`` over the last axis (the call at
    reference ``engine/gemma4_multilayer.cpp:228``).  Returns
    ``(w_q uint32 [..., D/8], scales [..., D/64], biases [..., D/64])``;
    scales/biases are in ``scale_dtype`` (default: x's dtype if f16/f32)."""
    _check_cuda("x", x)
    _need(x.dtype in _DT, "x must be float32, float16 or bfloat16")
    D = x.shape[-1]
    if scale_dtype is None:
        scale_dtype = x.dtype if x.dtype in (torch.float16, torch.float32) else torch.float16
    _need(scale_dtype in (torch.float16, torch.float32), "scale_dtype must be float16 or float32")
    lead = tuple(x.shape[:-1])
    rows = x.numel() // D if D else 0
    wq = torch.empty(lead + (D // 8,), dtype=torch.uint32, device=x.device)
    s = torch.empty(lead + (D // 64,), dtype=scale_dtype, device=x.device)
    b = torch.empty_like(s)
    call("tq_quantize_int4", _ptr(x), _DT[x.dtype], rows, D, group_size, bits, _MODES[mode],
         _ptr(wq), _ptr(s), _ptr(b), _DT[scale_dtype], _stream(stream))
    return wq, s, b


def dequantize(w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4, *, stream=None) -> torch.Tensor:
    """MLX ``dequantize`` (reference ``engine/gemma4_multilayer.cpp:307``):
    ``scale * nibble + bias`` as float32, shape ``[..., 8 * w_q.shape[-1]]``."""
    for n, t in (("w_q", w_q), ("scales", scales), ("biases", biases)):
        _check_cuda(n, t)
    _need(group_size == 64 and bits == 4, "only group_size=64, bits=4")
    D = w_q.shape[-1] * 8
    sbt = _sb_dtype("scales", scales)
    out = torch.empty(tuple(w_q.shape[:-1]) + (D,), dtype=torch.float32, device=w_q.device)
    rows = w_q.numel() // w_q.shape[-1] if w_q.numel() else 0
    call("tq_dequantize_int4", _ptr(w_q), _ptr(scales), _ptr(biases), sbt, rows, D, _ptr(out),
         _stream(stream))
    return out


class Int4KVCache:
    """Preallocated int4 KV cache [B, Hkv, capacity, .] with per-sequence
    lengths on the device: the in-place replacement for the reference's
    per-token ``concatenate`` (``engine/gemma4_multilayer.cpp:230-240``).

    ``ring=True`` makes it the window eviction of a sliding layer (the
    reference trims with ``slice``, ``engine/gemma4_multilayer.cpp:243-248``):
    ``lengths`` count tokens seen, token i lives in row i mod capacity, and
    attention covers the newest ``min(length, capacity)`` tokens -- exactly the
    reference window rule with window = capacity."""

    def __init__(self, batch: int, num_kv_heads: int, capacity: int, head_dim: int,
                 device, scale_dtype: torch.dtype = torch.float16, ring: bool = False):
        kw = dict(device=device)
        self.B, self.Hkv, self.cap, self.D = batch, num_kv_heads, capacity, head_dim
        self.ring = bool(ring)
        self.kq = torch.zeros((batch, num_kv_heads, capacity, head_dim // 8), dtype=torch.uint32, **kw)
        self.vq = torch.zeros_like(self.kq)
        self.ks = torch.zeros((batch, num_kv_heads, capacity, head_dim // 64), dtype=scale_dtype, **kw)
        self.kb = torch.zeros_like(self.ks)
        self.vs = torch.zeros_like(self.ks)
        self.vb = torch.zeros_like(self.ks)
        self.lengths = torch.zeros(batch, dtype=torch.int32, **kw)

    def tensors(self):
        return self.kq, self.ks, self.kb, self.vq, self.vs, self.vb

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, *, mode: str = "mlx",
               advance: bool = True, stream=None):
        """Quantize (B, Hkv, T, D) new rows into rows [len_b, len_b+T) (mod
        capacity for a ring)."""
        kv_append_int4(k_new, v_new, *self.tensors(), self.lengths, mode=mode, ring=self.ring,
                       stream=stream)
        if advance:
            self.lengths += k_new.shape[2]

    def attend(self, queries: torch.Tensor, gqa_factor: int, scale: float = 1.0,
               sliding_window: int = 0, windows: Optional[torch.Tensor] = None,
               max_kv_len: Optional[int] = None, stream=None) -> torch.Tensor:
        if self.ring:
            # the ring is the window: every stored row is attended
            _need(sliding_window == 0 and windows is None, "a ring cache takes no extra window")
            _need(max_kv_len is None or max_kv_len == self.cap, "a ring attends its capacity")
        return sdpa_int4_ragged(queries, *self.tensors(), self.lengths, gqa_factor, scale,
                                sliding_window, windows=windows, max_kv_len=max_kv_len,
                                stream=stream)


def kv_append_int4(k_new: torch.Tensor, v_new: torch.Tensor,
                   k_quant: torch.Tensor, k_scales: torch.Tensor, k_biases: torch.Tensor,
                   v_quant: torch.Tensor, v_scales: torch.Tensor, v_biases: torch.Tensor,
                   positions: torch.Tensor, *, mode: str = "mlx", ring: bool = False,
                   stream=None) -> None:
    """Quantize k_new / v_new (B, Hkv, T, D) and write them at rows
    positions[b] .. positions[b]+T-1 of the (B, Hkv, cap, .) caches (rows mod
    cap, last cap tokens only, when ``ring``)."""
    for n, t in (("k_new", k_new), ("v_new", v_new), ("k_quant", k_quant),
                 ("k_scales", k_scales), ("k_biases", k_biases), ("v_quant", v_quant),
                 ("v_scales", v_scales), ("v_biases", v_biases), ("positions", positions)):
        _check_cuda(n, t)
    _need(k_new.dim() == 4 and k_new.shape == v_new.shape and k_new.dtype == v_new.dtype,
          "k_new / v_new must both be (B, Hkv, T, D) of one dtype")
    _need(k_new.dtype in _DT, "k_new must be float32, float16 or bfloat16")
    B, Hkv, T, D = k_new.shape
    _need(k_quant.dim() == 4 and k_quant.shape[:2] == (B, Hkv) and k_quant.shape[3] == D // 8,
          "cache must be (B, Hkv, cap, D/8)")
    cap = k_quant.shape[2]
    sbt = _sb_dtype("k_scales", k_scales)
    _need(positions.dtype == torch.int32 and positions.numel() == B, "positions must be int32 [B]")
    call("tq_kv_append_int4_ring" if ring else "tq_kv_append_int4", _ptr(k_new), _ptr(v_new),
         _DT[k_new.dtype], _ptr(k_quant),
         _ptr(k_scales), _ptr(k_biases), _ptr(v_quant), _ptr(v_scales), _ptr(v_biases), sbt, B,
         Hkv, D, cap, _ptr(positions), T, _MODES[mode], _stream(stream))


def version() -> int:
    return _lib.load().tq_version()
