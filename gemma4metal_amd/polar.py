"""Python mirror of the reference's PolarQuant API (``lib/turboquant.h:52-165``)
and the 7-level PolarQuant + QJL key codec ("polar7": D = 128, level-1
angles 4-bit, levels 2-7 2-bit, a 128-bit QJL residual sketch).

Every computation runs in ``libturboquant_hip.so`` (C ABI in
``include/tq_c_api.h``); torch only holds device memory and the stream.
Function names, argument order and defaults follow the reference; its
``StreamOrDevice`` argument becomes ``stream``.  Codebooks are passed per
level, as in the reference, and concatenated into one device buffer for the
C ABI.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import TQ_F16, TQ_F32, call
from .turboquant import _check_cuda, _need, _ptr, _stream, workspace

P7_D = 128
P7_WORDS = 12
QJL_M = 128
P7_QTAB = 5136  # floats of per-head query tables (TQ_POLAR7_QTAB)


def _codebooks(cbs: Sequence[torch.Tensor]):
    """Concatenate the four per-level codebooks into one f32 device tensor and
    a host int[4] of their sizes."""
    _need(len(cbs) == 4, "four codebooks (levels 1..4) are required")
    for i, c in enumerate(cbs):
        _check_cuda(f"cb_l{i + 1}", c)
    cat = torch.cat([c.reshape(-1).to(torch.float32) for c in cbs]).contiguous()
    sizes = (ctypes.c_int * 4)(*[int(c.numel()) for c in cbs])
    return cat, sizes


def _sizes_ptr(sizes):
    return ctypes.cast(sizes, ctypes.c_void_p)


def _rows(vectors: torch.Tensor):
    _check_cuda("vectors", vectors)
    _need(vectors.dim() == 2 and vectors.dtype == torch.float32, "vectors must be (N, D) float32")
    return vectors.shape


# ---------------------------------------------------------------------------
# reference layouts (16-value blocks, 4 levels)
# ---------------------------------------------------------------------------

def polar_quantize(vectors: torch.Tensor, precondition: Optional[torch.Tensor],
                   cb_l1: torch.Tensor, cb_l2: torch.Tensor, cb_l3: torch.Tensor,
                   cb_l4: torch.Tensor, block_size: int = 16, stream=None):
    """``turboquant::polar_quantize`` (``lib/turboquant.h:52-60``): y = x P^T
    (``precondition`` None: x is already rotated), then the 4-level encode of
    every 16-value block.  Returns [idx_l1 u8 (N*nb*8), idx_l2 (N*nb*4),
    idx_l3 (N*nb*2), idx_l4 (N*nb), radii f16 (N*nb)]."""
    N, D = _rows(vectors)
    nb = D // 16
    if precondition is not None:
        _check_cuda("precondition", precondition)
    cb, sizes = _codebooks([cb_l1, cb_l2, cb_l3, cb_l4])
    dev = vectors.device
    outs = [torch.empty(N * nb * k, dtype=torch.uint8, device=dev) for k in (8, 4, 2, 1)]
    radii = torch.empty(N * nb, dtype=torch.float16, device=dev)
    call("tq_polar_quantize", _ptr(vectors), _ptr(precondition), _ptr(cb), _sizes_ptr(sizes), N, D,
         int(block_size), *[_ptr(o) for o in outs], _ptr(radii), _stream(stream))
    return outs + [radii]


def polar_quantize_packed(vectors: torch.Tensor, precondition: Optional[torch.Tensor],
                          cb_l1: torch.Tensor, cb_l2: torch.Tensor, cb_l3: torch.Tensor,
                          cb_l4: torch.Tensor, block_size: int = 16, stream=None):
    """``turboquant::polar_quantize_packed`` (``lib/turboquant.h:77-82``):
    [packed_l1 u32 (nb_total), packed_l2 u8, packed_l3 u8, packed_l4 u8,
    radii f16]."""
    N, D = _rows(vectors)
    nbt = N * (D // 16)
    if precondition is not None:
        _check_cuda("precondition", precondition)
    cb, sizes = _codebooks([cb_l1, cb_l2, cb_l3, cb_l4])
    dev = vectors.device
    p1 = torch.empty(nbt, dtype=torch.uint32, device=dev)
    p2, p3, p4 = (torch.empty(nbt, dtype=torch.uint8, device=dev) for _ in range(3))
    radii = torch.empty(nbt, dtype=torch.float16, device=dev)
    call("tq_polar_quantize_packed", _ptr(vectors), _ptr(precondition), _ptr(cb),
         _sizes_ptr(sizes), N, D, int(block_size), _ptr(p1), _ptr(p2), _ptr(p3), _ptr(p4),
         _ptr(radii), _stream(stream))
    return [p1, p2, p3, p4, radii]


def polar_dequantize(indices_l1, indices_l2, indices_l3, indices_l4, radii,
                     precondition: torch.Tensor, cb_l1, cb_l2, cb_l3, cb_l4,
                     block_size: int = 16, stream=None) -> torch.Tensor:
    """``turboquant::polar_dequantize`` (``lib/turboquant.h:62-74``):
    x = y P, D taken from ``precondition.shape[0]`` as the reference."""
    _check_cuda("precondition", precondition)
    D = precondition.shape[0]
    return _dequant_unpacked(indices_l1, indices_l2, indices_l3, indices_l4, radii, precondition,
                             (cb_l1, cb_l2, cb_l3, cb_l4), D, block_size, stream)


def polar_dequantize_fast(indices_l1, indices_l2, indices_l3, indices_l4, radii,
                          cb_l1, cb_l2, cb_l3, cb_l4, D: int, block_size: int = 16,
                          stream=None) -> torch.Tensor:
    """``turboquant::polar_dequantize_fast`` (``lib/turboquant.h:147-154``):
    y only (no preconditioner; score with P q)."""
    return _dequant_unpacked(indices_l1, indices_l2, indices_l3, indices_l4, radii, None,
                             (cb_l1, cb_l2, cb_l3, cb_l4), D, block_size, stream)


def _dequant_unpacked(i1, i2, i3, i4, radii, P, cbs, D, block_size, stream):
    for n, t in (("indices_l1", i1), ("indices_l2", i2), ("indices_l3", i3),
                 ("indices_l4", i4), ("radii", radii)):
        _check_cuda(n, t)
    _need(radii.dtype == torch.float16, "radii must be float16")
    nbt = radii.numel()
    N = nbt * 16 // D
    cb, sizes = _codebooks(list(cbs))
    out = torch.empty((N, D), dtype=torch.float32, device=radii.device)
    call("tq_polar_dequantize", _ptr(i1), _ptr(i2), _ptr(i3), _ptr(i4), _ptr(radii), _ptr(P),
         _ptr(cb), _sizes_ptr(sizes), N, D, int(block_size), _ptr(out), _stream(stream))
    return out


def polar_dequantize_packed(packed_l1, packed_l2, packed_l3, packed_l4, radii,
                            cb_l1, cb_l2, cb_l3, cb_l4, D: int, block_size: int = 16,
                            stream=None) -> torch.Tensor:
    """``turboquant::polar_dequantize_packed`` (``lib/turboquant.h:85-93``)."""
    return _dequant_packed(packed_l1, packed_l2, packed_l3, packed_l4, radii,
                           (cb_l1, cb_l2, cb_l3, cb_l4), None, D, block_size, stream)


def polar_dequantize_packed_fast(packed_l1, packed_l2, packed_l3, packed_l4, radii,
                                 cs_l1, cs_l2, cs_l3, cs_l4, D: int, block_size: int = 16,
                                 stream=None) -> torch.Tensor:
    """``turboquant::polar_dequantize_packed_fast`` (``lib/turboquant.h:95-103``):
    cs_l* are (n, 2) float32 {cos, sin} tables per codebook entry."""
    cs = [c.reshape(-1, 2) for c in (cs_l1, cs_l2, cs_l3, cs_l4)]
    return _dequant_packed(packed_l1, packed_l2, packed_l3, packed_l4, radii, None, cs, D,
                           block_size, stream)


def _dequant_packed(p1, p2, p3, p4, radii, cbs, cs, D, block_size, stream):
    for n, t in (("packed_l1", p1), ("packed_l2", p2), ("packed_l3", p3), ("packed_l4", p4),
                 ("radii", radii)):
        _check_cuda(n, t)
    nbt = radii.numel()
    N = nbt * 16 // D
    if cs is not None:
        for i, c in enumerate(cs):
            _check_cuda(f"cs_l{i + 1}", c)
        cst = torch.cat([c.reshape(-1).to(torch.float32) for c in cs]).contiguous()
        sizes = (ctypes.c_int * 4)(*[int(c.shape[0]) for c in cs])
        cb = None
    else:
        cb, sizes = _codebooks(list(cbs))
        cst = None
    out = torch.empty((N, D), dtype=torch.float32, device=radii.device)
    call("tq_polar_dequantize_packed", _ptr(p1), _ptr(p2), _ptr(p3), _ptr(p4), _ptr(radii),
         _ptr(cb), _ptr(cst), _sizes_ptr(sizes), N, D, int(block_size), _ptr(out),
         _stream(stream))
    return out


def compressed_score(queries, indices_l1, indices_l2, indices_l3, indices_l4, radii,
                     cb_l1, cb_l2, cb_l3, cb_l4, N: int, block_size: int = 16,
                     scale: float = 0.0884, *, num_kv_heads: Optional[int] = None,
                     stream=None) -> torch.Tensor:
    """``turboquant::compressed_score`` (``lib/turboquant.h:157-165``):
    (Nq, N) scores; keys of query head h are rows h*N .. h*N+N-1 (the
    reference, ``num_kv_heads`` None) or of kv head h // (Nq / num_kv_heads)."""
    _check_cuda("queries", queries)
    _need(queries.dim() == 2 and queries.dtype == torch.float32, "queries must be (Nq, D) f32")
    Nq, D = queries.shape
    Hkv = Nq if num_kv_heads is None else int(num_kv_heads)
    cb, sizes = _codebooks([cb_l1, cb_l2, cb_l3, cb_l4])
    out = torch.empty((Nq, N), dtype=torch.float32, device=queries.device)
    call("tq_compressed_score", _ptr(queries), Nq, _ptr(indices_l1), _ptr(indices_l2),
         _ptr(indices_l3), _ptr(indices_l4), _ptr(radii), _ptr(cb), _sizes_ptr(sizes), Hkv, int(N),
         D, int(block_size), float(scale), _ptr(out), _stream(stream))
    return out


def compressed_score_packed(queries, packed_l1, packed_l2, packed_l3, packed_l4, radii,
                            cb_l1, cb_l2, cb_l3, cb_l4, N: int, block_size: int = 16,
                            scale: float = 0.0884, *, num_kv_heads: Optional[int] = None,
                            stream=None) -> torch.Tensor:
    """``compressed_score`` over the packed layout."""
    _check_cuda("queries", queries)
    Nq, D = queries.shape
    Hkv = Nq if num_kv_heads is None else int(num_kv_heads)
    cb, sizes = _codebooks([cb_l1, cb_l2, cb_l3, cb_l4])
    out = torch.empty((Nq, N), dtype=torch.float32, device=queries.device)
    call("tq_compressed_score_packed", _ptr(queries), Nq, _ptr(packed_l1), _ptr(packed_l2),
         _ptr(packed_l3), _ptr(packed_l4), _ptr(radii), _ptr(cb), _sizes_ptr(sizes), Hkv, int(N),
         D, int(block_size), float(scale), _ptr(out), _stream(stream))
    return out


def compressed_sdpa(queries, indices_l1, indices_l2, indices_l3, indices_l4, radii,
                    cb_l1, cb_l2, cb_l3, cb_l4, values, block_size: int = 16,
                    scale: float = 0.0884, *, num_kv_heads: Optional[int] = None,
                    stream=None) -> torch.Tensor:
    """``turboquant::compressed_sdpa`` (``lib/turboquant.h:127-143``): softmax
    over the compressed-key scores times fp32 ``values`` (Hkv*N, D), output
    acc / (l + 1e-8)."""
    _check_cuda("queries", queries)
    _check_cuda("values", values)
    Nq, D = queries.shape
    Hkv = Nq if num_kv_heads is None else int(num_kv_heads)
    _need(values.dim() == 2 and values.shape[1] == D and values.shape[0] % Hkv == 0,
          "values must be (num_kv_heads * N, D)")
    N = values.shape[0] // Hkv
    cb, sizes = _codebooks([cb_l1, cb_l2, cb_l3, cb_l4])
    out = torch.empty((Nq, D), dtype=torch.float32, device=queries.device)
    nbytes = _lib.load().tq_compressed_sdpa_workspace_size(Nq, Hkv, D, N)
    sh = _stream(stream)
    ws = workspace(nbytes, queries.device, sh)
    call("tq_compressed_sdpa", _ptr(queries), Nq, _ptr(indices_l1), _ptr(indices_l2),
         _ptr(indices_l3), _ptr(indices_l4), _ptr(radii), _ptr(cb), _sizes_ptr(sizes),
         _ptr(values), Hkv, N, D, int(block_size), float(scale), _ptr(out), _ptr(ws), ws.numel(),
         sh)
    return out


def cos_sin_table(cb: torch.Tensor) -> torch.Tensor:
    """(n, 2) float32 {cos, sin} of each codebook angle, computed in float64
    (the tables of the ``_fast`` decoders)."""
    c = cb.detach().to(torch.float64)
    return torch.stack([torch.cos(c), torch.sin(c)], dim=-1).to(torch.float32).contiguous()


# ---------------------------------------------------------------------------
# polar7: 7-level PolarQuant + QJL over D = 128
# ---------------------------------------------------------------------------

def polar7_codebooks(device=None):
    """Uniform midpoint codebooks: level 1 (k+1/2) 2pi/16, levels 2-7
    (k+1/2) pi/8 (f32 angles), and their (cos, sin) tables."""
    cb1 = ((torch.arange(16, dtype=torch.float64) + 0.5) * (2 * math.pi / 16)).to(torch.float32)
    cb2 = ((torch.arange(4, dtype=torch.float64) + 0.5) * (math.pi / 8)).to(torch.float32)
    cb = torch.cat([cb1, cb2]).to(device)
    cs = torch.cat([cos_sin_table(cb1), cos_sin_table(cb2)]).reshape(-1).to(device)
    return cb.contiguous(), cs.contiguous()


class Polar7Codec:
    """Keys of one model layer in the polar7 layout: a D x D orthogonal
    preconditioner P, an m x D QJL sketch matrix S, the codebooks.

    Caches are ``angles`` (Hkv, cap, 12) u32, ``norms`` (Hkv, cap) u32 (fp16
    radius | fp16 ||r|| << 16), ``qjl`` (Hkv, cap, 4) u32 (optionally with a
    leading batch dimension for ``append``)."""

    def __init__(self, precondition: Optional[torch.Tensor], sketch: torch.Tensor,
                 codebooks: Optional[torch.Tensor] = None, cs_tables: Optional[torch.Tensor] = None):
        _check_cuda("sketch", sketch)
        _need(sketch.shape == (QJL_M, P7_D) and sketch.dtype == torch.float32, "sketch must be (128, 128) f32")
        if precondition is not None:
            _check_cuda("precondition", precondition)
            _need(precondition.shape == (P7_D, P7_D), "precondition must be (128, 128)")
        self.P, self.S = precondition, sketch
        if codebooks is None:
            codebooks, cs_tables = polar7_codebooks(sketch.device)
        self.cb, self.cs = codebooks.contiguous(), cs_tables.contiguous()
        # S P, so the query sketch S (P q) is one product of q
        self.SP = torch.empty_like(sketch)
        call("tq_polar7_sketch_precondition", _ptr(self.P), _ptr(self.S), _ptr(self.SP), _stream(None))
        torch.cuda.current_stream().synchronize()

    def new_cache(self, num_kv_heads: int, capacity: int, batch: Optional[int] = None):
        lead = (num_kv_heads, capacity) if batch is None else (batch, num_kv_heads, capacity)
        dev = self.S.device
        return (torch.zeros(lead + (P7_WORDS,), dtype=torch.uint32, device=dev),
                torch.zeros(lead, dtype=torch.uint32, device=dev),
                torch.zeros(lead + (4,), dtype=torch.uint32, device=dev))

    def encode(self, x: torch.Tensor, stream=None):
        """x (..., 128) f32 -> (angles (..., 12), norms (...), qjl (..., 4))."""
        _check_cuda("x", x)
        _need(x.shape[-1] == P7_D and x.dtype == torch.float32, "x must be (..., 128) f32")
        lead = tuple(x.shape[:-1])
        n = x.numel() // P7_D
        angles, norms, qjl = (torch.empty(lead + s, dtype=torch.uint32, device=x.device)
                              for s in ((P7_WORDS,), (), (4,)))
        call("tq_polar7_encode", _ptr(x), _ptr(self.P), _ptr(self.S), _ptr(self.cb), _ptr(self.cs),
             n, _ptr(angles), _ptr(norms), _ptr(qjl), _stream(stream))
        return angles, norms, qjl

    def append(self, k_new: torch.Tensor, angles, norms, qjl, positions: torch.Tensor,
               stream=None) -> None:
        """Encode k_new (B, Hkv, T, 128) into rows positions[b] .. +T-1 of
        (B, Hkv, cap, .) caches."""
        _check_cuda("k_new", k_new)
        _check_cuda("positions", positions)
        _need(k_new.dim() == 4 and k_new.shape[3] == P7_D, "k_new must be (B, Hkv, T, 128)")
        B, Hkv, T, _ = k_new.shape
        cap = angles.shape[2]
        call("tq_polar7_kv_append", _ptr(k_new), _ptr(self.P), _ptr(self.S), _ptr(self.cb),
             _ptr(self.cs), _ptr(angles), _ptr(norms), _ptr(qjl), B, Hkv, cap, _ptr(positions), T,
             _stream(stream))

    def prepare_query(self, q: torch.Tensor, *, with_vectors: bool = False, stream=None):
        """Query side of a decode step for q (Hq, 128) f32: the per-head
        tables the score kernels read ((Hq, TQ_POLAR7_QTAB) f32).  With
        ``with_vectors`` also returns q' = P q and S q' ((Hq, 128) each)."""
        _check_cuda("q", q)
        _need(q.dim() == 2 and q.shape[1] == P7_D and q.dtype == torch.float32, "q must be (Hq, 128) f32")
        Hq = q.shape[0]
        tab = torch.empty((Hq, P7_QTAB), dtype=torch.float32, device=q.device)
        qp = torch.empty_like(q) if with_vectors else None
        qs = torch.empty_like(q) if with_vectors else None
        call("tq_polar7_prepare_query_sp", _ptr(q), _ptr(self.P), _ptr(self.SP), _ptr(self.cs), Hq,
             _ptr(tab), _ptr(qp), _ptr(qs), _stream(stream))
        return (tab, qp, qs) if with_vectors else tab

    def score(self, q_tables, angles, norms, qjl, scale: float = 1.0, *,
              kv_len: Optional[int] = None, stream=None) -> torch.Tensor:
        """(Hq, kv_len) scores of the keys in the caches (Hkv, cap, .)."""
        Hq = q_tables.shape[0]
        Hkv, cap = angles.shape[0], angles.shape[1]
        n = cap if kv_len is None else int(kv_len)
        out = torch.empty((Hq, n), dtype=torch.float32, device=q_tables.device)
        call("tq_polar7_score", _ptr(q_tables), _ptr(angles), _ptr(norms), _ptr(qjl),
             _ptr(self.cs), Hq, Hkv, n, cap, float(scale), _ptr(out), _stream(stream))
        return out

    def score_q(self, q: torch.Tensor, angles, norms, qjl, scale: float = 1.0, *,
                kv_len: Optional[int] = None, stream=None) -> torch.Tensor:
        """``score`` straight from the query q (Hq, 128) f32: every workgroup
        builds its heads' query tables itself (one launch, no
        ``prepare_query``)."""
        _check_cuda("q", q)
        _need(q.dim() == 2 and q.shape[1] == P7_D and q.dtype == torch.float32 and q.is_contiguous(),
              "q must be contiguous (Hq, 128) f32")
        Hq = q.shape[0]
        Hkv, cap = angles.shape[0], angles.shape[1]
        n = cap if kv_len is None else int(kv_len)
        out = torch.empty((Hq, n), dtype=torch.float32, device=q.device)
        call("tq_polar7_score_q", _ptr(q), _ptr(self.P), _ptr(self.SP), _ptr(self.cs), _ptr(angles),
             _ptr(norms), _ptr(qjl), Hq, Hkv, n, cap, float(scale), _ptr(out), _stream(stream))
        return out

    def sdpa_int4v(self, q_tables, angles, norms, qjl, v_quant, v_scales, v_biases,
                   scale: float = 1.0, sliding_window: int = 0, *, kv_len: Optional[int] = None,
                   out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """Decode attention over the compressed keys with int4 V
        (Hkv, cap, 16) and scale/bias (Hkv, cap, 2); returns (Hq, 128) f32."""
        Hq = q_tables.shape[0]
        Hkv, cap = angles.shape[0], angles.shape[1]
        _check_cuda("v_quant", v_quant)
        _need(v_quant.shape == (Hkv, cap, P7_D // 8), "v_quant must be (Hkv, cap, 16)")
        _need(v_scales.dtype in (torch.float16, torch.float32), "v_scales must be f16 or f32")
        sbt = TQ_F16 if v_scales.dtype == torch.float16 else TQ_F32
        n = cap if kv_len is None else int(kv_len)
        if out is None:
            out = torch.empty((Hq, P7_D), dtype=torch.float32, device=q_tables.device)
        nbytes = _lib.load().tq_polar7_sdpa_workspace_size(Hq, Hkv, n)
        sh = _stream(stream)
        ws = workspace(nbytes, q_tables.device, sh)
        call("tq_polar7_sdpa_int4v", _ptr(q_tables), _ptr(angles), _ptr(norms), _ptr(qjl),
             _ptr(self.cs), _ptr(v_quant), _ptr(v_scales), _ptr(v_biases), sbt, _ptr(out), Hq, Hkv,
             n, cap, float(scale), int(sliding_window), _ptr(ws), ws.numel(), sh)
        return out

    def sdpa_int4v_q(self, q: torch.Tensor, angles, norms, qjl, v_quant, v_scales, v_biases,
                     scale: float = 1.0, sliding_window: int = 0, *, kv_len: Optional[int] = None,
                     out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """``sdpa_int4v`` straight from the query q (Hq, 128) f32: every
        workgroup builds its heads' query tables itself, so a decode step is
        one launch (no ``prepare_query``).  Returns (Hq, 128) f32."""
        _check_cuda("q", q)
        _need(q.dim() == 2 and q.shape[1] == P7_D and q.dtype == torch.float32 and q.is_contiguous(),
              "q must be contiguous (Hq, 128) f32")
        Hq = q.shape[0]
        Hkv, cap = angles.shape[0], angles.shape[1]
        _check_cuda("v_quant", v_quant)
        _need(v_quant.shape == (Hkv, cap, P7_D // 8), "v_quant must be (Hkv, cap, 16)")
        _need(v_scales.dtype in (torch.float16, torch.float32), "v_scales must be f16 or f32")
        sbt = TQ_F16 if v_scales.dtype == torch.float16 else TQ_F32
        n = cap if kv_len is None else int(kv_len)
        if out is None:
            out = torch.empty((Hq, P7_D), dtype=torch.float32, device=q.device)
        nbytes = _lib.load().tq_polar7_sdpa_workspace_size(Hq, Hkv, n)
        sh = _stream(stream)
        ws = workspace(nbytes, q.device, sh)
        call("tq_polar7_sdpa_int4v_q", _ptr(q), _ptr(self.P), _ptr(self.SP), _ptr(self.cs),
             _ptr(angles), _ptr(norms), _ptr(qjl), _ptr(v_quant), _ptr(v_scales), _ptr(v_biases),
             sbt, _ptr(out), Hq, Hkv, n, cap, float(scale), int(sliding_window), _ptr(ws),
             ws.numel(), sh)
        return out
