"""NumPy restatement of the reference's int4-KV decode-attention algorithm.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): this module is the
checker the HIP path is compared against.  It is never imported by
``gemma4metal_amd``.

What it restates, with the reference location each function follows:

* ``mlx_affine_quantize`` -- MLX's affine ``quantize(x, 64, 4)`` as called at
  ``engine/gemma4_multilayer.cpp:228-229`` and ``tests/test_sdpa_int4.cpp:25-26``.
  MLX is a third-party dependency that the reference clones at an unpinned
  HEAD (``CMakeLists.txt:7-14``, ``README.md:90``) and that is not installed
  here; the rule restated is the published CPU kernel of MLX's affine
  quantizer (min/max per group, zero-point-exact edge, ``std::rint``, IEEE
  fp32 division).  Pinned by the hand-derived known answers in
  ``tests/test_oracle_quant.py``.
* ``dequantize`` -- ``value = scale * nibble + bias`` with 8 nibbles per
  uint32, element i at bits [4i, 4i+4) (``lib/turboquant.metal:718-720``).
* ``sdpa_int4`` -- the math of ``sdpa_int4_vector`` (``lib/turboquant.metal:723-889``):
  q-head h reads kv-head ``h // gqa`` (``:745``), scores are ``scale * q.k``
  (``:762``), key ``ki`` is skipped when ``W > 0 and N-1-ki >= W`` (``:779``),
  and an all-zero softmax denominator yields 0 (``:886``).  Computed in
  float64 from the dequantized K/V, i.e. the reference oracle composition
  ``dequantize`` + ``scaled_dot_product_attention`` of
  ``tests/test_sdpa_int4.cpp:31-42``.
"""
from __future__ import annotations

import numpy as np

GROUP_SIZE = 64
BITS = 4
N_BINS = (1 << BITS) - 1
EPS = np.float32(1e-7)


# --------------------------------------------------------------------------
# dtype helpers (bf16 has no numpy dtype: carried as uint16 bit patterns)
# --------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16, returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rms_norm(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Weightless RMS norm over the last axis, as ``bare_rms_norm``
    (``engine/gemma4_multilayer.cpp:39-41``): ``x * rsqrt(mean(x^2) + eps)``."""
    x = np.asarray(x, dtype=np.float32)
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    return (x / np.sqrt(ms + eps)).astype(np.float32)


# --------------------------------------------------------------------------
# quantize / dequantize
# --------------------------------------------------------------------------

def mlx_affine_quantize(x: np.ndarray, group_size: int = GROUP_SIZE, bits: int = BITS):
    """MLX affine quantization of the last axis, all arithmetic in float32.

    Per group of ``group_size`` values::

        mx, mn = max, min
        scale  = max((mx - mn) / n_bins, 1e-7)
        side   = |mn| > |mx|
        scale  = side ? scale : -scale
        edge   = side ? mn : mx
        q0     = rint(edge / scale)
        if q0 != 0: scale = edge / q0; bias = edge   else: bias = 0
        q      = clamp(rint((x - bias) / scale), 0, n_bins)

    Returns ``(wq uint32 [..., D*bits/32], scales f32 [..., D/gs], biases f32)``.
    """
    assert bits == 4, "only 4-bit packing is on the path"
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    assert D % group_size == 0
    lead = x.shape[:-1]
    g = x.reshape(-1, D // group_size, group_size)
    n_bins = np.float32((1 << bits) - 1)
    mx = g.max(axis=-1)
    mn = g.min(axis=-1)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.maximum((mx - mn) / n_bins, EPS).astype(np.float32)
        side = np.abs(mn) > np.abs(mx)
        scale = np.where(side, scale, -scale).astype(np.float32)
        edge = np.where(side, mn, mx).astype(np.float32)
        q0 = np.rint(edge / scale).astype(np.float32)
        nz = q0 != 0
        scale = np.where(nz, edge / np.where(nz, q0, np.float32(1)), scale).astype(np.float32)
        bias = np.where(nz, edge, np.float32(0)).astype(np.float32)
        q = np.rint((g - bias[..., None]) / scale[..., None]).astype(np.float32)
    q = np.clip(q, 0, n_bins).astype(np.uint32)
    q = q.reshape(-1, D // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    wq = np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)
    return (wq.reshape(*lead, D // 8),
            scale.reshape(*lead, D // group_size),
            bias.reshape(*lead, D // group_size))


def minmax_affine_quantize(x: np.ndarray, group_size: int = GROUP_SIZE, bits: int = BITS):
    """Secondary mode: the literal textbook rule ``scale = (max-min)/15``,
    ``bias = min``, ``q = clamp(rint((x-bias)/scale), 0, 15)`` in float32
    (``scale`` floored at 1e-7 so a constant group stays finite)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    lead = x.shape[:-1]
    g = x.reshape(-1, D // group_size, group_size)
    n_bins = np.float32((1 << bits) - 1)
    mx = g.max(axis=-1)
    mn = g.min(axis=-1)
    scale = np.maximum((mx - mn) / n_bins, EPS).astype(np.float32)
    bias = mn.astype(np.float32)
    q = np.rint((g - bias[..., None]) / scale[..., None]).astype(np.float32)
    q = np.clip(q, 0, n_bins).astype(np.uint32).reshape(-1, D // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    wq = np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)
    return (wq.reshape(*lead, D // 8),
            scale.reshape(*lead, D // group_size),
            bias.reshape(*lead, D // group_size))


def quantize_int4(x: np.ndarray, sb_dtype: str = "f16", mode: str = "mlx"):
    """Quantize rows of ``x`` to the MLX int4 layout, then store scale/bias in
    ``sb_dtype`` ("f32" as the reference's ``lib/turboquant.h:199`` or "f16"
    as the benchmark's layout) by a round-to-nearest-even cast of the float32
    values the nibbles were computed with (MLX ``quantize`` then ``astype``)."""
    fn = mlx_affine_quantize if mode == "mlx" else minmax_affine_quantize
    wq, s, b = fn(x)
    if sb_dtype == "f16":
        return wq, s.astype(np.float16), b.astype(np.float16)
    if sb_dtype == "f32":
        return wq, s, b
    raise ValueError(sb_dtype)


def unpack_nibbles(wq: np.ndarray) -> np.ndarray:
    wq = np.asarray(wq, dtype=np.uint32)
    shifts = (np.arange(8, dtype=np.uint32) * 4)
    n = (wq[..., None] >> shifts) & 0xF
    return n.reshape(*wq.shape[:-1], wq.shape[-1] * 8)


def dequantize(wq, scales, biases, group_size: int = GROUP_SIZE, dtype=np.float64):
    """``scale * nibble + bias`` per group (``lib/turboquant.metal:719``)."""
    n = unpack_nibbles(wq).astype(dtype)
    D = n.shape[-1]
    s = np.repeat(np.asarray(scales).astype(dtype), group_size, axis=-1)
    b = np.repeat(np.asarray(biases).astype(dtype), group_size, axis=-1)
    assert s.shape[-1] == D
    return s * n + b


# --------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------

def attended_range(n: int, window: int):
    """Keys [lo, n) survive the reference window rule: key ``ki`` is skipped
    iff ``window > 0 and n - 1 - ki >= window`` (``lib/turboquant.metal:779``)."""
    lo = max(0, n - window) if window > 0 else 0
    return lo, n


def softmax_attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """float64 softmax(scale * q k^T) v for one query row; empty -> zeros."""
    if k.shape[0] == 0:
        return np.zeros(v.shape[-1], dtype=np.float64)
    s = (k @ q) * scale
    m = s.max()
    p = np.exp(s - m)
    den = p.sum()
    return (p @ v) / den if den != 0 else np.zeros(v.shape[-1])


def sdpa_int4(q, kq, ks, kb, vq, vs, vb, gqa_factor: int, scale: float = 1.0,
              sliding_window: int = 0, kv_len: int | None = None) -> np.ndarray:
    """Reference ``sdpa_int4`` (``lib/turboquant.h:196-207``) in float64.

    q: (Hq, D) float values (already rounded to the input dtype);
    kq/vq: (Hkv, cap, D/8) uint32; ks/kb/vs/vb: (Hkv, cap, D/64);
    ``kv_len`` defaults to ``cap`` (the reference's ``N = k_quant.shape(1)``,
    ``lib/turboquant.cpp:392``).  Returns (Hq, D) float64.
    """
    q = np.asarray(q, dtype=np.float64)
    scale = float(np.float32(scale))  # the reference's `float scale` (lib/turboquant.h:206)
    Hq, D = q.shape
    n = kq.shape[1] if kv_len is None else kv_len
    lo, hi = attended_range(n, sliding_window)
    out = np.zeros((Hq, D), dtype=np.float64)
    for kvh in range(kq.shape[0]):
        heads = [h for h in range(Hq) if h // gqa_factor == kvh]
        if not heads:
            continue
        K = dequantize(kq[kvh, lo:hi], ks[kvh, lo:hi], kb[kvh, lo:hi])
        V = dequantize(vq[kvh, lo:hi], vs[kvh, lo:hi], vb[kvh, lo:hi])
        for h in heads:
            out[h] = softmax_attend(q[h], K, V, scale)
    return out


def sdpa_int4_ragged(q, kq, ks, kb, vq, vs, vb, seq_lens, windows, gqa_factor: int,
                     scale: float = 1.0) -> np.ndarray:
    """Batched ragged decode: sequence b attends to its first ``seq_lens[b]``
    cached rows under its own window ``windows[b]``.  q: (B, Hq, D);
    caches: (B, Hkv, cap, .).  Returns (B, Hq, D) float64."""
    B = q.shape[0]
    return np.stack([
        sdpa_int4(q[b], kq[b], ks[b], kb[b], vq[b], vs[b], vb[b], gqa_factor, scale,
                  int(windows[b]), kv_len=int(seq_lens[b]))
        for b in range(B)])


def sdpa_int4_prefill(q, kq, ks, kb, vq, vs, vb, n_prior: int, gqa_factor: int,
                      scale: float = 1.0, sliding_window: int = 0) -> np.ndarray:
    """The engine's prefill fallback (``engine/gemma4_multilayer.cpp:
    343-364``) in float64: dequantize the cache (``:307-308``), build the
    additive mask md[i, j] = -1e9 where key j is in the future of query i
    (j > n_prior + i) or, with a window, outside it (n_prior + i - j >= W)
    (``:349-358``), then softmax(scale * q K^T + md) V per head with the kv
    head h // gqa (MLX's GQA broadcast).

    q: (n_new, Hq, D); caches (Hkv, cap, .) holding rows [0, n_prior+n_new).
    Returns (n_new, Hq, D) float64."""
    q = np.asarray(q, dtype=np.float64)
    scale = float(np.float32(scale))
    S, Hq, D = q.shape
    L = n_prior + S
    qpos = n_prior + np.arange(S)[:, None]
    j = np.arange(L)[None, :]
    masked = j > qpos
    if sliding_window > 0:
        masked |= (qpos - j) >= sliding_window
    md = np.where(masked, -1e9, 0.0)
    out = np.zeros((S, Hq, D), dtype=np.float64)
    for kvh in range(kq.shape[0]):
        K = dequantize(kq[kvh, :L], ks[kvh, :L], kb[kvh, :L])
        V = dequantize(vq[kvh, :L], vs[kvh, :L], vb[kvh, :L])
        for h in range(kvh * gqa_factor, (kvh + 1) * gqa_factor):
            z = scale * (q[:, h, :] @ K.T) + md
            z -= z.max(axis=1, keepdims=True)
            w = np.exp(z)
            out[:, h, :] = (w @ V) / w.sum(axis=1, keepdims=True)
    return out


def kv_append_int4(cache: dict, k_new: np.ndarray, v_new: np.ndarray, positions,
                   sb_dtype: str = "f16", mode: str = "mlx") -> None:
    """Quantize ``k_new``/``v_new`` (B, Hkv, T, D) and write them in place at
    rows ``positions[b] .. positions[b]+T-1`` of the (B, Hkv, cap, .) cache --
    the quantize + concatenate of ``engine/gemma4_multilayer.cpp:228-240``
    done as an in-place append."""
    kqn, ksn, kbn = quantize_int4(k_new, sb_dtype, mode)
    vqn, vsn, vbn = quantize_int4(v_new, sb_dtype, mode)
    T = k_new.shape[2]
    for b, p in enumerate(positions):
        p = int(p)
        cache["kq"][b, :, p:p + T] = kqn[b]
        cache["ks"][b, :, p:p + T] = ksn[b]
        cache["kb"][b, :, p:p + T] = kbn[b]
        cache["vq"][b, :, p:p + T] = vqn[b]
        cache["vs"][b, :, p:p + T] = vsn[b]
        cache["vb"][b, :, p:p + T] = vbn[b]


# --------------------------------------------------------------------------
# byte model
# --------------------------------------------------------------------------

def row_bytes(D: int, sb_bytes: int = 2) -> int:
    """Packed K+V bytes of one (kv-head, token) row: nibbles + scale + bias."""
    return 2 * (D // 2 + 2 * (D // GROUP_SIZE) * sb_bytes)


def decode_bytes(Hq: int, Hkv: int, D: int, attended: int, q_bytes: int = 2,
                 sb_bytes: int = 2) -> int:
    """Algorithmic HBM bytes of one decode call: every attended K/V row once,
    Q once, fp32 O once (split-K scratch excluded)."""
    return Hkv * attended * row_bytes(D, sb_bytes) + Hq * D * q_bytes + Hq * D * 4
