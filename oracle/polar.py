"""NumPy restatement of the reference's PolarQuant kernels, and of the QJL
residual sketch and compressed-key decode attention of the 7-level "polar7"
layout (D = 128).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference locations restated:

* encode -- ``polar_fused_quantize`` / ``polar_quantize_packed``
  (``lib/turboquant.metal:8-98``, ``:501-600``): per block of 2^L values,
  level 1 pairs (y[2j], y[2j+1]) -> angle atan2(b, a) wrapped to [0, 2pi)
  (``:35-36``) and radius sqrt(a^2 + b^2); each later level pairs the previous
  radii (angles in [0, pi/2], not wrapped, ``:54``); every angle is replaced
  by the index of the nearest codebook entry under the linear distance
  |theta - c|, first minimum wins (``:38-42``); the last radius is stored as
  fp16 (``:96``).  The reference hard-codes 16-value blocks (4 levels); the
  same recursion over one 128-value block (7 levels) is the polar7
  encoding.
* preconditioning -- ``y = x P^T`` before encoding (``lib/turboquant.cpp:102``),
  ``x = y P`` after decoding (``:122``).
* decode -- ``polar_inverse_dequantize`` / ``polar_inverse_packed`` /
  ``polar_inverse_packed_fast`` (``lib/turboquant.metal:100-164``,
  ``:602-704``): top-down, each value v of a level becomes
  (v cos(theta), v sin(theta)).
* packing -- level 1 index j at bits [4j, 4j+4) of a uint32 (``:540``),
  level 2..4 index j at bits [2j, 2j+2) of a uint8 (``:560,580,597``).
* scores -- ``tq_score_shared`` (``:424-499``): scores[h, n] =
  sum_d (scale q[h, d]) khat[h*N + n, d], keys indexed by query head
  (``:453``); this build adds GQA (kv head = h // gqa).
* attention -- ``sdpa_tq_sequential`` (``:166-224``): online softmax over the
  scores, fp32 values, output acc / (l + 1e-8) (``:222``).

Bit-exactness of the encoder.  The index decisions depend on float32
rounding, so the encoder is defined as an exact sequence of IEEE float32
operations that the HIP encoder performs in the same order (no fused
multiply-add): ``atan2_f32`` below (range reduction plus the alternating
Taylor series of atan, 10 terms), correctly rounded division and square
root, separately rounded products and sums.  Metal's atan2 and fma
contraction are not reproducible on any other machine, so the reference's
own bits are not the target; what is pinned (tests/test_oracle_polar.py) is
that every index equals the nearest-codebook index of the exact angle except
where the angle lies within 1e-5 rad of a decision boundary.

QJL (``README.md:11,176``; not implemented in the reference): the residual
r = y - yhat of the polar encoding (y-space, after the rotation) is sketched
as m = 128 sign bits of S r (bit i set iff (S r)_i >= 0), with S ~ N(0,1)
(m x D) and ||r|| stored as fp16.  Score estimate:
<q', yhat> + sqrt(pi/2)/m * ||r|| * <S q', sign(S r)>, q' = P q.
"""
from __future__ import annotations

import numpy as np

f32 = np.float32

PI = f32(np.pi)
PI_2 = f32(np.pi / 2)
PI_4 = f32(np.pi / 4)
TWO_PI = f32(2 * np.pi)
TAN_PI_8 = f32(np.tan(np.pi / 8))
# atan(u) = u + u * (s * sum_{k>=1} c_k s^(k-1)), s = u^2, c_k = (-1)^k/(2k+1)
ATAN_C = [f32((-1) ** k / (2 * k + 1)) for k in range(1, 11)]
QJL_M = 128


# --------------------------------------------------------------------------
# deterministic float32 atan2
# --------------------------------------------------------------------------

def atan2_f32(y, x):
    """atan2(y, x) in (-pi, pi] as a fixed sequence of float32 operations.

    |t| = min/max of |x|, |y|; for t > tan(pi/8) the argument is reduced with
    atan(t) = pi/4 + atan((t-1)/(t+1)); atan of the reduced argument
    (|u| <= tan(pi/8)) is the Taylor series to u^21 (truncation < 2e-10).
    Octant and sign fix-ups follow atan2's conventions including signed
    zeros (atan2(+-0, -0) = +-pi, atan2(+-0, +0) = +-0).
    """
    y = np.asarray(y, dtype=f32)
    x = np.asarray(x, dtype=f32)
    ax, ay = np.abs(x), np.abs(y)
    mx, mn = np.maximum(ax, ay), np.minimum(ax, ay)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = np.where(mx > 0, mn / np.where(mx > 0, mx, f32(1)), f32(0)).astype(f32)
        big = t > TAN_PI_8
        u = np.where(big, (t - f32(1)) / (t + f32(1)), t).astype(f32)
    s = (u * u).astype(f32)
    p = np.full_like(s, ATAN_C[-1])
    for c in reversed(ATAN_C[:-1]):
        p = (p * s).astype(f32)
        p = (p + c).astype(f32)
    r = (s * p).astype(f32)
    r = (u * r).astype(f32)
    a = (u + r).astype(f32)
    a = np.where(big, PI_4 + a, a).astype(f32)
    a = np.where(ay > ax, PI_2 - a, a).astype(f32)
    a = np.where(np.signbit(x), PI - a, a).astype(f32)
    a = np.where(np.signbit(y), -a, a).astype(f32)
    return a


def nearest_index(theta, cb):
    """Index of the nearest codebook entry, |theta - c| in float32, first
    minimum wins (lib/turboquant.metal:38-42)."""
    cb = np.asarray(cb, dtype=f32)
    d = np.abs(np.asarray(theta, dtype=f32)[..., None] - cb).astype(f32)
    return np.argmin(d, axis=-1).astype(np.int64)


# --------------------------------------------------------------------------
# rotation and encode / decode
# --------------------------------------------------------------------------

def rotate_f32(x, P):
    """y = x P^T, y_i = sum_d x_d P[i, d] accumulated d = 0..D-1 in float32
    with separately rounded products and sums (the encoder's rotation)."""
    x = np.asarray(x, dtype=f32)
    P = np.asarray(P, dtype=f32)
    acc = np.zeros(x.shape[:-1] + (P.shape[0],), dtype=f32)
    for d in range(x.shape[-1]):
        acc = (acc + (x[..., d:d + 1] * P[:, d]).astype(f32)).astype(f32)
    return acc


def encode_blocks(y, codebooks):
    """Polar-encode the last axis of y (length 2^L, L = len(codebooks)).

    Returns (indices, radius): indices[l] has shape (..., 2^(L-1-l)) int64
    for level l+1; radius is the final radius as float16.
    """
    r = np.asarray(y, dtype=f32)
    L = len(codebooks)
    assert r.shape[-1] == 1 << L
    idx = []
    for lvl in range(L):
        a, b = r[..., 0::2], r[..., 1::2]
        th = atan2_f32(b, a)
        if lvl == 0:
            th = np.where(th < 0, th + TWO_PI, th).astype(f32)
        idx.append(nearest_index(th, codebooks[lvl]))
        aa = (a * a).astype(f32)
        bb = (b * b).astype(f32)
        r = np.sqrt((aa + bb).astype(f32)).astype(f32)
    return idx, r[..., 0].astype(np.float16)


def cs_table(cb):
    """float32 (cos, sin) of each codebook angle: shape (n, 2)."""
    c = np.asarray(cb, dtype=f32).astype(np.float64)
    return np.stack([np.cos(c), np.sin(c)], axis=-1).astype(f32)


def decode_blocks_f32(indices, radius, cs_tables):
    """Top-down decode in float32 with the given (cos, sin) tables, each child
    one rounded product of its parent (the encoder's residual reference)."""
    v = np.asarray(radius).astype(f32)[..., None]
    for lvl in range(len(indices) - 1, -1, -1):
        cs = np.asarray(cs_tables[lvl], dtype=f32)[indices[lvl]]  # (..., n, 2)
        out = np.empty(v.shape[:-1] + (2 * v.shape[-1],), dtype=f32)
        out[..., 0::2] = (v * cs[..., 0]).astype(f32)
        out[..., 1::2] = (v * cs[..., 1]).astype(f32)
        v = out
    return v


def decode_blocks(indices, radius, codebooks):
    """Top-down decode in float64 from the codebook angles (the reference's
    runtime cos/sin variant)."""
    v = np.asarray(radius).astype(np.float64)[..., None]
    for lvl in range(len(indices) - 1, -1, -1):
        th = np.asarray(codebooks[lvl], dtype=f32).astype(np.float64)[indices[lvl]]
        out = np.empty(v.shape[:-1] + (2 * v.shape[-1],))
        out[..., 0::2] = v * np.cos(th)
        out[..., 1::2] = v * np.sin(th)
        v = out
    return v


# --------------------------------------------------------------------------
# reference layouts (16-value blocks, 4 levels)
# --------------------------------------------------------------------------

def polar_quantize(x, P, cbs, block=16):
    """lib/turboquant.cpp:97-110 + lib/turboquant.metal:8-98: returns the
    unpacked layout (idx_l1 u8 [nb*8], idx_l2 [nb*4], idx_l3 [nb*2],
    idx_l4 [nb], radii f16 [nb]) over nb = N*D/16 blocks in row-major order."""
    x = np.asarray(x, dtype=f32)
    y = rotate_f32(x, P) if P is not None else x
    blocks = y.reshape(-1, block)
    idx, rad = encode_blocks(blocks, cbs)
    return tuple(i.astype(np.uint8).reshape(-1) for i in idx) + (rad.reshape(-1),)


def pack_ref(idx_levels):
    """Unpacked u8 indices of the 4 levels -> the reference packed layout
    (lib/turboquant.metal:501-600): p1 u32 [nb], p2/p3/p4 u8 [nb]."""
    i1, i2, i3, i4 = (np.asarray(a, dtype=np.uint32) for a in idx_levels)
    nb = i4.shape[0]
    i1 = i1.reshape(nb, 8)
    i2 = i2.reshape(nb, 4)
    i3 = i3.reshape(nb, 2)
    p1 = np.zeros(nb, dtype=np.uint32)
    for j in range(8):
        p1 |= (i1[:, j] & 0xF) << (4 * j)
    p2 = np.zeros(nb, dtype=np.uint32)
    for j in range(4):
        p2 |= (i2[:, j] & 0x3) << (2 * j)
    p3 = np.zeros(nb, dtype=np.uint32)
    for j in range(2):
        p3 |= (i3[:, j] & 0x3) << (2 * j)
    return p1, p2.astype(np.uint8), p3.astype(np.uint8), (i4 & 0x3).astype(np.uint8)


def unpack_ref(p1, p2, p3, p4):
    p1 = np.asarray(p1, dtype=np.uint32)
    nb = p1.shape[0]
    i1 = np.stack([(p1 >> (4 * j)) & 0xF for j in range(8)], axis=1).reshape(-1)
    p2 = np.asarray(p2, dtype=np.uint32)
    i2 = np.stack([(p2 >> (2 * j)) & 0x3 for j in range(4)], axis=1).reshape(-1)
    p3 = np.asarray(p3, dtype=np.uint32)
    i3 = np.stack([(p3 >> (2 * j)) & 0x3 for j in range(2)], axis=1).reshape(-1)
    i4 = np.asarray(p4, dtype=np.uint32) & 0x3
    return [a.astype(np.int64) for a in (i1, i2, i3, i4)]


def polar_dequantize(i1, i2, i3, i4, radii, P, cbs, D, block=16):
    """Decode the unpacked layout to y (P is None: the ``_fast`` variants,
    lib/turboquant.cpp:191-200) or to x = y P (lib/turboquant.cpp:112-123)."""
    nb = np.asarray(radii).shape[0]
    idx = [np.asarray(i1, np.int64).reshape(nb, 8), np.asarray(i2, np.int64).reshape(nb, 4),
           np.asarray(i3, np.int64).reshape(nb, 2), np.asarray(i4, np.int64).reshape(nb, 1)]
    y = decode_blocks(idx, np.asarray(radii), cbs).reshape(-1, D)
    if P is not None:
        y = y @ np.asarray(P, dtype=f32).astype(np.float64)
    return y


def compressed_score(q, i1, i2, i3, i4, radii, cbs, N, scale, gqa=1, block=16):
    """lib/turboquant.metal:424-499 (+ GQA): scores (Nq, N), float64."""
    q = np.asarray(q, dtype=f32).astype(np.float64)
    Nq, D = q.shape
    k = polar_dequantize(i1, i2, i3, i4, radii, None, cbs, D, block)
    Hk = k.shape[0] // N
    k = k.reshape(Hk, N, D)
    out = np.empty((Nq, N))
    for h in range(Nq):
        out[h] = k[h // gqa] @ (np.float64(f32(scale)) * q[h])
    return out


def softmax_rows(s, axis=-1):
    m = np.max(s, axis=axis, keepdims=True)
    e = np.exp(s - m)
    return e, e.sum(axis=axis, keepdims=True)


def compressed_sdpa(q, i1, i2, i3, i4, radii, cbs, values, scale, gqa=1, block=16):
    """lib/turboquant.metal:166-224 (+ GQA): values (Hk*N, D) float32, output
    acc / (l + 1e-8) per head (``:222``)."""
    q = np.asarray(q, dtype=f32)
    Nq, D = q.shape
    values = np.asarray(values, dtype=f32).astype(np.float64)
    Hk = Nq // gqa
    N = values.shape[0] // Hk
    s = compressed_score(q, i1, i2, i3, i4, radii, cbs, N, scale, gqa, block)
    v = values.reshape(Hk, N, D)
    out = np.zeros((Nq, D))
    if N == 0:
        return out
    e, l = softmax_rows(s)
    for h in range(Nq):
        out[h] = (e[h] @ v[h // gqa]) / (l[h, 0] + 1e-8)
    return out


# --------------------------------------------------------------------------
# polar7: 7-level full-vector PolarQuant + QJL (D = 128)
# --------------------------------------------------------------------------

P7_D = 128
P7_LEVELS = 7
P7_WORDS = 12  # packed angle words per vector


def polar7_codebooks():
    """Uniform midpoint codebooks: level 1 (k+1/2) 2pi/16 (k < 16), levels
    2..7 (k+1/2) pi/8 (k < 4).  With midpoints the linear nearest-entry
    search equals the circular one (no wrap-around ambiguity at 2pi)."""
    cb1 = ((np.arange(16) + 0.5) * (2 * np.pi / 16)).astype(f32)
    cb2 = ((np.arange(4) + 0.5) * (np.pi / 8)).astype(f32)
    return cb1, cb2


def pack_polar7(idx):
    """idx[l] (N, 64 >> l) -> angles u32 (N, 12):
    words 0-7 level 1 (pair j at word j/8, bits 4(j%8)); words 8-9 level 2
    (pair j at word 8 + j/16, bits 2(j%16)); word 10 level 3 (bits 2j);
    word 11: level 4 bits 2j, level 5 at 16 + 2j, level 6 at 24 + 2j, level 7
    at bits 28-29."""
    N = idx[0].shape[0]
    w = np.zeros((N, P7_WORDS), dtype=np.uint32)
    i1 = idx[0].astype(np.uint32)
    for j in range(64):
        w[:, j // 8] |= (i1[:, j] & 0xF) << (4 * (j % 8))
    i2 = idx[1].astype(np.uint32)
    for j in range(32):
        w[:, 8 + j // 16] |= (i2[:, j] & 0x3) << (2 * (j % 16))
    i3 = idx[2].astype(np.uint32)
    for j in range(16):
        w[:, 10] |= (i3[:, j] & 0x3) << (2 * j)
    base = {3: 0, 4: 16, 5: 24, 6: 28}
    for lvl in (3, 4, 5, 6):
        il = idx[lvl].astype(np.uint32)
        for j in range(il.shape[1]):
            w[:, 11] |= (il[:, j] & 0x3) << (base[lvl] + 2 * j)
    return w


def unpack_polar7(w):
    w = np.asarray(w, dtype=np.uint32)
    idx = [np.stack([(w[:, j // 8] >> (4 * (j % 8))) & 0xF for j in range(64)], axis=1)]
    idx.append(np.stack([(w[:, 8 + j // 16] >> (2 * (j % 16))) & 0x3 for j in range(32)], axis=1))
    idx.append(np.stack([(w[:, 10] >> (2 * j)) & 0x3 for j in range(16)], axis=1))
    for base, n in ((0, 8), (16, 4), (24, 2), (28, 1)):
        idx.append(np.stack([(w[:, 11] >> (base + 2 * j)) & 0x3 for j in range(n)], axis=1))
    return [a.astype(np.int64) for a in idx]


def tree_sum_f32(v):
    """Pairwise sum over the last axis (adjacent pairs first), float32."""
    v = np.asarray(v, dtype=f32)
    while v.shape[-1] > 1:
        v = (v[..., 0::2] + v[..., 1::2]).astype(f32)
    return v[..., 0]


def sketch_f32(S, r):
    """(S r)_i = sum_d S[i, d] r_d, accumulated d = 0..D-1 in float32 with
    separately rounded products and sums."""
    S = np.asarray(S, dtype=f32)
    r = np.asarray(r, dtype=f32)
    acc = np.zeros(r.shape[:-1] + (S.shape[0],), dtype=f32)
    for d in range(r.shape[-1]):
        acc = (acc + (r[..., d:d + 1] * S[:, d]).astype(f32)).astype(f32)
    return acc


def polar7_encode(x, P, S, cb1=None, cb2=None):
    """polar7 key encoding of x (N, 128) float32.

    Returns (angles u32 (N, 12), norms f16 (N, 2) = (radius, ||r||),
    qjl u32 (N, 4) with bit i of word i/32 = [(S r)_i >= 0]).
    """
    if cb1 is None:
        cb1, cb2 = polar7_codebooks()
    x = np.asarray(x, dtype=f32)
    y = rotate_f32(x, P) if P is not None else x
    cbs = [cb1] + [cb2] * 6
    idx, rad = encode_blocks(y, cbs)
    cst = [cs_table(cb1)] + [cs_table(cb2)] * 6
    yhat = decode_blocks_f32(idx, rad, cst)
    r = (y - yhat).astype(f32)
    rn = np.sqrt(tree_sum_f32((r * r).astype(f32))).astype(f32)
    sk = sketch_f32(S, r)
    bits = (sk >= 0).astype(np.uint32)
    qjl = np.zeros((x.shape[0], 4), dtype=np.uint32)
    for i in range(QJL_M):
        qjl[:, i // 32] |= bits[:, i] << (i % 32)
    norms = np.stack([rad, rn.astype(np.float16)], axis=1)
    return pack_polar7(idx), norms, qjl


def polar7_decode(angles, norms, cb1=None, cb2=None):
    """yhat (N, 128) float64 from the packed angles and the fp16 radius."""
    if cb1 is None:
        cb1, cb2 = polar7_codebooks()
    idx = unpack_polar7(angles)
    cst = [cs_table(cb1)] + [cs_table(cb2)] * 6
    v = np.asarray(norms)[:, 0].astype(np.float64)[:, None]
    for lvl in range(6, -1, -1):
        cs = cst[lvl].astype(np.float64)[idx[lvl]]
        out = np.empty((v.shape[0], 2 * v.shape[1]))
        out[:, 0::2] = v * cs[..., 0]
        out[:, 1::2] = v * cs[..., 1]
        v = out
    return v


def qjl_signs(qjl):
    qjl = np.asarray(qjl, dtype=np.uint32)
    bits = np.stack([(qjl[:, i // 32] >> (i % 32)) & 1 for i in range(QJL_M)], axis=1)
    return bits.astype(np.float64) * 2.0 - 1.0


def polar7_scores(qp, qs, angles, norms, qjl, gqa, scale=1.0, cb1=None, cb2=None):
    """polar7 scores, float64: scores[h, n] = scale * (<q'_h, yhat_n> +
    sqrt(pi/2)/m * ||r_n|| * <qs_h, sign_n>) for keys of kv head h // gqa.

    qp (Hq, 128) = P q (the rotated query), qs (Hq, 128) = S qp;
    angles (Hkv, N, 12), norms (Hkv, N, 2), qjl (Hkv, N, 4)."""
    qp = np.asarray(qp, dtype=f32).astype(np.float64)
    qs = np.asarray(qs, dtype=f32).astype(np.float64)
    Hq = qp.shape[0]
    Hkv, N = angles.shape[0], angles.shape[1]
    coef = np.sqrt(np.pi / 2) / QJL_M
    out = np.empty((Hq, N))
    for hk in range(Hkv):
        yhat = polar7_decode(angles[hk], norms[hk], cb1, cb2)
        sg = qjl_signs(qjl[hk])
        rn = np.asarray(norms[hk])[:, 1].astype(np.float64)
        for g in range(gqa):
            h = hk * gqa + g
            out[h] = np.float64(f32(scale)) * (yhat @ qp[h] + coef * rn * (sg @ qs[h]))
    return out


def polar7_sdpa_int4v(qp, qs, angles, norms, qjl, vq, vs, vb, gqa, scale=1.0,
                      window=0, kv_len=None, cb1=None, cb2=None):
    """polar7 attention: softmax over the polar+QJL scores of the attended
    keys, times the int4-dequantized V; empty key set -> 0.  Keys/values of
    rows [0, kv_len) with the sdpa_int4 window rule."""
    from oracle import oracle as O
    Hkv = angles.shape[0]
    N = angles.shape[1] if kv_len is None else kv_len
    lo, hi = O.attended_range(N, window)
    s = polar7_scores(qp, qs, angles[:, lo:hi], norms[:, lo:hi], qjl[:, lo:hi], gqa,
                      scale, cb1, cb2)
    v = O.dequantize(vq[:, lo:hi], vs[:, lo:hi], vb[:, lo:hi])
    Hq = s.shape[0]
    out = np.zeros((Hq, v.shape[-1]))
    if hi <= lo:
        return out
    e, l = softmax_rows(s)
    for h in range(Hq):
        out[h] = (e[h] @ v[h // gqa]) / l[h, 0]
    return out


def qjl_query(qp, S):
    """S q' per head, float64."""
    return np.asarray(qp, dtype=f32).astype(np.float64) @ np.asarray(S, dtype=f32).astype(np.float64).T


def polar7_row_bytes(D: int = P7_D, sb_bytes: int = 2) -> int:
    """Bytes per (kv head, token) of the polar7 layout: K = 48 B angles + 16 B sketch
    + 4 B (radius, ||r||) fp16; V = int4 nibbles + fp16 scale/bias."""
    return P7_WORDS * 4 + QJL_M // 8 + 4 + D // 2 + 2 * (D // 64) * sb_bytes


def polar7_decode_bytes(Hq: int, Hkv: int, attended: int, q_bytes: int = 4) -> int:
    """Algorithmic bytes of one polar7 decode layer: the compressed K and
    int4 V rows once, q' and S q' (fp32) in, fp32 out."""
    return Hkv * attended * polar7_row_bytes() + 2 * Hq * P7_D * q_bytes + Hq * P7_D * 4
