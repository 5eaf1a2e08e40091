"""CPU: pins the quantize oracle (numpy + C restatements) with hand-derived
known answers, cross-restatement bit equality and error bounds.

The reference ships no quantization vectors (its only test draws unseeded
random data, tests/test_sdpa_int4.cpp:20-26) and MLX is not installed, so the
expected values below are derived by hand from the MLX affine rule; each case
is chosen so a plausible mistake (bias=min instead of the edge rule, a flipped
scale sign, round-half-away instead of rint, a reversed nibble order) fails.
"""
import numpy as np
import pytest

from oracle import oracle as O


def group(vals, fill=0.0):
    g = np.full(64, fill, np.float32)
    g[: len(vals)] = np.asarray(vals, np.float32)
    return g[None]


def test_known_answer_max_edge_reverses_nibbles():
    # x_i = i mod 16: mx=15 dominates -> scale=-1, bias=15, q = 15 - x.
    x = np.tile(np.arange(16, dtype=np.float32), 4)[None]
    wq, s, b = O.mlx_affine_quantize(x)
    assert s[0, 0] == np.float32(-1.0) and b[0, 0] == np.float32(15.0)
    assert wq[0, 0] == 0x89ABCDEF and wq[0, 1] == 0x01234567
    assert np.array_equal(O.dequantize(wq, s, b), x.astype(np.float64))
    # the literal min/max rule gives the un-reversed code instead
    wq2, s2, b2 = O.minmax_affine_quantize(x)
    assert s2[0, 0] == 1.0 and b2[0, 0] == 0.0 and wq2[0, 0] == 0x76543210


def test_known_answer_min_edge():
    # x_i = -(i mod 16): |mn|=15 dominates -> scale=+1, bias=-15, q = x + 15.
    x = -np.tile(np.arange(16, dtype=np.float32), 4)[None]
    wq, s, b = O.mlx_affine_quantize(x)
    assert s[0, 0] == 1.0 and b[0, 0] == -15.0
    assert wq[0, 0] == 0x89ABCDEF


def test_known_answer_rint_ties_to_even():
    # mx=15, mn=0 -> scale=-1, bias=15, q = rint(15 - x):
    # 7.5 -> 8 ; 6.5 -> 8.5 -> 8 ; 8.5 -> 6.5 -> 6 ; 0.5 -> 14.5 -> 14
    wq, s, b = O.mlx_affine_quantize(group([0, 15, 7.5, 6.5, 8.5, 0.5, 0, 0]))
    assert wq[0, 0] == 0xFFE6880F


def test_known_answer_mixed_sign_zero_point():
    # mn=-8 dominates mx=4: scale0=0.8, q0=rint(-8/0.8)=-10, scale=0.8, bias=-8
    wq, s, b = O.mlx_affine_quantize(group([-8, 4, 0, 1, -4]))
    assert s[0, 0] == np.float32(-8.0) / np.float32(-10.0) and b[0, 0] == -8.0
    assert wq[0, 0] == 0xAAA5BAF0
    deq = O.dequantize(wq, s, b)
    assert deq[0, 0] == -8.0 and abs(deq[0, 2]) < 1e-6  # zero (nearly) exact


def test_known_answer_constant_groups():
    wq, s, b = O.mlx_affine_quantize(group([], fill=0.0))
    assert wq[0, 0] == 0 and b[0, 0] == 0.0 and s[0, 0] == np.float32(-1e-7)
    wq, s, b = O.mlx_affine_quantize(group([], fill=3.0))
    assert np.all(wq == 0) and b[0, 0] == 3.0
    assert np.all(O.dequantize(wq, s, b) == 3.0)


def test_pack_order_and_groups():
    # two groups: group 0 ascending 0..15 (reversed code), group 1 all 5.
    x = np.concatenate([np.tile(np.arange(16, dtype=np.float32), 4),
                        np.full(64, 5.0, np.float32)])[None]
    wq, s, b = O.mlx_affine_quantize(x)
    assert wq.shape == (1, 16) and s.shape == (1, 2)
    assert np.all(wq[0, 8:] == 0) and b[0, 1] == 5.0
    n = O.unpack_nibbles(wq)
    assert list(n[0, :16]) == list(range(15, -1, -1))


@pytest.mark.parametrize("seed,scale", [(0, 1.0), (1, 1e-3), (2, 50.0), (3, 1e-30)])
def test_c_and_numpy_restatements_bit_equal(coracle, seed, scale):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((257, 256)) * scale).astype(np.float32)
    x[3] = 0.0
    x[4] = 7.25
    x[5, :64] = np.arange(64) % 16
    for mode, fn in ((0, O.mlx_affine_quantize), (1, O.minmax_affine_quantize)):
        a = fn(x)
        c = coracle.quantize_int4(x, mode)
        for u, v in zip(a, c):
            assert np.array_equal(u, v)


@pytest.mark.parametrize("seed", range(4))
def test_reconstruction_error_bound(seed):
    rng = np.random.default_rng(100 + seed)
    x = rng.standard_normal((64, 512)).astype(np.float32) * rng.uniform(0.01, 10)
    wq, s, b = O.mlx_affine_quantize(x)
    deq = O.dequantize(wq, s, b)
    err = np.abs(deq - x).reshape(64, 8, 64).max(-1)
    assert np.all(err <= np.abs(s) * 1.0001 + 1e-6)
    # nibbles cover the group range: both 0 and 15 appear in (almost) every group
    n = O.unpack_nibbles(wq).reshape(64, 8, 64)
    assert np.mean((n.min(-1) == 0) & (n.max(-1) >= 14)) > 0.95


def test_fp16_scale_storage_is_rne_cast():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    wq32, s32, b32 = O.quantize_int4(x, "f32")
    wq16, s16, b16 = O.quantize_int4(x, "f16")
    assert np.array_equal(wq32, wq16)
    assert s16.dtype == np.float16 and np.array_equal(s16, s32.astype(np.float16))
    assert np.array_equal(b16, b32.astype(np.float16))


def test_bf16_roundtrip_helpers():
    x = np.array([1.0, -2.5, 3.14159, 1e-20, 65504.0, 1.00390625], np.float32)
    b = O.f32_to_bf16_bits(x)
    y = O.bf16_bits_to_f32(b)
    assert y[0] == 1.0 and y[1] == -2.5
    assert np.all(np.abs(y - x) <= np.abs(x) * 2 ** -8)
    # 1 + 2^-8 is a tie between bf16 neighbours 1 and 1+2^-7: even mantissa -> 1.0
    assert y[5] == 1.0
