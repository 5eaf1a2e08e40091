"""CPU: pins the attention oracle against an independent library routine
(torch float64 scaled_dot_product_attention), closed forms and invariants, and
checks the two restatements (numpy, C) agree.  Also shows that plausible
mistakes planted in the oracle (on the CPU) are caught by these checks."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def make_case(seed, Hq, Hkv, D, L, sb="f16", cap=None):
    rng = np.random.default_rng(seed)
    cap = cap or L
    q = O.rms_norm(rng.standard_normal((Hq, D)).astype(np.float32))
    k = O.rms_norm(rng.standard_normal((Hkv, cap, D)).astype(np.float32))
    v = rng.standard_normal((Hkv, cap, D)).astype(np.float32)
    kq, ks, kb = O.quantize_int4(k, sb)
    vq, vs, vb = O.quantize_int4(v, sb)
    return q, (kq, ks, kb, vq, vs, vb)


def torch_reference(q, cache, gqa, scale, window, n):
    """softmax attention by torch's SDPA in float64 over the dequantized K/V,
    with the reference's window rule applied literally as a boolean mask
    (key ki is dropped iff window > 0 and n-1-ki >= window,
    lib/turboquant.metal:779)."""
    kq, ks, kb, vq, vs, vb = cache
    K = torch.from_numpy(O.dequantize(kq[:, :n], ks[:, :n], kb[:, :n]))
    V = torch.from_numpy(O.dequantize(vq[:, :n], vs[:, :n], vb[:, :n]))
    K = K.repeat_interleave(gqa, dim=0)[None]
    V = V.repeat_interleave(gqa, dim=0)[None]
    Q = torch.from_numpy(np.asarray(q, np.float64))[None, :, None, :]
    ki = torch.arange(n)
    keep = ~((window > 0) & ((n - 1 - ki) >= window))
    if not bool(keep.any()):
        return np.zeros(q.shape)
    out = torch.nn.functional.scaled_dot_product_attention(
        Q, K.contiguous(), V.contiguous(), attn_mask=keep[None, None, None, :], scale=scale)
    return out[0, :, 0, :].numpy()


@pytest.mark.parametrize("Hq,Hkv,D,L,W,scale", [
    (2, 1, 128, 33, 0, 1.0),        # tiny decode shape
    (16, 16, 256, 10, 0, 1.0),      # reference test shape (tests/test_sdpa_int4.cpp:13)
    (32, 16, 256, 300, 128, 1.0),   # sliding layer, window active
    (8, 1, 512, 77, 0, 0.125),      # global-layer-like GQA 8, D 512
    (6, 2, 128, 50, 50, 1.0),       # window == L (inactive)
])
def test_oracle_matches_torch_sdpa(Hq, Hkv, D, L, W, scale):
    q, cache = make_case(Hq * 1000 + L, Hq, Hkv, D, L)
    got = O.sdpa_int4(q, *cache, Hq // Hkv, scale, W)
    ref = torch_reference(q, cache, Hq // Hkv, scale, W, L)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-10)


def test_window_rule_examples():
    assert O.attended_range(5, 2) == (3, 5)
    assert O.attended_range(5, 0) == (0, 5)
    assert O.attended_range(1, 1024) == (0, 1)
    assert O.attended_range(786, 1024) == (0, 786)
    assert O.attended_range(0, 4) == (0, 0)


def test_single_key_returns_value_row():
    q, cache = make_case(1, 4, 2, 128, 1)
    out = O.sdpa_int4(q, *cache, 2)
    V = O.dequantize(*cache[3:])
    for h in range(4):
        np.testing.assert_allclose(out[h], V[h // 2, 0], atol=1e-12)


def test_identical_keys_give_mean_of_values():
    q, cache = make_case(2, 2, 1, 256, 20)
    kq, ks, kb, vq, vs, vb = cache
    kq[:] = kq[:, :1]; ks[:] = ks[:, :1]; kb[:] = kb[:, :1]
    out = O.sdpa_int4(q, kq, ks, kb, vq, vs, vb, 2)
    V = O.dequantize(vq, vs, vb)
    np.testing.assert_allclose(out[0], V[0].mean(0), atol=1e-12)


def test_two_key_closed_form():
    q, cache = make_case(3, 1, 1, 128, 2)
    K = O.dequantize(*cache[:3])[0]
    V = O.dequantize(*cache[3:])[0]
    s = K @ q[0].astype(np.float64) * float(np.float32(0.3))  # scale is a C float
    w1 = 1.0 / (1.0 + np.exp(s[0] - s[1]))      # sigmoid(s1 - s0)
    expect = (1 - w1) * V[0] + w1 * V[1]
    np.testing.assert_allclose(O.sdpa_int4(q, *cache, 1, 0.3)[0], expect, atol=1e-12)


def test_key_permutation_and_window_invariances():
    q, cache = make_case(4, 4, 2, 128, 40)
    base = O.sdpa_int4(q, *cache, 2)
    perm = np.random.default_rng(0).permutation(40)
    permuted = tuple(a[:, perm] for a in cache)
    np.testing.assert_allclose(O.sdpa_int4(q, *permuted, 2), base, atol=1e-12)
    np.testing.assert_allclose(O.sdpa_int4(q, *cache, 2, 1.0, 40), base, atol=1e-15)
    np.testing.assert_allclose(O.sdpa_int4(q, *cache, 2, 1.0, 1000), base, atol=1e-15)
    last = tuple(a[:, -7:] for a in cache)
    np.testing.assert_allclose(O.sdpa_int4(q, *cache, 2, 1.0, 7), O.sdpa_int4(q, *last, 2),
                               atol=1e-15)


def test_kv_len_prefix_of_capacity():
    q, cache = make_case(5, 2, 1, 128, 30, cap=64)
    pre = tuple(a[:, :30] for a in cache)
    np.testing.assert_allclose(O.sdpa_int4(q, *cache, 2, kv_len=30), O.sdpa_int4(q, *pre, 2),
                               atol=1e-15)


def test_empty_key_set_gives_zero():
    q, cache = make_case(6, 2, 1, 128, 8)
    assert np.all(O.sdpa_int4(q, *cache, 2, kv_len=0) == 0)


def test_ragged_is_per_sequence():
    rng = np.random.default_rng(9)
    B, Hq, Hkv, D, cap = 3, 4, 2, 128, 40
    q = O.rms_norm(rng.standard_normal((B, Hq, D)).astype(np.float32))
    k = O.rms_norm(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32))
    v = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    c = O.quantize_int4(k) + O.quantize_int4(v)
    lens, wins = [40, 1, 17], [0, 4, 5]
    got = O.sdpa_int4_ragged(q, *c, lens, wins, 2)
    for b in range(B):
        ref = torch_reference(q[b], tuple(a[b] for a in c), 2, 1.0, wins[b], lens[b])
        np.testing.assert_allclose(got[b], ref, atol=1e-10)


def test_c_oracle_matches_numpy_oracle(coracle):
    q, cache = make_case(11, 8, 4, 256, 100, cap=128)
    a = O.sdpa_int4(q, *cache, 2, 0.7, 37, kv_len=100)
    b = coracle.sdpa_int4_f64(q, *cache, 2, 0.7, 37, kv_len=100)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_c_cpu_baseline_close_to_oracle(coracle):
    q, cache = make_case(12, 32, 16, 256, 3000)
    base = coracle.DequantSdpaBaseline(q, *cache, 2, 1.0, 1024, threads=4)()
    ref = O.sdpa_int4(q, *cache, 2, 1.0, 1024)
    assert np.max(np.abs(base - ref)) < 1e-4


# ---- planted mistakes (in a copy of the oracle, on the CPU) are caught -------

def _mutant_sdpa(q, cache, gqa, mutation):
    kq, ks, kb, vq, vs, vb = cache
    Hq = q.shape[0]
    out = np.zeros(q.shape)
    for h in range(Hq):
        kvh = (h % kq.shape[0]) if mutation == "gqa_mod" else h // gqa
        K = O.dequantize(kq[kvh], ks[kvh], np.zeros_like(kb[kvh]) if mutation == "no_bias" else kb[kvh])
        V = O.dequantize(vq[kvh], vs[kvh], vb[kvh])
        out[h] = O.softmax_attend(q[h].astype(np.float64), K, V, 1.0)
    return out


@pytest.mark.parametrize("mutation", ["gqa_mod", "no_bias"])
def test_planted_mistakes_fail_library_check(mutation):
    Hq, Hkv = 8, 4
    q, cache = make_case(13, Hq, Hkv, 128, 24)
    ref = torch_reference(q, cache, 2, 1.0, 0, 24)
    assert np.max(np.abs(_mutant_sdpa(q, cache, 2, mutation) - ref)) > 1e-2
    assert np.max(np.abs(_mutant_sdpa(q, cache, 2, "none") - ref)) < 1e-10


def prefill_case(seed, S, prior, Hq, Hkv, D):
    rng = np.random.default_rng(seed)
    q = O.rms_norm(rng.standard_normal((S, Hq, D)).astype(np.float32))
    k = O.rms_norm(rng.standard_normal((Hkv, prior + S, D)).astype(np.float32))
    v = rng.standard_normal((Hkv, prior + S, D)).astype(np.float32)
    return q, O.quantize_int4(k) + O.quantize_int4(v)


def test_prefill_oracle_is_torch_causal_attention():
    """n_prior = 0, no window: exactly torch's is_causal attention (a library
    routine) over the dequantized cache, GQA by repeating kv heads."""
    S, Hq, Hkv, D = 40, 8, 2, 128
    q, cache = prefill_case(5, S, 0, Hq, Hkv, D)
    got = O.sdpa_int4_prefill(q, *cache, 0, Hq // Hkv, 0.7)
    kq, ks, kb, vq, vs, vb = cache
    K = torch.from_numpy(O.dequantize(kq, ks, kb)).repeat_interleave(Hq // Hkv, 0)[None]
    V = torch.from_numpy(O.dequantize(vq, vs, vb)).repeat_interleave(Hq // Hkv, 0)[None]
    Q = torch.from_numpy(np.asarray(q, np.float64)).permute(1, 0, 2)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(
        Q.contiguous(), K.contiguous(), V.contiguous(), is_causal=True, scale=float(np.float32(0.7)))
    np.testing.assert_allclose(got, ref[0].permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("S,prior,W", [(24, 50, 0), (24, 50, 16), (1, 70, 0), (9, 0, 4)])
def test_prefill_oracle_equals_per_query_decode(S, prior, W):
    """Query i of a prefill is the decode of a sequence of n_prior + i + 1
    keys under the same window (the decode oracle is pinned above)."""
    Hq, Hkv, D = 4, 2, 256
    q, cache = prefill_case(S + prior + W, S, prior, Hq, Hkv, D)
    got = O.sdpa_int4_prefill(q, *cache, prior, 2, 1.0, W)
    for i in range(S):
        ref = O.sdpa_int4(q[i], *cache, 2, 1.0, W, kv_len=prior + i + 1)
        np.testing.assert_allclose(got[i], ref, rtol=1e-10, atol=1e-10)


def test_prefill_oracle_catches_planted_causal_off_by_one(monkeypatch):
    """A mask that also hides the query's own key (j >= pos instead of
    j > pos) must fail the per-query decode comparison."""
    S, prior = 6, 10
    q, cache = prefill_case(9, S, prior, 2, 1, 128)
    real = np.where

    def shifted(cond, a, b):
        if isinstance(cond, np.ndarray) and cond.ndim == 2 and cond.shape == (S, prior + S):
            pos = prior + np.arange(S)[:, None]
            cond = cond | (np.arange(prior + S)[None, :] == pos)
        return real(cond, a, b)
    monkeypatch.setattr(O.np, "where", shifted)
    bad = O.sdpa_int4_prefill(q, *cache, prior, 2)
    monkeypatch.undo()
    ref = np.stack([O.sdpa_int4(q[i], *cache, 2, kv_len=prior + i + 1) for i in range(S)])
    assert np.abs(bad - ref).max() > 1e-3
