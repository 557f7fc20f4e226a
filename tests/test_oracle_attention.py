"""Pins oracle/attention.py: a single key returns its value, equal scores average the values, a window
equals slicing, GQA equals MHA with repeated KV heads, prefill rows equal decode at each position, and prefill
equals torch's scaled_dot_product_attention (float64, explicit mask) on the dequantized cache."""
import numpy as np
import torch

from oracle.attention import decode_attention, prefill_attention
from oracle.layout import PAGE, PagedCache
from oracle.numerics import bf16_round


def make(B, n, hkv, seed, table=None):
    rng = np.random.default_rng(seed)
    k = bf16_round(rng.standard_normal((B, n, hkv, 128)).astype(np.float32))
    v = bf16_round(rng.standard_normal((B, n, hkv, 128)).astype(np.float32))
    mp = (n + PAGE - 1) // PAGE
    if table is None:
        table = rng.permutation(B * mp).astype(np.int32).reshape(B, mp)
    cache = PagedCache(table.size, hkv)
    for b in range(B):
        cache.append(table, b, np.arange(n), k[b], v[b])
    return cache, table


def q_rows(shape, seed):
    return bf16_round(np.random.default_rng(seed).standard_normal(shape).astype(np.float32))


def test_single_key_returns_value():
    cache, table = make(2, 1, 2, 0)
    q = q_rows((2, 4, 128), 1)
    out = decode_attention(q, cache, table, np.array([1, 1]))
    for b in range(2):
        _, V = cache.gather_values(table, b, 1)
        assert np.allclose(out[b, :2], V[0, 0]) and np.allclose(out[b, 2:], V[0, 1])


def test_equal_scores_average_values():
    cache, table = make(1, 40, 1, 2)
    out = decode_attention(np.zeros((1, 1, 128)), cache, table, np.array([40]))
    _, V = cache.gather_values(table, 0, 40)
    assert np.allclose(out[0, 0], V[:, 0].astype(np.float64).mean(0))


def test_window_equals_slicing():
    n, w = 100, 30
    cache, table = make(1, n, 1, 3)
    q = q_rows((1, 1, 128), 4)
    out = decode_attention(q, cache, table, np.array([n]), window=w)
    K, V = cache.gather_values(table, 0, n)
    K, V = K[n - 1 - w:, 0].astype(np.float64), V[n - 1 - w:, 0].astype(np.float64)
    s = K @ q[0, 0].astype(np.float64) / np.sqrt(128)
    p = np.exp(s - s.max())
    assert np.allclose(out[0, 0], p @ V / p.sum())


def test_gqa_equals_repeated_mha():
    B, n, hkv, G = 2, 50, 2, 3
    cache, table = make(B, n, hkv, 5)
    q = q_rows((B, hkv * G, 128), 6)
    gqa = decode_attention(q, cache, table, np.array([n, n - 7]))
    rep = PagedCache(cache.k.shape[0], hkv * G)
    rep.k = np.repeat(cache.k, G, axis=1); rep.v = np.repeat(cache.v, G, axis=1)
    rep.ks = np.repeat(cache.ks, G, axis=1); rep.vs = np.repeat(cache.vs, G, axis=1)
    mha = decode_attention(q, rep, table, np.array([n, n - 7]))
    assert np.allclose(gqa, mha)


def test_prefill_rows_equal_decode_and_sdpa():
    B, ctx, T, hkv, G = 2, 45, 20, 2, 2
    cache, table = make(B, ctx + T, hkv, 7)
    q = q_rows((B, T, hkv * G, 128), 8)
    start = np.array([ctx, ctx])
    for window in (-1, 25):
        pre = prefill_attention(q, cache, table, start, window=window)
        for t in (0, 7, T - 1):
            dec = decode_attention(q[:, t], cache, table, start + t + 1, window=window)
            assert np.allclose(pre[:, t], dec)
        for b in range(B):
            K, V = cache.gather_values(table, b, ctx + T)
            pos = ctx + np.arange(T)
            keys = np.arange(ctx + T)
            ok = keys[None] <= pos[:, None]
            if window >= 0:
                ok &= keys[None] >= pos[:, None] - window
            qq = torch.from_numpy(q[b].astype(np.float64)).permute(1, 0, 2)                      # (Hq, T, D)
            kk = torch.from_numpy(np.repeat(K, G, axis=1).astype(np.float64)).permute(1, 0, 2)    # (Hq, n, D)
            vv = torch.from_numpy(np.repeat(V, G, axis=1).astype(np.float64)).permute(1, 0, 2)
            ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=torch.from_numpy(ok))
            assert np.allclose(pre[b], ref.permute(1, 0, 2).numpy())


def test_inactive_sequence_is_zero():
    cache, table = make(2, 10, 1, 9)
    out = decode_attention(q_rows((2, 1, 128), 1), cache, table, np.array([0, 10]))
    assert not out[0].any() and out[1].any()
