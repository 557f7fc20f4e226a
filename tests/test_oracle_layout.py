"""Pins oracle/layout.py: the page maps are bijections, a random-permutation block table gathers the same
bytes as the identity table, scatter-then-gather returns the written codes, and a Python-loop brute force."""
import numpy as np

from oracle.layout import K_OFF, PAGE, V_OFF, PagedCache, k_offset, v_offset
from oracle.numerics import bf16_round
from oracle.quant import quantize_rows


def test_maps_are_bijections():
    assert np.array_equal(np.sort(K_OFF.ravel()), np.arange(2048))
    assert np.array_equal(np.sort(V_OFF.ravel()), np.arange(2048))


def test_mfma_lane_chunks():
    # K: lane l = g*16 + slot reads dims g*32 + h*16 .. +15 as the 16 bytes at h*1024 + l*16
    for slot in range(16):
        for g in range(4):
            for h in range(2):
                dims = g * 32 + h * 16 + np.arange(16)
                assert np.array_equal(K_OFF[slot, dims], h * 1024 + (g * 16 + slot) * 16 + np.arange(16))
    # V: lane l = g*16 + r holds, for tile t, slots 4g..4g+3 of dim 16t + r as one dword
    for r in range(16):
        for g in range(4):
            for t in range(8):
                offs = [v_offset(4 * g + kk, 16 * t + r) for kk in range(4)]
                base = (t // 4) * 1024 + (g * 16 + r) * 16 + (t % 4) * 4
                assert offs == [base, base + 1, base + 2, base + 3]


def fill(table, B, n, hkv, seed):
    rng = np.random.default_rng(seed)
    k = bf16_round(rng.standard_normal((B, n, hkv, 128)).astype(np.float32))
    v = bf16_round(rng.standard_normal((B, n, hkv, 128)).astype(np.float32))
    cache = PagedCache(table.size, hkv)
    for b in range(B):
        cache.append(table, b, np.arange(n), k[b], v[b])
    return cache, k, v


def test_permuted_table_gathers_identical_bytes():
    B, n, hkv = 3, 70, 2
    mp = (n + PAGE - 1) // PAGE
    ident = np.arange(B * mp, dtype=np.int32).reshape(B, mp)
    perm = np.random.default_rng(5).permutation(B * mp).astype(np.int32).reshape(B, mp)
    c1, _, _ = fill(ident, B, n, hkv, 0)
    c2, _, _ = fill(perm, B, n, hkv, 0)
    for b in range(B):
        for x, y in zip(c1.gather(ident, b, n), c2.gather(perm, b, n)):
            assert np.array_equal(x, y)


def test_scatter_gather_round_trip_and_brute_force():
    B, n, hkv = 2, 37, 3
    mp = (n + PAGE - 1) // PAGE
    table = np.random.default_rng(6).permutation(B * mp).astype(np.int32).reshape(B, mp)
    cache, k, v = fill(table, B, n, hkv, 1)
    for b in range(B):
        kc, ks, vc, vs = cache.gather(table, b, n)
        wk, wks = quantize_rows(k[b])
        wv, wvs = quantize_rows(v[b])
        assert np.array_equal(kc, wk) and np.array_equal(ks, wks)
        assert np.array_equal(vc, wv) and np.array_equal(vs, wvs)
        for p in range(n):                       # brute force through the scalar offset maps
            page, slot = table[b, p // PAGE], p % PAGE
            for h in range(hkv):
                for d in range(0, 128, 9):
                    assert cache.k[page, h, k_offset(slot, d)] == wk[p, h, d]
                    assert cache.v[page, h, v_offset(slot, d)] == wv[p, h, d]
                assert cache.ks[page, h, slot] == wks[p, h]
