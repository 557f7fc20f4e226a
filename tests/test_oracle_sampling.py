"""Pins of oracle/sampling.py: Philox against Random123's known answers, the choice order against IEEE order and
numpy, Gumbel-max against softmax frequencies, the nucleus against a sort-based TopPLogitsWarper."""
import numpy as np
import pytest

from oracle import sampling

# Random123 kat_vectors, philox4x32 with 10 rounds: (counter, key) -> output
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,expected", KAT)
def test_philox_known_answers(counter, key, expected):
    assert sampling.philox4x32_10(counter, key) == expected


def test_philox_vectorized_matches_scalar():
    seed = (0x12345678 << 32) | 0x9ABCDEF0
    rows = np.array([0, 1, 77, 65535, 2 ** 31 + 5])
    out = sampling.philox4x32_10_rows(rows, 41, seed)
    for r, words in zip(rows, out):
        assert tuple(int(w) for w in words) == sampling.philox4x32_10((int(r), 41, 0, 0), (0x9ABCDEF0, 0x12345678))


def test_gumbel_is_standard_gumbel():
    g = sampling.gumbel(7, 3, np.arange(200000)).astype(np.float64)
    assert abs(g.mean() - 0.5772156649) < 0.01          # Euler-Mascheroni
    assert abs(g.var() - np.pi ** 2 / 6) < 0.03
    assert np.isfinite(g).all()


def test_choice_key_orders_like_ieee():
    rng = np.random.default_rng(0)
    special = np.array([-np.inf, -3e38, -1.0, -1e-40, -0.0, 0.0, 1e-40, 1.0, 3e38, np.inf], np.float32)
    scores = np.concatenate([special, rng.standard_normal(500).astype(np.float32) * 10])
    keys = sampling.choice_key(scores, np.zeros(len(scores), np.int64))
    for i in range(len(scores)):
        for j in range(len(scores)):
            if scores[i] > scores[j]:
                assert keys[i] > keys[j]
    # equal scores: the lower row wins; a key's row comes back
    k = sampling.choice_key(np.float32([1.5, 1.5]), np.array([3, 9]))
    assert k[0] > k[1] and sampling.key_row(k[0]) == 3 and sampling.key_row(k[1]) == 9
    assert sampling.key_row(0) == -1


def test_greedy_is_argmax_with_masks():
    rng = np.random.default_rng(1)
    for _ in range(20):
        s = rng.standard_normal(1024).astype(np.float32)
        s[rng.integers(0, 1024, 3)] = s.max()             # exact ties: the lowest row
        tok, alt = sampling.choose(s, lazy=int(np.argmax(s)))
        assert tok == int(np.argmax(s))
        masked = s.copy()
        masked[tok] = -np.inf
        assert alt == int(np.argmax(masked))
        allowed = rng.random(1024) < 0.3
        words = np.packbits(allowed, bitorder="little").view("<u4")
        tok, _ = sampling.choose(s, allow=words)
        assert tok == int(np.argmax(np.where(allowed, s, -np.inf)))
    none, none_alt = sampling.choose(np.zeros(64, np.float32), allow=np.zeros(2, np.uint32))
    assert none == -1 and none_alt == -1


def test_gumbel_max_samples_softmax():
    """Frequencies of Gumbel-max choices over many positions match softmax(z / T) (chi-square, 8 categories)."""
    s = np.float32([2.0, 1.5, 1.0, 0.5, 0.0, -0.5, -1.0, -2.0])
    T, cap = 0.7, 15.0
    z = sampling.capped(s, cap).astype(np.float64)
    p = np.exp(z / T - np.max(z / T))
    p /= p.sum()
    n = 20000
    counts = np.zeros(8)
    for i in range(n):
        tok, _ = sampling.choose(s, temperature=T, seed=11, gen=i, softcap=cap)
        counts[tok] += 1
    chi2 = np.sum((counts - n * p) ** 2 / (n * p))
    assert chi2 < 24.3  # 7 degrees of freedom, p = 0.001


def test_nucleus_matches_sorted_cumsum():
    rng = np.random.default_rng(2)
    for top_p in (0.5, 0.9, 0.99):
        s = (rng.standard_normal(4096) * 3).astype(np.float32)
        z = sampling.capped(s, 15.0)
        keep, e = sampling.nucleus_keep(z, 0.8, top_p, np.ones(4096, bool))
        # TopPLogitsWarper: sort descending, keep the smallest prefix whose mass reaches top_p
        order = np.argsort(-e, kind="stable")
        probs = e[order] / e.sum()
        mass_before = np.cumsum(probs) - probs
        expected = np.zeros(4096, bool)
        expected[order[mass_before < top_p]] = True
        assert (keep == expected).all()
        tok, alt = sampling.choose(s, temperature=0.8, top_p=top_p, seed=5, gen=2)
        assert keep[tok] and alt == -1


def brute_cut(e, top_p):
    """Every candidate threshold tried in turn: the least e_i whose rows at or below it weigh more than the drop."""
    w = [int(np.floor(float(x) * 2.0 ** 38 + 0.5)) for x in np.asarray(e, np.float32)]
    total = sum(w)
    if total == 0:
        return None
    keep_out = (1.0 - float(np.float32(top_p))) * float(total)
    drop = min(total - 1, int(keep_out)) if keep_out < float(total - 1) else total - 1
    best = None
    for x in e:
        mass = sum(wj for ej, wj in zip(e, w) if ej <= x)
        if mass > drop and (best is None or x < best):
            best = x
    return best


def kept_by_cut(e, cut):
    e = np.asarray(e, np.float32)
    return (e.view(np.uint32) >= np.uint32(cut)) & (np.floor(e.astype(np.float64) * 2.0 ** 38 + 0.5) > 0)


def test_fixed_point_cut_matches_the_float64_rule():
    """Away from a mass boundary (continuous random logits) the integer rule keeps exactly TopPLogitsWarper's rows."""
    rng = np.random.default_rng(7)
    for vocab, T, top_p, spread in ((4096, 0.8, 0.5, 3), (65536, 1.0, 0.9, 2), (50000, 0.6, 0.99, 4),
                                    (1000, 1.3, 0.1, 1), (32768, 0.7, 0.95, 6)):
        z = sampling.capped((rng.standard_normal(vocab) * spread).astype(np.float32), 15.0)
        allowed = rng.random(vocab) < 0.9
        keep, e64 = sampling.nucleus_keep(z, T, top_p, allowed)
        zt = np.where(allowed, z / np.float32(T), -np.inf).astype(np.float32)
        e = np.where(allowed, np.exp(zt - zt[allowed].max()), 0).astype(np.float32)
        cut = sampling.nucleus_cut_fixed(e, top_p)
        assert (kept_by_cut(e, cut) == keep).all(), (vocab, top_p)


def test_fixed_point_cut_against_brute_force():
    rng = np.random.default_rng(8)
    for trial in range(400):
        n = int(rng.integers(1, 9))
        e = rng.choice([0.0, 1e-13, 0.03, 0.25, 0.5, 0.5, 0.7, 1.0], n).astype(np.float32)
        e[int(rng.integers(n))] = 1.0                           # the largest row has e = 1
        top_p = float(rng.choice([0.0, 0.1, 0.3, 0.5, 0.75, 0.9, 0.999, rng.random()]))
        want = brute_cut(e, top_p)
        got = sampling.nucleus_cut_fixed(e, top_p)
        assert got == np.float32(want).view(np.uint32), (e, top_p)


def test_fixed_point_cut_special_cases():
    e = np.array([0.2, 1.0, 0.0, 1.0, 0.5], np.float32)
    assert kept_by_cut(e, sampling.nucleus_cut_fixed(e, 0.0)).tolist() == [False, True, False, True, False]
    # equal rows are kept or dropped together: the two 0.5 rows are 1/3 of the mass, so they go when at least 1/3 may
    # be dropped (top_p <= 2/3) and both stay otherwise
    e = np.array([0.5, 1.0, 0.5, 1.0], np.float32)
    for top_p, kept in ((0.6, [False, True, False, True]), (0.66, [False, True, False, True]),
                        (0.67, [True] * 4), (0.7, [True] * 4)):
        assert kept_by_cut(e, sampling.nucleus_cut_fixed(e, top_p)).tolist() == kept, top_p
    # no allowed row: nothing has weight, nothing is kept
    assert sampling.nucleus_cut_fixed(np.zeros(64, np.float32), 0.9) == 0xFFFFFFFF
    # a row under 2^-39 of the largest weighs nothing and is never kept, even at top_p close to 1
    e = np.array([1.0, 2.0 ** -41], np.float32)
    assert kept_by_cut(e, sampling.nucleus_cut_fixed(e, 0.999999)).tolist() == [True, False]
