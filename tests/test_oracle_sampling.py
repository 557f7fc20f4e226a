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
