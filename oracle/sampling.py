"""The decoder's token choice — test infrastructure only.

Restates model/kernels/decode.cu:90-105 (choice_key, gumbel), 170-229 (the ARGMAX epilogue with CHOICE) and
361-411 (k_nucleus), as the build's choose_kernel computes them:

    temperature 0:          the largest logit among the allowed rows, ties to the lowest row
    temperature T > 0:      the largest z / T + g(seed, i, row), z = c tanh(s / c), g Gumbel noise
    T > 0 and top_p < 1:    the same over the nucleus: keep e >= e*, the least e with C(e) > (1 - top_p) sum e,
                            C(x) = sum of e <= x, e = exp(z / T - max z / T) (transformers' TopPLogitsWarper)
    alternative:            the best allowed row but `lazy` (none, -1, for nucleus slots)

Gumbel noise: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11;
the Random123 constants) at counter (row, i, 0, 0) with key (seed mod 2^32, seed >> 32); the first two output
words give r = (x0 2^32 + x1) >> 12, u = (2 r + 1) 2^-53, g = -log(-log(u)) in float64, rounded to float32.

The device takes the nucleus threshold in exact fixed point (csrc/decoder.hip:nucleus_cut): a row weighs
round(e 2^38) as an integer, and e* is the least e whose rows at or below it weigh more than (1 - top_p) of the
total, with the drop floor((1 - top_p) total) capped at total - 1. `nucleus_cut_fixed` restates that rule by sorting;
it differs from the float64 rule of `nucleus_keep` only for rows within about 2^-38 of the largest e of the
threshold's mass.

Pinned by tests/test_oracle_sampling.py: Philox against the Random123 known-answer vectors; the key order
against IEEE order on random and special floats (largest score wins, ties to the lowest row); greedy choice
against numpy argmax; Gumbel-max sampling frequencies against softmax(z / T) (chi-square); the nucleus against a
float64 sort-and-cumsum restatement of TopPLogitsWarper; the fixed-point cut against that float64 rule, against a
brute-force search over every candidate threshold on small inputs, and on its special cases (top_p <= 0 keeps the
maximum rows, equal rows are kept together, no allowed row keeps nothing).
"""
import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF


def philox4x32_10(counter, key):
    """counter (4 ints), key (2 ints) -> 4 uint32 words (Python ints)."""
    c0, c1, c2, c3 = (int(x) & MASK32 for x in counter)
    k0, k1 = (int(x) & MASK32 for x in key)
    for r in range(10):
        if r:
            k0 = (k0 + W0) & MASK32
            k1 = (k1 + W1) & MASK32
        p0, p1 = M0 * c0, M1 * c2
        c0, c1, c2, c3 = ((p1 >> 32) ^ c1 ^ k0) & MASK32, p1 & MASK32, ((p0 >> 32) ^ c3 ^ k1) & MASK32, p0 & MASK32
    return c0, c1, c2, c3


def philox4x32_10_rows(rows, i, seed):
    """Vectorized over counter word 0: rows (n,) ints at counter (row, i, 0, 0), key from seed -> (n, 4) uint64."""
    c0 = np.asarray(rows, np.uint64) & np.uint64(MASK32)
    c1 = np.full_like(c0, np.uint64(int(i) & MASK32))
    c2 = np.zeros_like(c0)
    c3 = np.zeros_like(c0)
    k0, k1 = np.uint64(int(seed) & MASK32), np.uint64((int(seed) >> 32) & MASK32)
    m32 = np.uint64(MASK32)
    for r in range(10):
        if r:
            k0 = (k0 + np.uint64(W0)) & m32
            k1 = (k1 + np.uint64(W1)) & m32
        p0 = np.uint64(M0) * c0
        p1 = np.uint64(M1) * c2
        c0, c1, c2, c3 = ((p1 >> np.uint64(32)) ^ c1 ^ k0) & m32, p1 & m32, ((p0 >> np.uint64(32)) ^ c3 ^ k1) & m32, \
            p0 & m32
    return np.stack([c0, c1, c2, c3], axis=-1)


def gumbel(seed, i, rows):
    """Gumbel noise (float32) of rows at generated position i under seed."""
    x = philox4x32_10_rows(rows, i, seed)
    r = ((x[:, 0] << np.uint64(32)) | x[:, 1]) >> np.uint64(12)
    u = np.ldexp(2.0 * r.astype(np.float64) + 1.0, -53)
    return (-np.log(-np.log(u))).astype(np.float32)


def choice_key(score, row):
    """The 64-bit order key of (score float32, row): larger key = larger score, then lower row."""
    bits = np.asarray(score, np.float32).view(np.uint32).astype(np.uint64)
    neg = (bits & np.uint64(0x80000000)) != 0
    ordered = np.where(neg, (~bits) & np.uint64(MASK32), bits | np.uint64(0x80000000))
    return (ordered << np.uint64(32)) | (np.uint64(MASK32) - np.asarray(row, np.uint64))


def key_row(key):
    """A key's row, -1 for key 0 (nothing chosen)."""
    return int(np.int32(np.uint32(MASK32 - (int(key) & MASK32))))


def allowed_rows(vocab, mask_words):
    """uint32 words (vocab / 32) -> bool (vocab,): bit t % 32 of word t // 32."""
    words = np.asarray(mask_words, np.uint32)
    return ((words[np.arange(vocab) // 32] >> (np.arange(vocab) % 32).astype(np.uint32)) & 1).astype(bool)


def capped(logits, softcap):
    s = np.asarray(logits, np.float32)
    return (np.float32(softcap) * np.tanh(s / np.float32(softcap))).astype(np.float32)


def nucleus_keep(z, temperature, top_p, allowed):
    """The kept rows of TopPLogitsWarper over e = exp(z / T - max), float64, by sorting: the smallest rows whose
    cumulative sum stays <= (1 - top_p) sum are dropped; ties at the threshold are kept together."""
    zt = np.where(allowed, z.astype(np.float64) / temperature, -np.inf)
    e = np.exp(zt - np.max(zt))
    drop = (1.0 - top_p) * e.sum()
    order = np.sort(e)
    below = np.cumsum(order)
    # the least e* with C(e*) > drop: C(x) = sum of e <= x
    idx = np.searchsorted(below, drop, side="right")
    least = order[min(idx, len(order) - 1)]
    return (e >= least) & allowed, e


NUCLEUS_FRAC_BITS = 38


def nucleus_cut_fixed(e, top_p):
    """The device's nucleus threshold: e (float32, in [0, 1], 0 for rows not allowed) and top_p -> the uint32 IEEE
    pattern of e*. Rows with e >= e* and a positive weight form the nucleus; 0xFFFFFFFF when no row has weight."""
    e = np.asarray(e, np.float32)
    weight = np.floor(e.astype(np.float64) * 2.0 ** NUCLEUS_FRAC_BITS + 0.5).astype(np.uint64)
    total = int(weight.sum(dtype=np.uint64))
    if total == 0:
        return MASK32
    keep_out = (1.0 - float(np.float32(top_p))) * float(total)
    drop = total - 1 if keep_out >= float(total - 1) else int(keep_out)
    keys, which = np.unique(e.view(np.uint32), return_inverse=True)   # ascending patterns: ascending e (e >= 0)
    per_key = np.zeros(keys.size, np.uint64)
    np.add.at(per_key, which, weight)
    at_or_below = np.cumsum(per_key, dtype=np.uint64)
    return int(keys[np.argmax(at_or_below > np.uint64(drop))])


def choose(logits, *, temperature=0.0, top_p=1.0, seed=0, gen=0, allow=None, lazy=-1, softcap=15.0):
    """One slot's (token, alternative) from fp32 logits, as the device chooses them. allow: uint32 mask words or
    None (every row). The nucleus threshold is taken in float64 (the device's fp32 bisection can differ only for
    rows within fp32 rounding of the threshold)."""
    s = np.asarray(logits, np.float32)
    vocab = s.shape[0]
    rows = np.arange(vocab)
    ok = np.ones(vocab, bool) if allow is None else allowed_rows(vocab, allow)
    if temperature > 0:
        z = capped(s, softcap)
        score = (z / np.float32(temperature)).astype(np.float32) + gumbel(seed, gen, rows)
        score = score.astype(np.float32)
        if top_p < 1:
            keep, _ = nucleus_keep(z, temperature, top_p, ok)
            keys = np.where(keep, choice_key(score, rows), np.uint64(0))
            return key_row(keys.max()), -1
    else:
        score = s
    keys = np.where(ok, choice_key(score, rows), np.uint64(0))
    best = keys.max()
    alt_keys = np.where(rows != lazy, keys, np.uint64(0))
    return key_row(best), key_row(alt_keys.max())
