"""CPU replay of decode_kernel's work split (nanochat_amd/csrc/attention.hip: chunks cut at multiples of 64 pages, or of
16 pages for a unit of at most 67 pages, a last piece under 4 pages joined to the one before it (checked against a
from-scratch cut of the page range); the
per-work-group prefixes over sequences of full and partial chunks; full chunks numbered first (a unit's rotated by its
index), then partial ones (every chunk of a unit of 16-page chunks);
item k to work-group k % G, wave (k / G) % 4; partial slot = the chunk's unit-order index; the unit's chunks counted
in arrived[u], the last to finish merging slots slot - j .. + nch) for many shapes: every (unit, page) is attended
exactly once, by an item whose page range depends on nothing but the unit's own length; partial slots stay inside the
workspace bound (item_bound); every chunk of a multi-chunk unit names the same first slot, the unit's chunks fill it in
order and arrive exactly nch times (so one merge runs and the count returns to zero); the sequences left with no item
are exactly those the kernel fills with zero or NaN rows; work-groups' page loads differ by at most about one chunk."""
import numpy as np
import pytest

PAGE = 16
WAVES = 4
SPLIT = 64
SHORT = 16


def unit_pages(L, window, max_len):
    if L <= 0 or L > max_len:
        return 0, 0
    p = L - 1
    begin = max(p - window, 0) if window >= 0 else 0
    return p // PAGE + 1 - begin // PAGE, begin // PAGE


MIN_TAIL = 4
SHORT_UNIT = SPLIT + MIN_TAIL - 1   # a unit of at most this many pages is cut every 16 pages


def cut(n):
    return SHORT if n <= SHORT_UNIT else SPLIT


def chunk_ranges(pg0, n):
    """Logical page ranges of a unit's chunks, from first principles: cut [pg0, pg0 + n) at every multiple of 64 pages
    (16 if n <= 67), then join a last piece shorter than 4 pages to the one before it."""
    if n <= 0:
        return []
    e, S = pg0 + n, cut(n)
    cuts = [pg0] + list(range((pg0 // S + 1) * S, e, S)) + [e]
    pieces = [(a, b) for a, b in zip(cuts, cuts[1:])]
    if len(pieces) >= 2 and pieces[-1][1] - pieces[-1][0] < MIN_TAIL:
        pieces[-2:] = [(pieces[-2][0], e)]
    return pieces


def unit_split(pg0, n):
    """(chunks, chunk 0 partial, full, partial) of logical pages [pg0, pg0 + n), as the kernel computes them."""
    if n <= 0:
        return 0, 0, 0, 0
    S = cut(n)
    e, c0 = pg0 + n, pg0 // S
    pieces = (e - 1) // S - c0 + 1
    tail = e - max(pg0, ((e - 1) // S) * S)
    nch = pieces - int(pieces >= 2 and tail < MIN_TAIL)
    if S == SHORT:
        return nch, 1, 0, nch
    size0 = (e if nch == 1 else (c0 + 1) * S) - pg0
    sizel = e - (c0 + nch - 1) * S
    p0 = int(size0 < S)
    npart = p0 + int(nch > 1 and sizel < S)
    return nch, p0, nch - npart, npart


def chunk_pages(pg0, n, nch, j):
    S = cut(n)
    c = pg0 // S + j
    return (pg0 if j == 0 else c * S), (pg0 + n if j == nch - 1 else (c + 1) * S)


def item_bound(B, hkv, max_len, window):
    n = -(-max_len // PAGE)
    if window >= 0:
        n = min(n, window // PAGE + 2)
    return B * hkv * max(-(-n // SPLIT) + 1, -(-min(n, SHORT_UNIT) // SHORT) + 1)


def replay(seq_lens, hkv, workers, window, max_len):
    """Returns {(b, kvh, logical page): (first, last) of the item that attended it} and checks the bookkeeping."""
    B = len(seq_lens)
    units = [unit_pages(L, window, max_len) for L in seq_lens]
    split = [unit_split(pg0, n) for n, pg0 in units]
    cf, cp = np.zeros(B + 1, np.int64), np.zeros(B + 1, np.int64)
    for b in range(B):
        cf[b + 1] = cf[b] + hkv * split[b][2]
        cp[b + 1] = cp[b] + hkv * split[b][3]
    NF, N = int(cf[B]), int(cf[B] + cp[B])
    G = -(-min(workers, 4 * item_bound(B, hkv, max_len, window)) // WAVES)
    seen, partials, first_slot, arrived, load = {}, {}, {}, {}, np.zeros(G, np.int64)
    for wg in range(G):
        for wave in range(WAVES):
            for k in range(wg + G * wave, N, 4 * G):
                if k < NF:
                    b = max(i for i in range(B) if cf[i] <= k)
                    nch, p0, nfull, npart = split[b]
                    kvh, jf = divmod(k - cf[b], nfull)
                    rot = (b * hkv + kvh + (int(cf[b]) + kvh * nfull) // G) % nfull   # rotated by index and round
                    j = (jf + rot) % nfull + p0
                else:
                    k2 = k - NF
                    b = max(i for i in range(B) if cp[i] <= k2)
                    nch, p0, nfull, npart = split[b]
                    kvh, jp = divmod(k2 - cp[b], npart)
                    j = jp if cut(units[b][0]) == SHORT else (0 if p0 and jp == 0 else nch - 1)
                n, pg0 = units[b]
                first, last = chunk_pages(pg0, n, nch, j)
                assert (first, last) == chunk_ranges(pg0, n)[j]
                assert 0 < last - first <= SPLIT + MIN_TAIL - 1
                assert (last - first >= SPLIT) == (k < NF)
                load[wg] += last - first
                for lp in range(first, last):
                    key = (b, kvh, lp)
                    assert key not in seen, key
                    seen[key] = (first, last)
                slot = int(cf[b] + cp[b]) + kvh * nch + j
                u = b * hkv + kvh
                if nch > 1:
                    assert 0 <= slot < item_bound(B, hkv, max_len, window)
                    assert slot not in partials
                    partials[slot] = (u, j)
                    assert first_slot.setdefault(u, slot - j) == slot - j
                    arrived[u] = arrived.get(u, 0) + 1
    for b, (n, pg0) in enumerate(units):
        # no item: exactly the sequences decode_fill_rows finds by their empty chunk ranges
        assert (n == 0) == (cf[b + 1] == cf[b] and cp[b + 1] == cp[b])
        nch = split[b][0]
        for kvh in range(hkv):
            u = b * hkv + kvh
            for lp in range(pg0, pg0 + n):
                assert (b, kvh, lp) in seen
            if nch > 1:
                assert arrived[u] == nch
                assert [partials[first_slot[u] + j] for j in range(nch)] == [(u, j) for j in range(nch)]
            else:
                assert u not in arrived
    assert len(seen) == sum(hkv * n for n, _ in units)
    if N >= G:   # every work-group has an item: loads differ by at most about one chunk of each kind
        assert load.max() - load.min() <= 2 * (SPLIT + MIN_TAIL) * -(-N // (4 * G)) + SPLIT + MIN_TAIL
    return seen


@pytest.mark.parametrize("seed", range(40))
def test_schedule_covers_every_page_once(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 40))
    hkv = int(rng.choice([1, 2, 4, 8, 10]))
    max_len = int(rng.integers(1, 5000))
    lens = rng.integers(-2, max_len + 1, B)
    if seed % 7 == 0:
        lens[rng.integers(0, B)] = max_len + 5   # longer than the launch's bound: no items
    window = int(rng.choice([-1, 0, 15, 16, 100, 700, 1500]))
    workers = int(rng.integers(1, 70))
    replay(lens, hkv, workers, window, max_len)


def test_more_workers_than_items():
    replay([1, 2, 0, 17], 4, 4096, -1, 32)
    replay([5], 1, 6, -1, 16)


def test_a_sequences_split_does_not_depend_on_the_batch():
    """The items of a sequence of length L (its chunk ranges) are the same alone, in any batch, at any place in it,
    for any worker count."""
    rng = np.random.default_rng(1)
    for window in (-1, 300, 2000):
        for L in (1, 16, 1024, 1025, 1040, 2049, 5000):
            alone = replay([L], 2, 3, window, 6000)
            mine = {k[1:]: v for k, v in alone.items()}
            for trial in range(4):
                others = list(rng.integers(0, 6000, int(rng.integers(1, 9))))
                at = int(rng.integers(0, len(others) + 1))
                lens = others[:at] + [L] + others[at:]
                got = replay(lens, 2, int(rng.integers(1, 50)), window, 6000)
                assert {k[1:]: v for k, v in got.items() if k[0] == at} == mine


@pytest.mark.parametrize("window", [-1, 0, 100, 1071, 1072, 1500])
def test_short_and_long_cuts_at_their_boundary(window):
    """Units of 1..70 pages either side of the 67-page boundary (16-page cuts up to it, 64-page cuts past it), alone
    and in a batch with longer sequences, every page once, the chunk sizes as cut."""
    for L in list(range(1, 70 * PAGE + 1, 7)) + [1056, 1057, 1072, 1073, 1088, 1089]:
        n, pg0 = unit_pages(L, window, 8000)
        pieces = chunk_ranges(pg0, n)
        if n <= SHORT_UNIT:
            assert all(b - a <= SHORT + MIN_TAIL - 1 for a, b in pieces)
            assert len(pieces) <= -(-n // SHORT) + 1
        else:
            assert all(b - a <= SPLIT + MIN_TAIL - 1 for a, b in pieces)
        alone = replay([L], 3, 8, window, 8000)
        got = replay([5000, L, 3000], 3, 40, window, 8000)
        assert {k[1:]: v for k, v in got.items() if k[0] == 1} == {k[1:]: v for k, v in alone.items()}
