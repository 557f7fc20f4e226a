"""CPU replay of decode_kernel's work split (nanochat_amd/csrc/attention.hip: chunks cut at multiples of 64 pages; the
per-work-group prefixes over sequences of full and partial chunks; full chunks numbered first, then partial ones;
item k to work-group k % G, wave (k / G) % 4; partial slot = the chunk's unit-order index; meta written by each unit's
chunk 0) for many shapes: every (unit, page) is attended exactly once, by an item whose page range depends on nothing
but the unit's own length; partial slots stay inside the workspace bound (item_bound); meta names exactly a unit's
chunks, in order; work-groups' page loads differ by at most about one chunk."""
import numpy as np
import pytest

PAGE = 16
WAVES = 4
SPLIT = 64


def unit_pages(L, window, max_len):
    if L <= 0 or L > max_len:
        return 0, 0
    p = L - 1
    begin = max(p - window, 0) if window >= 0 else 0
    return p // PAGE + 1 - begin // PAGE, begin // PAGE


def unit_split(pg0, n):
    """(chunks, lead partial, full, partial) of logical pages [pg0, pg0 + n)."""
    if n <= 0:
        return 0, 0, 0, 0
    e = pg0 + n
    nch = (e - 1) // SPLIT - pg0 // SPLIT + 1
    lead, trail = int(pg0 % SPLIT != 0), int(e % SPLIT != 0)
    npart = int(lead or trail) if nch == 1 else lead + trail
    return nch, lead, nch - npart, npart


def item_bound(B, hkv, max_len, window):
    n = -(-max_len // PAGE)
    if window >= 0:
        n = min(n, window // PAGE + 2)
    return B * hkv * (-(-n // SPLIT) + 1)


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
    seen, partials, meta, load = {}, {}, {}, np.zeros(G, np.int64)
    for wg in range(G):
        for wave in range(WAVES):
            for k in range(wg + G * wave, N, 4 * G):
                if k < NF:
                    b = max(i for i in range(B) if cf[i] <= k)
                    nch, lead, nfull, npart = split[b]
                    kvh, jf = divmod(k - cf[b], nfull)
                    j = jf + lead
                else:
                    k2 = k - NF
                    b = max(i for i in range(B) if cp[i] <= k2)
                    nch, lead, nfull, npart = split[b]
                    kvh, jp = divmod(k2 - cp[b], npart)
                    j = 0 if nch == 1 or (lead and jp == 0) else nch - 1
                n, pg0 = units[b]
                chunk = pg0 // SPLIT + j
                first, last = max(pg0, chunk * SPLIT), min(pg0 + n, (chunk + 1) * SPLIT)
                assert first < last
                assert (last - first == SPLIT) == (k < NF)
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
                if j == 0:
                    meta[u] = (slot, nch)
    for b, (n, pg0) in enumerate(units):
        for kvh in range(hkv):
            for lp in range(pg0, pg0 + n):
                assert (b, kvh, lp) in seen
            if n:
                first, count = meta[b * hkv + kvh]
                if count > 1:
                    assert [partials[first + j] for j in range(count)] == [(b * hkv + kvh, j) for j in range(count)]
    assert len(seen) == sum(hkv * n for n, _ in units)
    if N >= G:   # every work-group has an item: loads differ by at most about one chunk of each kind
        assert load.max() - load.min() <= 2 * SPLIT * -(-N // (4 * G)) + SPLIT
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
