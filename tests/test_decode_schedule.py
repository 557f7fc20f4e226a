"""CPU replay of decode_kernel's work split (nanochat_amd/csrc/attention.hip: the per-work-group item prefix over
sequences, items (sequence, KV head, chunk) taken round-robin by W waves, chunks cut at multiples of 64 pages,
partial slot = item index, meta written by each unit's chunk 0) for many shapes: every (unit, page) is attended exactly
once, by an item whose page range depends on nothing but the unit's own length; partial slots stay inside the
workspace bound (item_bound); meta names exactly a unit's items, in chunk order."""
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


def unit_chunks(pg0, n):
    return (pg0 + n - 1) // SPLIT - pg0 // SPLIT + 1 if n > 0 else 0


def item_bound(B, hkv, max_len, window):
    n = -(-max_len // PAGE)
    if window >= 0:
        n = min(n, window // PAGE + 2)
    return B * hkv * (-(-n // SPLIT) + 1)


def replay(seq_lens, hkv, workers, window, max_len):
    """Returns {(b, kvh, logical page): (first, last) of the item that attended it} and checks the bookkeeping."""
    B = len(seq_lens)
    units = [unit_pages(L, window, max_len) for L in seq_lens]
    cum = np.zeros(B + 1, np.int64)
    for b in range(B):
        cum[b + 1] = cum[b] + hkv * unit_chunks(units[b][1], units[b][0])
    N = int(cum[B])
    W = min(workers, N)
    seen, partials, meta = {}, {}, {}
    grid = -(-workers // WAVES)
    for wid in range(grid * WAVES):
        if wid >= W:
            continue
        for it in range(wid, N, W):
            b = max(i for i in range(B) if cum[i] <= it)
            n, pg0 = units[b]
            nch = unit_chunks(pg0, n)
            local = it - cum[b]
            kvh, j = divmod(local, nch)
            chunk = pg0 // SPLIT + j
            first, last = max(pg0, chunk * SPLIT), min(pg0 + n, (chunk + 1) * SPLIT)
            assert first < last
            for lp in range(first, last):
                key = (b, kvh, lp)
                assert key not in seen, key
                seen[key] = (first, last)
            u = b * hkv + kvh
            if nch > 1:
                assert 0 <= it < item_bound(B, hkv, max_len, window)
                assert it not in partials
                partials[it] = (u, j)
            if j == 0:
                meta[u] = (it, nch)
    for b, (n, pg0) in enumerate(units):
        for kvh in range(hkv):
            for lp in range(pg0, pg0 + n):
                assert (b, kvh, lp) in seen
            if n:
                first, count = meta[b * hkv + kvh]
                if count > 1:
                    assert [partials[first + j] for j in range(count)] == [(b * hkv + kvh, j) for j in range(count)]
    assert len(seen) == sum(hkv * n for n, _ in units)
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
