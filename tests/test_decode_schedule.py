"""CPU replay of decode_kernel's work split (nanochat_amd/csrc/attention.hip: the per-work-group page prefix,
each wave's run [wid P / W, (wid + 1) P / W), the unit walk, partial slots u + wid and meta) for many shapes:
every (unit, page) is attended exactly once, slots stay inside the workspace, and meta names exactly the waves
that wrote a unit's partials."""
import numpy as np
import pytest

PAGE = 16
WAVES = 4


def unit_pages(L, window, max_pages):
    if L <= 0 or L > max_pages * PAGE:
        return 0, 0
    p = L - 1
    begin = max(p - window, 0) if window >= 0 else 0
    return p // PAGE + 1 - begin // PAGE, begin // PAGE


def replay(seq_lens, hkv, workers, window, max_pages):
    B = len(seq_lens)
    npg = [unit_pages(L, window, max_pages) for L in seq_lens]
    cum = np.zeros(B + 1, np.int64)
    for b in range(B):
        cum[b + 1] = cum[b] + hkv * npg[b][0]
    P = int(cum[B])
    W = min(workers, P)
    seen, partials, meta = {}, {}, {}
    worker_of = lambda x: ((x + 1) * W - 1) // P
    grid = -(-workers // WAVES)
    for wid in range(grid * WAVES):
        if wid >= W:
            continue
        s, e = wid * P // W, (wid + 1) * P // W
        assert s < e   # W <= P: every run holds at least one page
        b = max(i for i in range(B) if cum[i] <= s)
        while s < e and b < B:
            np_, pg0 = npg[b]
            if np_ == 0 or cum[b + 1] <= s:
                b += 1
                continue
            kvh = (s - cum[b]) // np_
            us = cum[b] + kvh * np_
            ue = us + np_
            seg_end = min(e, ue)
            for lp in range(pg0 + s - us, pg0 + seg_end - us):
                key = (b, kvh, lp)
                assert key not in seen, key
                seen[key] = wid
            w0, w1 = worker_of(us), worker_of(ue - 1)
            u = b * hkv + kvh
            if w0 != w1:
                slot = u + wid
                assert 0 <= slot < B * hkv + W
                assert slot not in partials
                partials[slot] = u
            if wid == w0:
                meta[u] = (u + w0, w1 - w0 + 1)
            s = seg_end
    # coverage: every page of every active unit exactly once
    for b, (np_, pg0) in enumerate(npg):
        for kvh in range(hkv):
            for lp in range(pg0, pg0 + np_):
                assert (b, kvh, lp) in seen
            if np_:
                first, count = meta[b * hkv + kvh]
                if count > 1:
                    assert [partials.get(first + j) for j in range(count)] == [b * hkv + kvh] * count
    assert len(seen) == P


@pytest.mark.parametrize("seed", range(40))
def test_schedule_covers_every_page_once(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 40))
    hkv = int(rng.choice([1, 2, 4, 8, 10]))
    max_len = int(rng.integers(1, 3000))
    max_pages = -(-max_len // PAGE)
    lens = rng.integers(-2, max_len + 1, B)
    if seed % 7 == 0:
        lens[rng.integers(0, B)] = max_pages * PAGE + 5   # past the block table: no pages
    window = int(rng.choice([-1, 0, 15, 16, 100, 700]))
    workers = int(rng.integers(1, 70))
    replay(lens, hkv, workers, window, max_pages)


def test_more_workers_than_pages():
    replay([1, 2, 0, 17], 4, 4096, -1, 2)
    replay([5], 1, 6, -1, 1)
