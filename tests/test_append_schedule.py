"""CPU replay of append_kernel's work split (nanochat_amd/csrc/kv_append.hip): grid x = (sequence b, k-th cache page its
new positions touch), pages_per_seq = (T + 14) / 16 + 1; work-group (b, k) takes the positions of page
floor(max(start, 0) / 16) + k that lie in [max(start, 0), start + min(T, num_new[b])), cut at rope_len when fused.
For random starts (negative, page-aligned or not), counts (zero, short, past T) and rope limits, every new position
of every sequence is taken by exactly one work-group, no work-group takes a position outside the new range, and
pages_per_seq work-groups always suffice."""
import numpy as np
import pytest

PAGE = 16


def pages_per_seq(T):
    return (T + PAGE - 2) // PAGE + 1


def replay(start, num_new, T, rope_len=None):
    """{(b, position): work-group k} as the kernel assigns them."""
    pps = pages_per_seq(T)
    taken = {}
    for b, sp in enumerate(start):
        n = T if num_new is None else min(int(num_new[b]), T)
        lo, hi = max(int(sp), 0), int(sp) + n
        if rope_len is not None:
            hi = min(hi, rope_len)
        if lo >= hi:
            continue
        for k in range(pps):
            lp = lo // PAGE + k
            pg0 = lp * PAGE
            s_lo, s_hi = max(lo, pg0) - pg0, min(hi, pg0 + PAGE) - pg0
            for slot in range(s_lo, s_hi):
                key = (b, pg0 + slot)
                assert key not in taken, key
                taken[key] = k
    return taken


@pytest.mark.parametrize("seed", range(60))
def test_every_new_position_once(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 9))
    T = int(rng.choice([1, 2, 15, 16, 17, 31, 32, 33, int(rng.integers(1, 300))]))
    start = rng.integers(-40, 200, B)
    aligned = rng.random(B) < 0.3
    start[aligned] = (start[aligned] // PAGE) * PAGE     # some starts on a page boundary
    num_new = rng.integers(-2, T + 5, B) if seed % 3 else None
    rope_len = int(rng.integers(1, 300)) if seed % 4 == 0 else None
    taken = replay(start, num_new, T, rope_len)
    for b in range(B):
        n = T if num_new is None else min(int(num_new[b]), T)
        want = {p for p in range(int(start[b]), int(start[b]) + max(n, 0))
                if p >= 0 and (rope_len is None or p < rope_len)}
        got = {p for (bb, p) in taken if bb == b}
        assert got == want, (b, sorted(want - got)[:5], sorted(got - want)[:5])


def test_pages_per_seq_is_the_most_pages_t_positions_touch():
    for T in range(1, 200):
        most = max(((s + T - 1) // PAGE) - (s // PAGE) + 1 for s in range(PAGE))
        assert pages_per_seq(T) == most, T
