"""The decoder runtime (libnanochat_decode.so through the dec_* ABI) against the CPU oracle: prefill caches, step
logits, the choice (greedy, masks, alternative, Gumbel-max, nucleus), the prompt store, inactive slots and
continuous batching. Logits are compared teacher-forced: each step's inputs are the tokens the device chose."""
import numpy as np
import pytest
import torch

from nanochat_amd.decoder import DecoderRuntime, Request, serve
from nanochat_amd.workloads import model_tensors
from oracle import model as om
from oracle import sampling

pytestmark = pytest.mark.gpu

# tiny: 3 layers (a 40-key window on layer 0, value embeddings on layers 0 and 2); wide: the config-5 width
SHAPES = {
    "tiny": dict(layers=3, hidden=256, ffn=1024, vocab=2048, max_length=160, windows=[40, 160, 160], ve_layers=(0, 2)),
    "wide": dict(layers=2, hidden=1664, ffn=6656, vocab=4096, max_length=96, windows=[96, 96], ve_layers=()),
    # wider than 2,048: the step's o and fc GEMMs take two K-slices, so the MLP's rstd comes from rstd_kernel
    "wider": dict(layers=2, hidden=2304, ffn=9216, vocab=4096, max_length=64, windows=[64, 20], ve_layers=(1,)),
}
# logits against the float64 oracle on the same inputs, relative to the largest |logit|: fp32 GEMM accumulation
# flips bf16 roundings of intermediate activations and fp8 codes downstream (fp32 GEMMs alone move the oracle's
# own logits by ~0.6% max, ~0.08% mean of that scale); the device's attention adds bf16 probabilities in PV
LOGIT_MAX_REL = 2e-2
LOGIT_MEAN_REL = 3e-3
# a choice may differ from the oracle's only between scores this close (relative)
NEAR_TIE = 1e-5


def build(device, shape, seed=0):
    s = dict(SHAPES[shape])
    max_length = s.pop("max_length")
    m = model_tensors(s["layers"], s["hidden"], s["ffn"], s["vocab"], max_length, seed=seed, std=0.05,
                      theta=10000.0, ve_layers=s["ve_layers"], windows=s["windows"], device=device)
    return m, om.weights_from_tensors(m), max_length


def prompts(lengths, vocab, seed):
    rng = np.random.default_rng(seed)
    return [[0] + list(rng.integers(1, vocab, n - 1)) for n in lengths]


def check_logits(got, want, label):
    """Returns the absolute max-error bound used, for near-argmax checks."""
    err = np.abs(got.astype(np.float64) - want)
    scale = np.abs(want).max()
    print(f"{label}: logits max abs {err.max():.3e} mean abs {err.mean():.3e} (scale {scale:.2f})", flush=True)
    assert err.max() <= LOGIT_MAX_REL * scale and err.mean() <= LOGIT_MEAN_REL * scale, label
    return LOGIT_MAX_REL * scale


def check_cache(dec, orc, layer, b, n, label):
    """Layer 0's rows come from exact inputs: codes equal but for rare neighbours (an fp32-accumulated GEMM output
    rounding to the other bf16). Deeper layers inherit the accumulated rounding noise of the layers before (fp32
    GEMMs alone move the oracle's own deeper-layer values by ~1% RMS), so they are compared as values."""
    from oracle.quant import dequantize_rows

    k, v, s = dec.cache_rows(layer, b, 0, n)
    c = orc.codes[b]
    for name, got, want, i in (("k", k, c["k"][layer, :n], 0), ("v", v, c["v"][layer, :n], 1)):
        x = dequantize_rows(got, s[..., i]).astype(np.float64)
        y = dequantize_rows(want, c["scale"][layer, :n, :, i]).astype(np.float64)
        if layer == 0:
            same = np.mean(got == want)
            assert same >= 0.995, f"{label} {name}: {same:.4f} of the codes equal"
            # a differing value is within one e4m3 step of the oracle's plus a bf16 ulp of the row's absmax
            # (448 scale): an element that is a near-cancellation of row-sized terms moves by the latter
            step = np.maximum(np.abs(x), np.abs(y)) * 2 ** -3 + 448 * s[..., i, None] * 2 ** -7
            far = np.argwhere(np.abs(x - y) > step)
            detail = [(tuple(f), int(got[tuple(f)]), int(want[tuple(f)]), float(x[tuple(f)]), float(y[tuple(f)]),
                       float(s[f[0], f[1], i]), float(c["scale"][layer, f[0], f[1], i])) for f in far[:8]]
            assert len(far) == 0, f"{label} {name}: {len(far)} far codes (pos, head, dim), got, want: {detail}"
            rel = np.abs(s[..., i] - c["scale"][layer, :n, :, i]) / np.maximum(c["scale"][layer, :n, :, i], 1e-30)
            assert rel.max() <= 2 ** -7, f"{label} {name} scales: {rel.max():.3e}"
        rms = np.sqrt(np.mean((x - y) ** 2) / np.mean(y ** 2))
        worst = np.abs(x - y).max() / np.abs(y).max()
        print(f"{label} {name}: rel rms {rms:.2e} rel max {worst:.2e}", flush=True)
        assert rms <= 0.04 and worst <= 0.2, f"{label} {name}: rel rms {rms:.3e}, rel max {worst:.3e}"


def run_steps(dec, orc, inputs, positions, slots, steps, label, temperature=None):
    """Greedy steps over `slots` (all active), checking logits, choice and alternative; returns the new inputs."""
    inputs, positions = list(inputs), list(positions)
    rows = max(slots) + 1
    for step in range(steps):
        tokens = dec.step()
        got = dec.logits(rows)
        want = orc.head(orc.body(inputs, positions, slots))
        bound = check_logits(got[slots], want, f"{label} step {step}")
        for i, b in enumerate(slots):
            tok, alt = sampling.choose(got[b], lazy=dec.bos)
            assert tokens[b] == tok and dec.alternatives[b] == alt, (label, step, b)
            # the device's choice is also (nearly) the oracle's best
            assert want[i][tok] >= want[i].max() - 2 * bound
        inputs = [int(tokens[b]) for b in slots]
        positions = [p + 1 for p in positions]
    return inputs, positions


@pytest.mark.parametrize("shape", ["tiny", "wide", "wider"])
def test_prefill_and_greedy_steps_match_oracle(device, shape):
    m, w, max_length = build(device, shape)
    lengths = {"tiny": [23, 64, 5, 81], "wide": [17, 40, 3], "wider": [12, 30, 2]}[shape]
    ids = prompts(lengths, m.vocab, seed=1)
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=8)
    try:
        orc = om.DecoderOracle(w, max_length)
        slots = list(range(len(ids)))
        for b in slots:
            dec.place(b, ids[b])
        dec.prefill()
        rows = [(t, p, b) for b in slots for p, t in enumerate(ids[b][:-1])]
        orc.body(*map(list, zip(*rows)), cache_only_last=True)
        for layer in range(len(m.layers)):
            for b in slots:
                check_cache(dec, orc, layer, b, len(ids[b]) - 1, f"{shape} layer {layer} slot {b}")
        dec.activate(slots)
        run_steps(dec, orc, [i[-1] for i in ids], [len(i) - 1 for i in ids], slots, 6, shape)
    finally:
        dec.close()


def test_prompt_store_round_trip_and_reuse(device):
    m, w, max_length = build(device, "tiny")
    ids = prompts([50, 30], m.vocab, seed=2)
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=200, max_slots=8)
    try:
        for b in (0, 1):
            dec.place(b, ids[b])
        dec.prefill()                                  # prefills, then stores both prompts (positions 0, 64)
        assert dec.stored == {tuple(ids[0]): 0, tuple(ids[1]): 64}
        dec.place(5, ids[0])   # loaded from the store, not prefilled
        assert not dec.queued
        n = len(ids[0]) - 1
        pool = dec.pages()[1]
        # the prompt's 3 whole pages are the store's (shared), the partial 4th a pool page of the slot's own
        row = dec.table(5)
        assert list(row[:3]) == [pool + e for e in range(3)] and 0 <= row[3] < pool
        for layer in range(len(m.layers)):
            a, s_ = dec.cache_rows(layer, 0, 0, n), dec.cache_rows(layer, -1, 0, n)
            c = dec.cache_rows(layer, 5, 0, n)
            for x, y, z in zip(a, s_, c):
                assert np.array_equal(x, y) and np.array_equal(x, z), layer
            t1 = dec.cache_rows(layer, -1, 64, len(ids[1]) - 1)
            for x, y in zip(dec.cache_rows(layer, 1, 0, len(ids[1]) - 1), t1):
                assert np.array_equal(x, y), layer
        dec.activate([0, 1, 5])
        tokens = dec.step()
        got = dec.logits(6)
        # same cache bytes and inputs, and a step's sums for a slot do not depend on the other slots: equal bits
        assert tokens[0] == tokens[5]
        assert np.array_equal(got[0], got[5])
    finally:
        dec.close()


def test_shared_store_pages_copy_on_write(device):
    """A loaded prompt's whole pages are shared with the store; every later write into the slot or the store gives
    the writer a page of its own with the shared page's bytes copied first: prefill rows inside shared pages, a save
    over shared store pages; a load at another page phase copies and shares nothing. Cache bytes compared through the
    block tables after each."""
    m, w, max_length = build(device, "tiny")
    ids = prompts([50, 41], m.vocab, seed=12)
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=400, max_slots=8)
    L = len(m.layers)
    try:
        for b in (0, 1):
            dec.place(b, ids[b])
            dec.prefill()                               # A = ids[0] at store 0, B = ids[1] at store 64
        assert dec.stored == {tuple(ids[0]): 0, tuple(ids[1]): 64}
        nA, nB = len(ids[0]) - 1, len(ids[1]) - 1
        A = [dec.cache_rows(l, 0, 0, nA) for l in range(L)]
        B = [dec.cache_rows(l, 1, 0, nB) for l in range(L)]
        store = dec.pages()[1]   # store page i is pool + i

        def same(got, want):
            return all(np.array_equal(x, y) for x, y in zip(got, want))

        def own(row):
            return all(0 <= p < store for p in row)

        dec.lib.dec_load_prompt(dec.handle, 3, 0, 0, nA)           # slot 3 shares A's pages 0..2
        assert list(dec.table(3)[:3]) == [store, store + 1, store + 2]
        lo = 20                                                     # rows lo..nB-1 of B's tokens over pages 1, 2
        dec.lib.dec_prefill(dec.handle, nB - lo, np.ascontiguousarray(
            np.array([ids[1][lo:-1], range(lo, nB), [3] * (nB - lo)], dtype=np.int32)).ctypes.data)
        row = dec.table(3)
        assert row[0] == store and own(row[1:3])
        for l in range(L):
            assert same(dec.cache_rows(l, 3, 0, lo), [x[:lo] for x in A[l]]), l              # copied before the rows
            assert same(dec.cache_rows(l, 3, nB, nA - nB), [x[nB:] for x in A[l]]), l       # and after them
            assert same(dec.cache_rows(l, -1, 0, nA), A[l]), l                              # the store still holds A

        dec.lib.dec_load_prompt(dec.handle, 4, 0, 0, nA)           # slot 4 shares A ...
        dec.lib.dec_save_prompt(dec.handle, 1, 0, 0, nB)           # ... then B overwrites store positions 0..39
        row4 = dec.table(4)
        assert own(row4[:3]) and not set(row4[:3]) & set(dec.table(3)[:3])
        for l in range(L):
            assert same(dec.cache_rows(l, 4, 0, nA), A[l]), l            # slot 4 kept A
            assert same(dec.cache_rows(l, -1, 0, nB), B[l]), l

        dec.lib.dec_load_prompt(dec.handle, 6, 3, 64, nB)          # another page phase: copied, nothing shared
        row6 = dec.table(6)
        last = (3 + nB - 1) // 16
        assert own(row6[:last + 1]) and all(p == -1 for p in row6[last + 1:])
        for l in range(L):
            assert same(dec.cache_rows(l, 6, 3, nB), B[l]), l
        free, pool = dec.pages()
        for b in range(dec.batch):
            dec.release(b)
        assert dec.pages() == (pool, pool)
    finally:
        dec.close()


def test_page_pool_smaller_than_full_slots(device):
    """A pool of 10 pages for 8 slots of max_length 160 (10 pages each): serve admits requests while their longest
    extent fits the pool, returns each request's pages when it ends, and gives every request the same tokens as a
    decoder whose slots all reserve max_length (a request's tokens do not depend on the batch)."""
    m, w, max_length = build(device, "tiny")
    reqs = [Request(input_ids=p, max_new_tokens=8) for p in prompts([30, 17, 25, 31, 9, 22, 28, 14, 31, 5],
                                                                      m.vocab, seed=31)]
    results = {}
    for pool in (None, 10):
        rt = DecoderRuntime(m, bos_token_id=0, max_length=max_length, max_slots=8, pool_pages=pool)
        try:
            assert rt.batch == 8
            results[pool] = dict(serve(rt, reqs))
            free, size = rt.pages()
            assert free == size and size == (8 * 10 if pool is None else pool)
        finally:
            rt.close()
    assert results[None] == results[10]
    assert sorted(results[10]) == list(range(len(reqs)))


def test_masks_and_alternative(device):
    m, w, max_length = build(device, "tiny")
    ids = prompts([12, 20, 9], m.vocab, seed=3)
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=8)
    try:
        for b in range(3):
            dec.place(b, ids[b])
        dec.prefill()
        rng = np.random.default_rng(4)
        allowed = rng.random(m.vocab) < 0.05
        dec.masks[1] = np.packbits(allowed, bitorder="little").view("<u4")
        dec.masks[2] = 0
        dec.masks[2, 0] = 1                       # slot 2 may choose only BOS: its alternative is none (-1)
        dec.activate(range(3), masked=[1, 2])
        tokens = dec.step()
        got = dec.logits(3)
        for b in range(3):
            tok, alt = sampling.choose(got[b], allow=None if b == 0 else dec.masks[b], lazy=0)
            assert tokens[b] == tok and dec.alternatives[b] == alt, b
        assert allowed[tokens[1]]
        assert tokens[2] == 0 and dec.alternatives[2] == -1
        # take the alternative of slot 1: its next input is the alternative token
        alt1 = int(dec.alternatives[1])
        dec.take_alternative(1)
        dec.activate(range(3))
        orc = om.DecoderOracle(w, max_length)
        rows = [(t, p, b) for b in range(3) for p, t in enumerate(ids[b][:-1])]
        orc.body(*map(list, zip(*rows)), cache_only_last=True)
        orc.body([i[-1] for i in ids], [len(i) - 1 for i in ids], [0, 1, 2])
        inputs = [int(tokens[0]), alt1, int(tokens[2])]
        run_steps(dec, orc, inputs, [len(i) for i in ids], [0, 1, 2], 1, "after take_alt")
    finally:
        dec.close()


def near_tie_ok(got_tok, want_tok, scores):
    return got_tok == want_tok or abs(scores[got_tok] - scores[want_tok]) <= NEAR_TIE * max(1.0, abs(scores[want_tok]))


def test_sampling_matches_oracle_choice(device):
    m, w, max_length = build(device, "tiny")
    ids = prompts([10, 14, 18, 22], m.vocab, seed=5)
    params = [(0.9, 1.0, 7), (0.7, 0.8, 123456789012345), (1.3, 0.5, 2 ** 63 + 5), (0.0, 0.5, 1)]
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=8)
    try:
        for b, (T, p, seed) in enumerate(params):
            dec.place(b, ids[b], temperature=T, top_p=p, seed=seed)
        dec.prefill()
        dec.activate(range(4))
        for step in range(5):
            tokens = dec.step()
            got = dec.logits(4)
            for b, (T, p, seed) in enumerate(params):
                tok, alt = sampling.choose(got[b], temperature=T, top_p=p, seed=seed, gen=step, lazy=0,
                                           softcap=m.softcap)
                if T > 0:
                    z = sampling.capped(got[b], m.softcap)
                    scores = (z / np.float32(T)).astype(np.float32) + sampling.gumbel(seed, step, np.arange(m.vocab))
                    if p < 1:
                        keep, e = sampling.nucleus_keep(z, T, p, np.ones(m.vocab, bool))
                        if not keep[tokens[b]]:   # only a row at the nucleus boundary may differ
                            kept = e[keep]
                            assert abs(e[tokens[b]] - kept.min()) <= 1e-5 * kept.min(), (step, b)
                        else:
                            assert near_tie_ok(int(tokens[b]), tok, scores), (step, b)
                        assert dec.alternatives[b] == -1
                    else:
                        assert near_tie_ok(int(tokens[b]), tok, scores), (step, b)
                        assert near_tie_ok(int(dec.alternatives[b]), alt, scores), (step, b)
                else:
                    assert tokens[b] == tok and dec.alternatives[b] == alt
    finally:
        dec.close()


def test_inactive_slot_holds_still(device):
    m, w, max_length = build(device, "tiny")
    ids = prompts([15, 25, 35], m.vocab, seed=6)
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=8)
    try:
        for b in range(3):
            dec.place(b, ids[b])
        dec.prefill()
        orc = om.DecoderOracle(w, max_length)
        rows = [(t, p, b) for b in range(3) for p, t in enumerate(ids[b][:-1])]
        orc.body(*map(list, zip(*rows)), cache_only_last=True)
        dec.activate([0, 2])                           # slot 1 idles this step
        inputs, pos = run_steps(dec, orc, [ids[0][-1], ids[2][-1]], [14, 34], [0, 2], 1, "slot 1 idle")
        _, _, s = dec.cache_rows(0, 1, len(ids[1]) - 1, 1)
        assert np.all(s == 0)                          # its next position was not written
        dec.activate([0, 1, 2])
        run_steps(dec, orc, [inputs[0], ids[1][-1], inputs[1]], [pos[0], 24, pos[1]], [0, 1, 2], 2, "slot 1 back")
    finally:
        dec.close()


def test_serve_continuous_batching(device):
    """serve() over more requests than slots: every output token is (nearly) the oracle's greedy choice given the
    tokens before it; stopping criteria and max_new_tokens end requests; slots are refilled."""
    m, w, max_length = build(device, "tiny")
    ids = prompts([9, 30, 12, 44, 7], m.vocab, seed=7)
    stop_after = {3: 2}
    requests = [Request(input_ids=ids[i], max_new_tokens=5,
                        stopping_criteria=(lambda out, k=stop_after.get(i): k is not None and len(out) >= k))
                for i in range(5)]
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=300, max_slots=2)
    try:
        assert dec.batch == 2
        timings = {}
        done = dict(serve(dec, requests, timings))
        assert sorted(done) == list(range(5))
        assert sorted(timings) == list(range(5)) and all(a <= b <= c for a, b, c in timings.values())
        for i, out in done.items():
            assert 1 <= len(out) <= 5
            if i == 3:
                assert len(out) == 2
            orc = om.DecoderOracle(w, max_length)
            seq = ids[i] + out
            n = len(ids[i]) - 1
            orc.body(seq[:n], list(range(n)), [0] * n, cache_only_last=True)
            for j, tok in enumerate(out):
                want = orc.head(orc.body([seq[n + j]], [n + j], [0]))[0]
                assert want[tok] >= want.max() - 2 * LOGIT_MAX_REL * np.abs(want).max(), (i, j)
    finally:
        dec.close()


def test_steps_are_deterministic(device):
    """Two decoders fed the same prompts give bit-identical logits: no GEMM or attention kernel the step runs sums
    in a run-dependent order."""
    m, w, max_length = build(device, "wide")
    ids = prompts([20, 33, 7], m.vocab, seed=9)
    out = []
    for _ in range(2):
        dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=8)
        try:
            for b in range(3):
                dec.place(b, ids[b])
            dec.prefill()
            dec.activate(range(3))
            logits = []
            for _ in range(3):
                dec.step()
                logits.append(dec.logits(3))
            out.append(np.stack(logits))
        finally:
            dec.close()
    assert np.array_equal(out[0], out[1])


def test_two_lane_steps_match_one_lane_and_oracle(device):
    """A step over more than 64 slots runs as two concurrent lanes (slots [0, 64) on the caller's stream, the rest on
    the decoder's own, their attentions alternating): slots of both lanes match the oracle teacher-forced, the logits
    match the one-lane step's within the fp32-order tolerance (the lanes' GEMMs and split-K attention add in another
    order), the choices agree but at near-ties, and two two-lane runs are bit-identical."""
    m, w, max_length = build(device, "tiny")
    n = 100
    lengths = [4 + (13 * b) % 37 for b in range(n)]
    ids = prompts(lengths, m.vocab, seed=11)
    runs = []
    for split in (0, 1, 1):
        dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=128)
        try:
            assert dec.batch >= n
            dec.lib.dec_debug_set_split(dec.handle, split)
            for b in range(n):
                dec.place(b, ids[b])
            dec.prefill()
            dec.activate(range(n))
            steps = []
            for _ in range(2):
                tokens = dec.step()
                steps.append((dec.logits(n), tokens[:n].copy()))
            runs.append(steps)
        finally:
            dec.close()
    one, two, again = runs
    for (la, ta), (lb, tb) in zip(two, again):
        assert np.array_equal(la, lb) and np.array_equal(ta, tb)
    (l1, t1), (l2, t2) = one[0], two[0]
    scale = np.abs(l1).max()
    err = np.abs(l1.astype(np.float64) - l2)
    print(f"one lane vs two lanes: max {err.max():.3e} mean {err.mean():.3e} (scale {scale:.2f})", flush=True)
    # the same bound as against the oracle: reordered fp32 sums flip bf16 roundings and fp8 codes downstream
    assert err.max() <= LOGIT_MAX_REL * scale and err.mean() <= LOGIT_MEAN_REL * scale
    for b in range(n):
        if t1[b] != t2[b]:
            assert abs(l2[b][t1[b]] - l2[b][t2[b]]) <= 2 * err.max(), b
    orc = om.DecoderOracle(w, max_length)
    rows = [(t, p, b) for b in range(n) for p, t in enumerate(ids[b][:-1])]
    orc.body(*map(list, zip(*rows)), cache_only_last=True)
    sample = [0, 1, 63, 64, 65, 99]
    want = orc.head(orc.body([ids[b][-1] for b in sample], [lengths[b] - 1 for b in sample], sample))
    check_logits(l2[sample], want, "two lanes step 0")


@pytest.mark.parametrize("slots", [3, 100])
def test_graph_replays_match_eager_steps(device, slots):
    """With graphs on, the step's body replays a captured graph from its third step on (the first runs eagerly, the
    second captures): every replay, each after the host's own work and a synchronization (dec_tokens), gives logits
    and tokens bit-identical to the same steps launched kernel by kernel; one lane (3 slots) and two lanes (100)."""
    m, w, max_length = build(device, "tiny")
    lengths = [4 + (13 * b) % 37 for b in range(slots)]
    ids = prompts(lengths, m.vocab, seed=12)
    runs = []
    for graphs in (0, 1):
        dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=128)
        try:
            dec.lib.dec_debug_set_graphs(dec.handle, graphs)
            dec.lib.dec_debug_set_split(dec.handle, 1)
            for b in range(slots):
                dec.place(b, ids[b])
            dec.prefill()
            dec.activate(range(slots))
            steps = []
            for _ in range(6):
                tokens = dec.step()
                steps.append((dec.logits(slots), tokens[:slots].copy()))
            runs.append(steps)
        finally:
            dec.close()
    for i, ((le, te), (lg, tg)) in enumerate(zip(*runs)):
        assert np.array_equal(le, lg) and np.array_equal(te, tg), f"step {i}"


def test_a_requests_tokens_do_not_depend_on_the_batch(device):
    """The reference's contract (inference/decoder.py:124-125): a request's tokens depend on neither the batch nor the
    store. One prompt decoded (a) alone in slot 0, (b) in slot 2 of a ragged batch prefilled in the same dec_prefill
    call, (c) in slot 5 of another batch with its prefill split over two dec_prefill calls, and (d) loaded from the
    prompt store into slot 3: its cache bytes (every layer), and its logits and tokens over four steps, are
    bit-identical."""
    m, w, max_length = build(device, "tiny")
    P = prompts([57], m.vocab, seed=21)[0]
    others = prompts([23, 81, 5, 40, 66], m.vocab, seed=22)
    L, n = len(m.layers), len(P) - 1

    def run(slot, batch, split_at=None, from_store=False):
        dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=200, max_slots=8)
        try:
            if from_store:                      # P prefilled in slot 7 and stored; the slot under test loads it
                dec.place(7, P)
                dec.prefill()
                assert dec.place(slot, P)
            for b, ids in batch.items():
                dec.place(b, ids)
            if not from_store:
                dec.place(slot, P)
            if split_at is None:
                dec.prefill()
            else:                               # the queued rows in two calls, the second starting inside P
                rows = np.concatenate([np.stack([np.array(q[:-1]), np.arange(len(q) - 1), np.full(len(q) - 1, b)])
                                       for b, q in dec.queued], axis=1).astype(np.int32)
                cut = rows.shape[1] - (n - split_at)
                for part in (rows[:, :cut], rows[:, cut:]):
                    part = np.ascontiguousarray(part)
                    dec.lib.dec_prefill(dec.handle, part.shape[1], part.ctypes.data)
                dec.queued = []
            cache = [dec.cache_rows(layer, slot, 0, n) for layer in range(L)]
            dec.activate(sorted(set(batch) | {slot}))
            steps = []
            for _ in range(4):
                tokens = dec.step()
                steps.append((dec.logits(8)[slot].copy(), int(tokens[slot])))
            return cache, steps
        finally:
            dec.close()

    ref = run(0, {})
    cases = {"ragged batch, one prefill call": run(2, {0: others[0], 1: others[1], 3: others[2]}),
             "another slot, prefill split over two calls": run(5, {b: others[b] for b in range(5)}, split_at=20),
             "loaded from the prompt store": run(3, {0: others[3], 4: others[4]}, from_store=True)}
    for label, (cache, steps) in cases.items():
        for layer in range(L):
            for x, y in zip(cache[layer], ref[0][layer]):
                assert np.array_equal(x, y), (label, layer)
        for i, ((lg, tg), (lr, tr)) in enumerate(zip(steps, ref[1])):
            assert tg == tr and np.array_equal(lg, lr), (label, i)


def test_more_than_128_slots(device):
    """A step over more slots than one slot-GEMM block holds (128): the GEMMs, the o GEMM's tile sums, fc's rstd and
    proj_norm run per block of 128 slots. One prompt in slot 5 (first block) and slot 140 (second block), among 158
    other active slots with other prompts, gives bit-identical logits and tokens over three steps; slot 140 is also
    (nearly) the float64 oracle's greedy choice."""
    m, w, max_length = build(device, "tiny")
    dec = DecoderRuntime(m, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=160)
    try:
        assert dec.batch == 160
        P = prompts([19], m.vocab, seed=31)[0]
        others = prompts([3 + (b % 11) for b in range(160)], m.vocab, seed=32)
        for b in range(160):
            dec.place(b, P if b in (5, 140) else others[b])
        dec.prefill()
        dec.activate(range(160))
        orc = om.DecoderOracle(w, max_length)
        n = len(P) - 1
        orc.body(P[:n], list(range(n)), [0] * n, cache_only_last=True)
        tok = P[-1]
        for step in range(3):
            tokens = dec.step()
            got = dec.logits(160)
            print(f"160 slots step {step}: tokens {tokens[5]} {tokens[140]}", flush=True)
            assert tokens[5] == tokens[140] and np.array_equal(got[5], got[140]), step
            want = orc.head(orc.body([tok], [n + step], [0]))[0]
            assert want[tokens[140]] >= want.max() - 2 * LOGIT_MAX_REL * np.abs(want).max(), step
            tok = int(tokens[140])
    finally:
        dec.close()
