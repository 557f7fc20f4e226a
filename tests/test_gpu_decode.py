"""GPU parity of split-K decode attention against the float64 oracle (max abs <= 2e-2, mean <= 2e-3), plus the
properties that hold at full size: page-permutation invariance (bitwise), determinism, batch independence (a
sequence's output bits alone, in a ragged batch, at another place in it and under any worker count), inactive
sequences and out-of-pool pages."""
from pathlib import Path

import numpy as np
import pytest
import torch

from nanochat_amd.attention import decode_attention
from nanochat_amd.workloads import DECODE, DecodeWorkload, decode_inputs
from oracle.attention import decode_attention as oracle_decode
from tests.conftest import ATTN_MAX_ABS, ATTN_MEAN_ABS
from tests.paged_util import attn_errors, check_relative, device_cache, f32, magnitude_cache, oracle_cache

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def run(w: DecodeWorkload, device, seed=0, window=-1, workers=0, seqs=None, inp=None):
    inp = inp or decode_inputs(w, seed)
    cache, table, lens = device_cache(inp, w.kv_heads, device)
    q = inp["q"].to(device)
    out = decode_attention(q, cache, table, lens, inp["max_seq_len"], window=window, workers=workers)
    torch.cuda.synchronize()
    seqs = range(w.batch) if seqs is None else seqs
    ocache, otable, olens = oracle_cache(inp, w.kv_heads, seqs)
    qs = f32(inp["q"][list(seqs)])
    want = oracle_decode(qs, ocache, otable, olens, window=window)
    check_relative(out[list(seqs)], want, oracle_decode(qs, magnitude_cache(ocache), otable, olens, window=window))
    return out, want, inp, (cache, table, lens, q)


SMALL = [
    DecodeWorkload("mha-tiny", 3, 4, 4, 100, ctx_min=1),
    DecodeWorkload("gqa4", 2, 16, 4, 1000, ctx_min=513, paged=True, outliers=0.01),
    DecodeWorkload("gqa8-window", 4, 8, 1, 200, ctx_min=30, paged=True),
    DecodeWorkload("c2-like", 2, 10, 10, 4096, ctx_min=300),
    DecodeWorkload("gqa16", 1, 16, 1, 77, paged=True),
    DecodeWorkload("gqa2-odd", 5, 4, 2, 33, ctx_min=1, paged=True),
]


@pytest.mark.parametrize("w", SMALL, ids=lambda w: w.name)
@pytest.mark.parametrize("workers", [0, 1, 6])
def test_decode_matches_oracle(device, w, workers):
    window = 50 if "window" in w.name else -1
    out, want, _, _ = run(w, device, window=window, workers=workers)
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("window", [0, 1, 15, 16, 17, 100])
def test_decode_windows(device, window):
    w = DecodeWorkload("win", 3, 8, 2, 300, ctx_min=1, paged=True)
    out, want, _, _ = run(w, device, seed=window, window=window, workers=4)
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)


def test_config1_golden_output(device):
    want = np.load(GOLDEN / "config1.npz")
    out, _, _, _ = run(DECODE["c1"], device)
    mx, mean = attn_errors(out, want["out_f64"])
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)


def test_permutation_invariance_and_determinism(device):
    w = DecodeWorkload("perm", 4, 16, 4, 700, ctx_min=100, paged=True, outliers=0.01)
    inp = decode_inputs(w, 1)
    outs = []
    for table in (inp["block_table"], torch.arange(inp["num_pages"], dtype=torch.int32).view_as(inp["block_table"])):
        cache, tab, lens = device_cache({**inp, "block_table": table}, w.kv_heads, device)
        for _ in range(2):
            outs.append(decode_attention(inp["q"].to(device), cache, tab, lens, inp["max_seq_len"]).cpu())
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))


def test_worker_count_changes_no_bit(device):
    """Waves take whole items (1,024-position chunks with their own softmax state), so the number of waves decides
    only who computes an item, never its sums."""
    w = DecodeWorkload("workers", 3, 8, 2, 5000, ctx_min=900, paged=True, outliers=0.01)
    inp = decode_inputs(w, 2)
    cache, table, lens = device_cache(inp, w.kv_heads, device)
    q = inp["q"].to(device)
    ref = decode_attention(q, cache, table, lens, inp["max_seq_len"], workers=1).view(torch.int16)
    for workers in (2, 5, 64, 0):
        o = decode_attention(q, cache, table, lens, inp["max_seq_len"], workers=workers).view(torch.int16)
        assert torch.equal(o, ref), workers


@pytest.mark.parametrize("window", [-1, 700, 2000])
def test_batch_independence(device, window):
    """A sequence's output bits do not depend on the rest of the launch (the reference's decoder promises tokens that
    depend on neither the batch nor the store, inference/decoder.py:124-125): decoded alone, inside a ragged batch,
    and at another place of a reordered batch, they are equal. Lengths cover one chunk, chunk boundaries (1,024 and
    1,025 keys) and several chunks."""
    w = DecodeWorkload("batch-ind", 10, 16, 4, 6000, ctx_min=1, paged=True, outliers=0.01)
    inp = decode_inputs(w, 11)
    inp["ctx_lens"][:6] = torch.tensor([1023, 1024, 2047, 5999, 40, 3333], dtype=torch.int32)
    cache, table, lens = device_cache(inp, w.kv_heads, device)
    q = inp["q"].to(device)
    mx = inp["max_seq_len"]
    full = decode_attention(q, cache, table, lens, mx, window=window).view(torch.int16).cpu()
    order = torch.randperm(w.batch, generator=torch.Generator().manual_seed(window + 5))
    perm = decode_attention(q[order].contiguous(), cache, table[order].contiguous(), lens[order].contiguous(), mx,
                            window=window).view(torch.int16).cpu()
    assert torch.equal(perm, full[order])
    for b in range(w.batch):
        alone = decode_attention(q[b:b + 1].contiguous(), cache, table[b:b + 1].contiguous(),
                                 lens[b:b + 1].contiguous(), mx, window=window, workers=3).view(torch.int16).cpu()
        assert torch.equal(alone[0], full[b]), b
    # and next to sequences of other lengths: the others replaced by copies of sequence 3 (5,999 keys)
    mixed = lens.clone()
    mixed[6:] = lens[3]
    tab = table.clone()
    tab[6:] = table[3]
    other = decode_attention(q, cache, tab, mixed, mx, window=window).view(torch.int16).cpu()
    assert torch.equal(other[:6], full[:6])


def test_inactive_and_bad_pages(device):
    w = DecodeWorkload("inactive", 3, 4, 2, 64, paged=True)
    inp = decode_inputs(w, 3)
    cache, table, lens = device_cache(inp, w.kv_heads, device)
    lens[1] = 0
    q = inp["q"].to(device)
    for workers in (2, 0):
        out = decode_attention(q, cache, table, lens, inp["max_seq_len"], workers=workers)
        assert out[1].abs().sum().item() == 0 and torch.isfinite(out.float()).all()
    bad = table.clone()
    bad[2, 1] = cache.num_pages + 5
    for workers in (2, 0):
        out = decode_attention(q, cache, bad, lens, inp["max_seq_len"], workers=workers).float()
        assert torch.isnan(out[2]).all() and torch.isfinite(out[0]).all()
    long = lens.clone()
    long[0] = inp["max_seq_len"] + 1          # longer than the launch's bound: NaN, the others unchanged
    out = decode_attention(q, cache, table, long, inp["max_seq_len"]).float()
    assert torch.isnan(out[0]).all() and torch.isfinite(out[2]).all()


@pytest.mark.parametrize("name", ["c3u", "c3", "c2"])
def test_full_size_subset(device, name):
    """BASELINE shapes at full size; the float64 oracle checks four sequences (first, last, two inside)."""
    w = DECODE[name]
    seqs = [0, w.batch // 3, 2 * w.batch // 3, w.batch - 1]
    out, want, _, _ = run(w, device, seqs=seqs)
    mx, mean = attn_errors(out[seqs], want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)
    assert torch.isfinite(out.float()).all()


def test_single_key_returns_dequantized_value(device):
    """One cached position: softmax weight 1, so out = bf16(code * bf16(v_scale)) elementwise."""
    w = DecodeWorkload("one-key", 4, 8, 2, 0, paged=True, outliers=0.05)
    inp = decode_inputs(w, 4)
    out, want, _, _ = run(w, device, inp=inp)
    v = want.astype(np.float32)          # the dequantized value itself
    got = out.float().cpu().numpy()
    assert np.all(np.abs(got - v) <= np.abs(v) * 2.0 ** -7 + 1e-30)


@pytest.mark.parametrize("n", [2, 3, 5, 8, 17, 33])
def test_few_keys(device, n):
    w = DecodeWorkload(f"few{n}", 6, 16, 4, n - 1, paged=True, outliers=0.02)
    run(w, device, seed=n, workers=2)


def test_workspace_reuse_across_shapes(device):
    """Calls with different (B, Hkv) in a row sharing the cached workspace, each checked."""
    shapes = [DecodeWorkload("wsA", 8, 16, 4, 900, paged=True), DecodeWorkload("wsB", 6, 10, 10, 1200),
              DecodeWorkload("wsA", 8, 16, 4, 900, paged=True), DecodeWorkload("wsC", 3, 8, 2, 2000, ctx_min=100)]
    for i, w in enumerate(shapes):
        for workers in (4, 0):
            out, want, _, _ = run(w, device, seed=i, workers=workers)
            mx, mean = attn_errors(out, want)
            assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (w.name, workers, mx, mean)


@pytest.mark.parametrize("workers", [0, 3])
def test_growing_scores_rescale_mid_stream(device, workers):
    """Key magnitudes growing along each sequence: the running max passes its reference by more than 2^8 again and
    again after the first page pair, so the lazy rescale's slow path runs mid-stream (and the chunks start on small
    references that the in-kernel merge must reconcile)."""
    w = DecodeWorkload("grow", 2, 8, 2, 600, ctx_min=400, paged=True)
    inp = decode_inputs(w, seed=9)
    n = inp["k_cache"].shape[1]
    ramp = torch.linspace(0.2, 6.0, n).view(1, n, 1, 1)
    inp["k_cache"] = (inp["k_cache"].float() * ramp).bfloat16()
    inp["q"] = (inp["q"].float() * 3.0).bfloat16()
    out, want, _, _ = run(w, device, workers=workers, inp=inp)
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("window", [-1, 1023, 1024, 3000])
def test_chunk_boundaries(device, window):
    """Lengths around the 1,024-position split points (1, 1,023, 1,024, 1,025, 2,048, 2,049 keys and up to 9,001),
    with windows whose start falls inside a chunk: every piece and the in-kernel merge meet the oracle bound."""
    w = DecodeWorkload("chunks", 8, 8, 2, 9000, ctx_min=1, paged=True)
    inp = decode_inputs(w, seed=7)
    inp["ctx_lens"][:] = torch.tensor([0, 1022, 1023, 1024, 2047, 2048, 5000, 9000], dtype=torch.int32)
    out, want, _, _ = run(w, device, seed=7, window=window, inp=inp)
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("window", [-1, 300, 1000, 1060])
def test_short_unit_cuts(device, window):
    """Units of at most 67 pages are cut every 16 pages (a last piece under 4 pages joined): lengths around those cuts
    (16, 17, 20, 21 pages), the 67 / 68-page boundary between the short and the 1,024-position cut, and windows that
    leave a long sequence a short, unaligned unit. Every piece and the merge meet the oracle bound, and each sequence's
    bits are the same decoded alone."""
    w = DecodeWorkload("short-cuts", 12, 8, 2, 5000, ctx_min=1, paged=True, outliers=0.01)
    inp = decode_inputs(w, seed=13)
    inp["ctx_lens"][:] = torch.tensor([255, 256, 319, 320, 1039, 1070, 1071, 1072, 1087, 2500, 4096, 4999],
                                      dtype=torch.int32)
    out, want, _, (cache, table, lens, q) = run(w, device, seed=13, window=window, inp=inp)
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)
    full = out.view(torch.int16).cpu()
    for b in range(w.batch):
        alone = decode_attention(q[b:b + 1].contiguous(), cache, table[b:b + 1].contiguous(),
                                 lens[b:b + 1].contiguous(), inp["max_seq_len"], window=window,
                                 workers=2).view(torch.int16).cpu()
        assert torch.equal(alone[0], full[b]), b
