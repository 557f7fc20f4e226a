"""GPU parity of the MFMA chunked prefill against the float64 oracle (max abs <= 2e-2, mean <= 2e-3), the
fused append that precedes it, and its agreement with decode attention at each row's position."""
import numpy as np
import pytest
import torch

from nanochat_amd.attention import decode_attention, prefill_attention, qk_norm_rope_append
from nanochat_amd.kv_cache import PagedKVCache
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.workloads import PREFILL, PrefillWorkload, prefill_inputs
from oracle.attention import prefill_attention as oracle_prefill
from oracle.layout import PAGE, PagedCache
from oracle.numerics import bf16_round
from oracle.rope import qk_norm_rope
from tests.conftest import ATTN_MAX_ABS, ATTN_MEAN_ABS
from tests.paged_util import attn_errors, check_relative, f32, magnitude_cache

pytestmark = pytest.mark.gpu


def device_prefill(w: PrefillWorkload, inp: dict, device, window=-1):
    """Existing cache through nc_kv_append_fp8, then the chunk's fused append and the prefill attention."""
    cache = PagedKVCache(inp["num_pages"], w.kv_heads, device)
    table = inp["block_table"].to(device)
    start = inp["start_pos"].to(device)
    if w.ctx:
        zeros = torch.zeros_like(start)
        cache.append(inp["k_cache"].to(device), inp["v_cache"].to(device), zeros, table, num_new=start)
    cos, sin = rotary_tables(w.ctx + w.chunk + 1, w.theta, device)
    q = qk_norm_rope_append(inp["qkv"].to(device), w.q_heads, cache, table, start, inp["q_gain"].to(device),
                            inp["k_gain"].to(device), cos, sin)
    out = prefill_attention(q, cache, table, start, window=window)
    torch.cuda.synchronize()
    return out, q, cache, table, start, cos.cpu().numpy(), sin.cpu().numpy()


def oracle_for(w: PrefillWorkload, inp: dict, seqs, cos, sin):
    """The oracle's q (normed, rotated) and a compact cache of sequences `seqs` after the chunk's append."""
    n = w.ctx + w.chunk
    mp = (n + PAGE - 1) // PAGE
    table = np.arange(len(seqs) * mp, dtype=np.int32).reshape(len(seqs), mp)
    cache = PagedCache(table.size, w.kv_heads)
    H, G = w.q_heads, w.kv_heads
    x = f32(inp["qkv"]).reshape(w.batch, w.chunk, H + 2 * G, 128)
    pos = w.ctx + np.arange(w.chunk)
    c, s = cos[pos][:, None], sin[pos][:, None]
    qs = []
    for i, b in enumerate(seqs):
        if w.ctx:
            cache.append(table, i, np.arange(w.ctx), f32(inp["k_cache"][b]), f32(inp["v_cache"][b]))
        q = qk_norm_rope(x[b, :, :H], inp["q_gain"].numpy(), c, s)
        k = qk_norm_rope(x[b, :, H:H + G], inp["k_gain"].numpy(), c, s)
        cache.append(table, i, pos, k, x[b, :, H + G:])
        qs.append(q)
    return np.stack(qs), cache, table


CASES = [
    PrefillWorkload("gqa4", 2, 16, 4, 45, 20, paged=True),
    PrefillWorkload("mha", 2, 6, 6, 100, 33, paged=True),
    PrefillWorkload("gqa16", 1, 16, 1, 17, 9, paged=False),
    PrefillWorkload("fresh", 3, 8, 2, 0, 70, paged=True),
    PrefillWorkload("gqa2-odd", 2, 6, 3, 31, 50, paged=True),
]


@pytest.mark.parametrize("w", CASES, ids=lambda w: w.name)
@pytest.mark.parametrize("window", [-1, 25])
def test_prefill_matches_oracle(device, w, window):
    inp = prefill_inputs(w, seed=len(w.name))
    out, q, _, _, start, cos, sin = device_prefill(w, inp, device, window)
    seqs = list(range(w.batch))
    oq, ocache, otable = oracle_for(w, inp, seqs, cos, sin)
    want = oracle_prefill(oq, ocache, otable, np.full(len(seqs), w.ctx), window=window)
    check_relative(out, want, oracle_prefill(oq, magnitude_cache(ocache), otable, np.full(len(seqs), w.ctx),
                                             window=window))
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)


def test_prefill_rows_equal_decode(device):
    w = PrefillWorkload("rows", 2, 16, 4, 300, 40, paged=True)
    inp = prefill_inputs(w, seed=11)
    out, q, cache, table, start, _, _ = device_prefill(w, inp, device)
    for t in (0, 17, 39):
        lens = start + t + 1
        dec = decode_attention(q[:, t].contiguous(), cache, table, lens, w.ctx + w.chunk)
        assert (dec.float() - out[:, t].float()).abs().max().item() <= 1e-2


def test_config4_full_size_subset(device):
    w = PREFILL["c4"]
    inp = prefill_inputs(w, seed=0)
    out, q, *_, cos, sin = device_prefill(w, inp, device)
    seqs = [0, w.batch - 1]
    oq, ocache, otable = oracle_for(w, inp, seqs, cos, sin)
    assert np.array_equal(bf16_round(oq), q[seqs].float().cpu().numpy())
    want = oracle_prefill(oq, ocache, otable, np.full(len(seqs), w.ctx))
    check_relative(out[seqs], want, oracle_prefill(oq, magnitude_cache(ocache), otable, np.full(len(seqs), w.ctx)))
    mx, mean = attn_errors(out[seqs], want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)
    assert torch.isfinite(out.float()).all()


def test_bad_page_gives_nan_for_its_sequence_only(device):
    """A block-table entry outside the page pool: every row of that sequence that reads it is NaN, the other
    sequence's rows are unchanged (both the LDS-staged and the register kernel check every pair they compute)."""
    w = PrefillWorkload("bad", 2, 16, 4, 45, 20, paged=True)
    inp = prefill_inputs(w, seed=5)
    out, q, cache, table, start, _, _ = device_prefill(w, inp, device)
    bad = table.clone()
    bad[1, 1] = cache.num_pages + 5            # keys 16..31: seen by every row of sequence 1 (no window)
    got = prefill_attention(q, cache, bad, start).float()
    torch.cuda.synchronize()
    assert torch.isnan(got[1]).all()
    assert torch.equal(got[0], out[0].float())


def test_growing_scores_rescale_mid_stream(device):
    """Cached keys whose magnitude grows twentyfold along the sequence: every chunk row's running max passes its
    reference by more than 2^8 several times after the first page pair (the lazy rescale's slow path mid-stream)."""
    w = PrefillWorkload("grow", 2, 16, 4, 200, 40, paged=True)
    inp = prefill_inputs(w, seed=12)
    ramp = torch.linspace(1.0, 20.0, w.ctx).view(1, w.ctx, 1, 1)
    inp["k_cache"] = (inp["k_cache"].float() * ramp).bfloat16()
    out, q, _, _, start, cos, sin = device_prefill(w, inp, device)
    seqs = list(range(w.batch))
    oq, ocache, otable = oracle_for(w, inp, seqs, cos, sin)
    want = oracle_prefill(oq, ocache, otable, np.full(len(seqs), w.ctx))
    check_relative(out, want, oracle_prefill(oq, magnitude_cache(ocache), otable, np.full(len(seqs), w.ctx)))
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("window", [-1, 25])
def test_long_block_table_takes_register_kernel(device, window):
    """A block-table row longer than the 4,096 entries a workgroup stages in LDS sends the launch to the
    register-prefetch kernel (`prefill_kernel`): the same sequences, their table padded to 4,100 entries, meet the
    oracle bound there and agree with the LDS-staged kernel's output; a bad entry still turns only its own
    sequence into NaN."""
    w = PrefillWorkload("wide", 2, 6, 3, 31, 50, paged=True)
    inp = prefill_inputs(w, seed=31)
    narrow = inp["block_table"]
    wide = torch.zeros((narrow.shape[0], 4100), dtype=narrow.dtype)
    wide[:, :narrow.shape[1]] = narrow
    lds_out = device_prefill(w, inp, device, window)[0]
    out, q, cache, table, start, cos, sin = device_prefill(w, dict(inp, block_table=wide), device, window)
    assert table.shape[1] == 4100
    seqs = list(range(w.batch))
    oq, ocache, otable = oracle_for(w, inp, seqs, cos, sin)
    want = oracle_prefill(oq, ocache, otable, np.full(len(seqs), w.ctx), window=window)
    check_relative(out, want, oracle_prefill(oq, magnitude_cache(ocache), otable, np.full(len(seqs), w.ctx),
                                             window=window))
    mx, mean = attn_errors(out, want)
    assert mx <= ATTN_MAX_ABS and mean <= ATTN_MEAN_ABS, (mx, mean)
    mx, _ = attn_errors(out, f32(lds_out).astype(np.float64))
    assert mx <= ATTN_MAX_ABS, mx

    bad = table.clone()
    bad[1, (w.ctx + w.chunk - 1) // PAGE] = cache.num_pages + 5   # the last page: every window sees it
    got = prefill_attention(q, cache, bad, start, window=window).float()
    torch.cuda.synchronize()
    assert torch.isnan(got[1, -1]).all()
    assert torch.equal(got[0], out[0].float())
