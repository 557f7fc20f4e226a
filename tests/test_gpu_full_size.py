"""Every sequence of the BASELINE decode and prefill configurations at full size, against the PyTorch float32
restatement of the same attention (oracle/cpu_step.py, pinned against the float64 oracle by
tests/test_oracle_cpu_step.py; its quantizer gives the float64 oracle's codes exactly, so the CPU cache holds the
device's bytes). The float64 oracle is too slow for whole batches at these sizes; float32 accumulation over 8,193 keys
stays far inside the tolerances. Bounds: the north star's (max abs <= 2e-2, mean <= 2e-3) over all rows, and per
element within 2^-7 of sum_j p_j |v_j| (attention over the same cache with |v|). Where outputs exceed 1 in magnitude (a
short window over config 3's 8-sigma outlier values reaches |out| = 4.4, whose bf16 rounding alone is 2^-9 of it), the
absolute bounds scale with the largest output; the per-element bound is the same everywhere."""
import numpy as np
import pytest
import torch

from nanochat_amd.attention import decode_attention, prefill_attention, qk_norm_rope_append
from nanochat_amd.kv_cache import PagedKVCache
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.workloads import DECODE, PREFILL, decode_inputs, prefill_inputs
from oracle import cpu_step as cs
from oracle.numerics import bf16_round
from oracle.rope import qk_norm_rope
from tests.conftest import ATTN_MAX_ABS, ATTN_MEAN_ABS
from tests.paged_util import device_cache

pytestmark = pytest.mark.gpu
REL_BOUND = 2.0 ** -7


def check(got: torch.Tensor, want: torch.Tensor, want_mag: torch.Tensor, what: str) -> None:
    err = (got.float().cpu().double() - want.double()).abs()
    scale = max(1.0, want.abs().max().item())
    assert err.max().item() <= ATTN_MAX_ABS * scale and err.mean().item() <= ATTN_MEAN_ABS * scale, \
        (what, err.max(), err.mean(), scale)
    worst = (err - REL_BOUND * want_mag.double()).max().item()
    assert worst <= 1e-4, f"{what}: error exceeds 2^-7 of sum p|v| by {worst}"


def cpu_attend(q: torch.Tensor, cache: cs.PagedCpuCache, table: torch.Tensor, positions: torch.Tensor,
               lengths: torch.Tensor, rows: int = 8, window: int = -1) -> tuple[torch.Tensor, torch.Tensor]:
    """Attention and its magnitude (|v|) over the CPU cache, `rows` sequences at a time (memory)."""
    outs, mags = [], []
    for b0 in range(0, q.shape[0], rows):
        sl = slice(b0, b0 + rows)
        K, V = cache.gather(table[sl], lengths[sl])
        outs.append(cs.attend(q[sl], K, V, positions[sl], lengths[sl], window))
        mags.append(cs.attend(q[sl], K, V.abs(), positions[sl], lengths[sl], window))
    return torch.cat(outs), torch.cat(mags)


@pytest.mark.parametrize("name,window", [("c3u", -1), ("c3", -1), ("c2", -1), ("c3u", 1024), ("c3", 700)])
def test_decode_every_sequence(device, name, window):
    """Every sequence; with a window (a sliding-window layer) the keys before p - window are skipped whole chunks
    and partial pages at a time."""
    w = DECODE[name]
    inp = decode_inputs(w, seed=0)
    print(f"full-size decode {name}: B={w.batch} Hq={w.q_heads} Hkv={w.kv_heads} ctx<={w.ctx} window={window}",
          flush=True)
    cache, table, lens = device_cache(inp, w.kv_heads, device)
    out = decode_attention(inp["q"].to(device), cache, table, lens, inp["max_seq_len"], window=window)
    torch.cuda.synchronize()

    ctable = inp["block_table"]
    ccache = cs.PagedCpuCache(inp["num_pages"], w.kv_heads)
    for b in range(w.batch):
        n = int(inp["ctx_lens"][b])
        if n:
            ccache.store(ctable, b, torch.arange(n), inp["k_cache"][b, :n].float(), inp["v_cache"][b, :n].float())
        ccache.store(ctable, b, torch.tensor([n]), inp["k_new"][b].float(), inp["v_new"][b].float())
    clens = inp["ctx_lens"].long() + 1
    want, mag = cpu_attend(inp["q"].float()[:, None], ccache, ctable, (clens - 1)[:, None], clens, window=window)
    check(out, want[:, 0], mag[:, 0], f"{name} window {window}")


@pytest.mark.parametrize("window", [-1, 700])
def test_prefill_every_sequence_c4(device, window):
    w = PREFILL["c4"]
    inp = prefill_inputs(w, seed=0)
    print(f"full-size prefill c4: B={w.batch} chunk={w.chunk} ctx={w.ctx} window={window}", flush=True)
    cache = PagedKVCache(inp["num_pages"], w.kv_heads, device)
    table = inp["block_table"].to(device)
    start = inp["start_pos"].to(device)
    cache.append(inp["k_cache"].to(device), inp["v_cache"].to(device), torch.zeros_like(start), table, num_new=start)
    cos, sin = rotary_tables(w.ctx + w.chunk + 1, w.theta, device)
    q = qk_norm_rope_append(inp["qkv"].to(device), w.q_heads, cache, table, start, inp["q_gain"].to(device),
                            inp["k_gain"].to(device), cos, sin)
    out = prefill_attention(q, cache, table, start, window=window)
    torch.cuda.synchronize()

    # the chunk's rows through the float64 oracle's norm + rotation (bit-exact to the device: checked for every q)
    H, G = w.q_heads, w.kv_heads
    x = inp["qkv"].float().numpy().reshape(w.batch, w.chunk, H + 2 * G, 128)
    pos = w.ctx + np.arange(w.chunk)
    c, s = cos.cpu().numpy()[pos][:, None], sin.cpu().numpy()[pos][:, None]
    oq = qk_norm_rope(x[:, :, :H], inp["q_gain"].numpy(), c, s)
    ok = qk_norm_rope(x[:, :, H:H + G], inp["k_gain"].numpy(), c, s)
    assert np.array_equal(bf16_round(oq), q.float().cpu().numpy())

    ctable = inp["block_table"]
    ccache = cs.PagedCpuCache(inp["num_pages"], G)
    cpos = torch.arange(w.chunk) + w.ctx
    for b in range(w.batch):
        ccache.store(ctable, b, torch.arange(w.ctx), inp["k_cache"][b].float(), inp["v_cache"][b].float())
        ccache.store(ctable, b, cpos, torch.from_numpy(bf16_round(ok[b])).float(),
                     torch.from_numpy(x[b, :, H + G:]).float())
    lengths = torch.full((w.batch,), w.ctx + w.chunk)
    positions = cpos[None, :].expand(w.batch, -1)
    want, mag = cpu_attend(torch.from_numpy(bf16_round(oq)).float(), ccache, ctable, positions, lengths, rows=2,
                           window=window)
    check(out, want, mag, f"c4 window {window}")
