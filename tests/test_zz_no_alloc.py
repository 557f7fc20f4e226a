"""nc_decode_attn_fp8_noalloc (workspace in a static device array) against nc_decode_attn_fp8 (caller's workspace):
bit-identical outputs on two calls in a row, the second with a smaller input, both through the C ABI; and the use it
exists for, a call captured into a HIP graph (as this file's first test, so in a process that has not called it
before, its first call, with the device lookup of its array, happens under capture), replayed with new sequence
lengths between the replays."""
import pytest
import torch

from nanochat_amd.attention import decode_attention
from nanochat_amd.native import check, hip_library, pointer, stream
from nanochat_amd.workloads import DecodeWorkload, decode_inputs
from tests.paged_util import device_cache

pytestmark = pytest.mark.gpu


def noalloc(q, cache, table, lens, max_seq_len, window):
    B, Hq, _ = q.shape
    out = torch.full_like(q, float("nan"))
    check(hip_library().nc_decode_attn_fp8_noalloc(
        pointer(q), pointer(cache.k_pages), pointer(cache.v_pages), pointer(cache.kv_scale), pointer(table),
        table.size(1), cache.num_pages, pointer(lens), max_seq_len, B, Hq, cache.num_kv_heads, window,
        128 ** -0.5, 0, pointer(out), stream()))
    return out


def test_noalloc_under_graph_capture(device):
    w = DecodeWorkload("noalloc-graph", 10, 16, 4, 3000, ctx_min=1, paged=True)
    inp = decode_inputs(w, seed=31)
    cache, table, lens = device_cache(inp, w.kv_heads, device)
    q = inp["q"].to(device)
    lens_in = lens.clone()
    window = 900
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = noalloc(q, cache, table, lens_in, inp["max_seq_len"], window)
    shorter = torch.clamp(lens - torch.arange(1, lens.numel() + 1, device=device, dtype=lens.dtype) * 97, min=1)
    shorter[3] = 0                                          # an inactive sequence gives zeros
    for replay, new_lens in enumerate((lens, shorter, lens)):
        lens_in.copy_(new_lens)
        graph.replay()
        torch.cuda.synchronize()
        want = decode_attention(q, cache, table, new_lens, inp["max_seq_len"], window=window)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), replay
        if replay == 1:
            assert (out[3] == 0).all() and torch.isfinite(out.float()).all()


@pytest.mark.parametrize("window", [-1, 1500])
def test_noalloc_matches_workspace_entry_point(device, window):
    shapes = [DecodeWorkload("noalloc-big", 24, 16, 4, 6000, ctx_min=1, paged=True, outliers=0.01),
              DecodeWorkload("noalloc-small", 3, 8, 2, 700, ctx_min=1, paged=True)]
    for i, w in enumerate(shapes):
        inp = decode_inputs(w, seed=20 + i)
        cache, table, lens = device_cache(inp, w.kv_heads, device)
        q = inp["q"].to(device)
        want = decode_attention(q, cache, table, lens, inp["max_seq_len"], window=window)
        got = noalloc(q, cache, table, lens, inp["max_seq_len"], window)
        torch.cuda.synchronize()
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (w.name, window)
