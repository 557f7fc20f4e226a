"""nc_decode_attn_fp8_noalloc (workspace in a static device array) against nc_decode_attn_fp8 (caller's workspace):
bit-identical outputs on two calls in a row, the second with a smaller input, both through the C ABI."""
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
