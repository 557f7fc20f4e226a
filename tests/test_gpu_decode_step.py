"""The fused decode step (nc_decode_step_fp8) against the two launches it replaces (nc_qk_norm_rope_append_fp8 with
start_pos = seq_lens - 1, then nc_decode_attn_fp8) on the same inputs: the query rows, every cache byte and scale and
the attention output, bit for bit. Lengths sit on both sides of every page, page-pair and 1,024-position split
boundary; GQA 1, 4 and 16; windows; inactive and over-long sequences; an out-of-pool page; several steps in a row;
config 3u at full size. The two-launch path is pinned to the float64 oracle by test_gpu_append.py and
test_gpu_decode.py. Value embeddings have no two-launch form in the C ABI: with them the query and K bytes still
equal the two-launch run's and the V rows are checked against oracle/ve_gate.py's mix."""
import numpy as np
import pytest
import torch

from nanochat_amd.attention import decode_attention, decode_step, qk_norm_rope_append
from nanochat_amd.kv_cache import PagedKVCache, pages_for
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.workloads import DECODE, decode_inputs
from oracle import ve_gate as ove
from oracle.quant import quantize_rows
from tests.paged_util import read_sequence

pytestmark = pytest.mark.gpu

# every boundary a unit's pages can sit on: 1 token, a page (16), a page pair (32), a chunk (1,024 = 64 pages), a last
# piece of 3 pages (joined to the chunk before it, 2,096 keys) or 4 (a chunk of its own, 2,097), and for a unit of at
# most 67 pages the 16-page cuts (256, 320 keys) and the 67 / 68-page boundary (1,072 keys)
EDGE_LENGTHS = [1, 2, 15, 16, 17, 31, 32, 33, 48, 256, 257, 320, 321, 1023, 1024, 1025, 1040, 1056, 1072, 1073, 1088,
                1264, 1265, 1280, 1281, 2047, 2048, 2049, 2096, 2097, 3000]


def bf16_randn(gen, *shape, outliers=0.0):
    x = torch.randn(*shape, generator=gen, dtype=torch.float32)
    if outliers:
        mask = torch.rand(*shape, generator=gen) < outliers
        x[mask] = 8 * torch.sign(x[mask])
    return x.to(torch.bfloat16)


class State:
    """A cache holding `lengths[b] - 1` context tokens per sequence (position of the step's token: lengths[b] - 1),
    room for `steps` steps, a random page permutation, and the steps' qkv rows."""

    def __init__(self, lengths, Hq, Hkv, steps, seed, device, spare_pages=3):
        gen = torch.Generator().manual_seed(seed)
        self.B, self.Hq, self.Hkv, self.steps = len(lengths), Hq, Hkv, steps
        self.lengths = torch.tensor(lengths, dtype=torch.int32)
        ctx = max(1, max(lengths) - 1)
        self.max_len = max(lengths) + steps
        mp = pages_for(self.max_len)
        self.num_pages = self.B * mp + spare_pages
        self.table = torch.randperm(self.num_pages, generator=gen)[: self.B * mp].to(torch.int32).view(self.B, mp)
        kc = bf16_randn(gen, self.B, ctx, Hkv, 128, outliers=0.01)
        vc = bf16_randn(gen, self.B, ctx, Hkv, 128, outliers=0.01)
        self.qkv = bf16_randn(gen, steps, self.B, (Hq + 2 * Hkv) * 128, outliers=0.01)
        self.q_gain = 1.0 + 0.1 * torch.randn(128, generator=gen)
        self.k_gain = 1.0 + 0.1 * torch.randn(128, generator=gen)
        self.device = device
        self.cache = PagedKVCache(self.num_pages, Hkv, device)
        self.dtable = self.table.to(device)
        ctx_lens = (self.lengths - 1).clamp(min=0).to(device)
        self.cache.append(kc.to(device), vc.to(device), torch.zeros_like(ctx_lens), self.dtable, num_new=ctx_lens)
        self.cos, self.sin = rotary_tables(self.max_len, 1e6, device)
        self.gains = self.q_gain.to(device), self.k_gain.to(device)
        torch.cuda.synchronize()

    def clone_cache(self):
        c = PagedKVCache(self.num_pages, self.Hkv, self.device)
        c.k_pages.copy_(self.cache.k_pages)
        c.v_pages.copy_(self.cache.v_pages)
        c.kv_scale.copy_(self.cache.kv_scale)
        return c


def two_launch(s, cache, qkv, seq_lens, window, max_len, workers=0):
    q = qk_norm_rope_append(qkv.view(s.B, 1, -1), s.Hq, cache, s.dtable, seq_lens - 1, *s.gains, s.cos, s.sin)
    out = decode_attention(q.view(s.B, s.Hq, 128), cache, s.dtable, seq_lens, max_len, window=window, workers=workers)
    return q.view(s.B, s.Hq, 128), out


def fused(s, cache, qkv, seq_lens, window, max_len, workers=0, ve=None):
    q = torch.full((s.B, s.Hq, 128), -1.0, dtype=torch.bfloat16, device=s.device)
    out = decode_step(qkv, s.Hq, cache, s.dtable, seq_lens, *s.gains, s.cos, s.sin, max_len, window=window,
                      workers=workers, q_out=q, ve=ve)
    return q, out


def bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


def assert_same_cache(a, b):
    assert torch.equal(a.k_pages, b.k_pages)
    assert torch.equal(a.v_pages, b.v_pages)
    assert torch.equal(bits(a.kv_scale), bits(b.kv_scale))


def run_both(s, window=-1, workers=0, seq_lens=None, active=None):
    """Every step through both paths from the same starting cache; everything compared after each step."""
    ca, cb = s.clone_cache(), s.clone_cache()
    base = s.lengths.to(s.device) if seq_lens is None else seq_lens
    for t in range(s.steps):
        lens = torch.where(base > 0, base + t, base) if active is None else base
        qkv = s.qkv[t].to(s.device)
        qa, oa = two_launch(s, ca, qkv, lens, window, s.max_len, workers)
        qb, ob = fused(s, cb, qkv, lens, window, s.max_len, workers)
        torch.cuda.synchronize()
        on = (lens > 0) & (lens <= s.max_len)
        assert torch.equal(bits(qa[on]), bits(qb[on])), f"step {t}: query rows"
        assert torch.equal(bits(oa), bits(ob)), f"step {t}: attention output"
        assert_same_cache(ca, cb)
    return ca, cb


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (16, 4), (16, 1)])
def test_step_equals_append_then_attend(device, Hq, Hkv):
    s = State(EDGE_LENGTHS, Hq, Hkv, steps=3, seed=Hq + Hkv, device=device)
    run_both(s)


@pytest.mark.parametrize("window", [0, 1, 16, 100, 1030])
def test_step_windows(device, window):
    s = State(EDGE_LENGTHS, 8, 2, steps=2, seed=window, device=device)
    run_both(s, window=window, workers=6)


@pytest.mark.parametrize("workers", [1, 5, 64])
def test_step_worker_counts(device, workers):
    s = State([1, 700, 1025, 2100, 64], 16, 4, steps=2, seed=workers, device=device)
    run_both(s, workers=workers)


def test_step_inactive_and_overlong(device):
    """seq_lens <= 0: no append, zero rows; a sequence longer than max_seq_len: NaN rows, no append (the two-launch
    path's append would write it, so only the other sequences' bytes are compared)."""
    s = State([40, 40, 40, 40], 8, 2, steps=1, seed=3, device=device)
    ca, cb = s.clone_cache(), s.clone_cache()
    lens = torch.tensor([40, 0, -3, 40], dtype=torch.int32, device=device)
    qkv = s.qkv[0].to(device)
    qa, oa = two_launch(s, ca, qkv, lens, -1, s.max_len)
    qb, ob = fused(s, cb, qkv, lens, -1, s.max_len)
    torch.cuda.synchronize()
    assert torch.equal(bits(oa), bits(ob))
    assert not ob[1:3].float().abs().sum().item()
    assert_same_cache(ca, cb)
    before = PagedKVCache(s.num_pages, s.Hkv, device)
    for name in ("k_pages", "v_pages", "kv_scale"):
        getattr(before, name).copy_(getattr(cb, name))
    long = torch.tensor([40, s.max_len + 1, 40, 40], dtype=torch.int32, device=device)
    _, ob = fused(s, cb, qkv, long, -1, s.max_len)
    torch.cuda.synchronize()
    assert torch.isnan(ob[1].float()).all() and not torch.isnan(ob[[0, 2, 3]].float()).any()
    kc, ks, vc, vs = read_sequence(cb, s.dtable, 1, s.max_len)
    kb, ksb, vb, vsb = read_sequence(before, s.dtable, 1, s.max_len)
    assert np.array_equal(kc, kb) and np.array_equal(vc, vb)


def test_step_out_of_pool_page(device):
    """A token page outside the pool: NaN rows for that sequence, nothing stored; the others are unaffected."""
    s = State([20, 37, 1100], 8, 2, steps=1, seed=9, device=device)
    table = s.dtable.clone()
    table[1, 36 // 16] = s.num_pages + 5
    ca, cb = s.clone_cache(), s.clone_cache()
    lens = s.lengths.to(device)
    qkv = s.qkv[0].to(device)
    s.dtable, keep = table, s.dtable
    try:
        qa, oa = two_launch(s, ca, qkv, lens, -1, s.max_len)
        qb, ob = fused(s, cb, qkv, lens, -1, s.max_len)
    finally:
        s.dtable = keep
    torch.cuda.synchronize()
    assert torch.isnan(ob[1].float()).all() and torch.isnan(oa[1].float()).all()
    assert torch.equal(bits(oa[[0, 2]]), bits(ob[[0, 2]]))
    assert_same_cache(ca, cb)


@pytest.mark.parametrize("C", [512, 1664])
def test_step_value_embeddings(device, C):
    """With value embeddings: q rows and K bytes equal the two-launch run's (which has none); V codes and scales
    equal, bit for bit, the mix v + 2 sigmoid(gate . h) e quantized with the gate in the append's fixed fp32 order
    (oracle/ve_gate.py:cache_gate)."""
    lengths = [1, 17, 33, 1025, 2049, 300]
    s = State(lengths, 16, 4, steps=1, seed=11, device=device)
    gen = torch.Generator().manual_seed(12)
    vocab = 50
    h = bf16_randn(gen, s.B, C)
    table = bf16_randn(gen, vocab, C)
    gate = (0.05 * torch.randn(s.Hkv, C, generator=gen)).float()
    tokens = torch.randint(0, vocab, (s.B,), generator=gen, dtype=torch.int32)
    ve = tuple(t.to(device) for t in (h, table, gate, tokens))
    ca, cb = s.clone_cache(), s.clone_cache()
    lens = s.lengths.to(device)
    qkv = s.qkv[0].to(device)
    qa, _ = two_launch(s, ca, qkv, lens, -1, s.max_len)
    qb, _ = fused(s, cb, qkv, lens, -1, s.max_len, ve=ve)
    torch.cuda.synchronize()
    assert torch.equal(bits(qa), bits(qb))
    assert torch.equal(ca.k_pages, cb.k_pages) and torch.equal(bits(ca.k_scale), bits(cb.k_scale))
    g = ove.cache_gate(h.float().numpy(), gate.numpy())                               # (B, Hkv) fp32
    v = s.qkv[0].view(s.B, -1)[:, (s.Hq + s.Hkv) * 128:].float().numpy()
    mixed = ove.mix(v, g, tokens.numpy(), table.float().numpy()[:, :s.Hkv * 128])   # head kvh: columns 128 kvh ..
    codes, scales = quantize_rows(mixed.reshape(-1, 128))
    codes, scales = codes.reshape(s.B, s.Hkv, 128), scales.reshape(s.B, s.Hkv)
    for b, n in enumerate(lengths):
        _, _, vc, vs = read_sequence(cb, s.dtable, b, n)
        assert np.array_equal(vc[n - 1], codes[b]), b
        assert np.array_equal(vs[n - 1], scales[b]), b


def test_step_config3u_full_size(device):
    """Config 3u (64 x 8,192 cached + 1, 16/4 heads, 1% outliers, permuted pages): two steps, both paths."""
    w = DECODE["c3u"]
    inp = decode_inputs(w, seed=0)
    s = State.__new__(State)
    s.B, s.Hq, s.Hkv, s.steps, s.device = w.batch, w.q_heads, w.kv_heads, 2, device
    s.max_len = w.ctx + 2
    mp = pages_for(s.max_len)
    s.num_pages = s.B * mp
    gen = torch.Generator().manual_seed(1)
    s.table = torch.randperm(s.num_pages, generator=gen).to(torch.int32).view(s.B, mp)
    s.dtable = s.table.to(device)
    s.cache = PagedKVCache(s.num_pages, s.Hkv, device)
    ctx = inp["ctx_lens"].to(device)
    s.cache.append(inp["k_cache"].to(device), inp["v_cache"].to(device), torch.zeros_like(ctx), s.dtable, num_new=ctx)
    s.lengths = inp["ctx_lens"] + 1
    s.qkv = torch.stack([torch.cat([inp["q"].reshape(s.B, -1), inp["k_new"].reshape(s.B, -1),
                                    inp["v_new"].reshape(s.B, -1)], dim=1)] * 2)
    s.cos, s.sin = rotary_tables(s.max_len, 1e6, device)
    s.gains = (torch.ones(128, device=device), torch.ones(128, device=device))
    torch.cuda.synchronize()
    run_both(s)
