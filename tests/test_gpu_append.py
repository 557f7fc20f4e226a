"""GPU parity of the append entry points against the oracle: fp8 cache bytes and scales bit-exact, q/k after
the fused norm + rotation bit-exact (bf16)."""
import dataclasses
from pathlib import Path

import numpy as np
import pytest
import torch

from nanochat_amd.attention import qk_norm_rope_append
from nanochat_amd.kv_cache import PagedKVCache, contiguous_block_table, permuted_block_table
from nanochat_amd.qk_prologue import qk_forward
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.workloads import DECODE, decode_inputs
from oracle.layout import K_OFF, PAGE, V_OFF
from oracle.numerics import bf16_bits, bf16_to_f32
from oracle.rope import qk_norm_rope
from tests.paged_util import device_cache, expected_codes, f32, read_sequence

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def append_rows(rows: np.ndarray, device) -> tuple:
    """Append fp32-held bf16 rows (n, 128) as n tokens of one KV head of one sequence; read them back."""
    n = rows.shape[0]
    x = torch.from_numpy(rows).to(torch.bfloat16).view(1, n, 1, 128).to(device)
    mp = (n + 15) // 16
    table = contiguous_block_table(1, mp, device)
    cache = PagedKVCache(mp, 1, device)
    cache.append(x, x, torch.zeros(1, dtype=torch.int32, device=device), table)
    torch.cuda.synchronize()
    return read_sequence(cache, table, 0, n)


def test_every_bf16_value(device):
    """All finite bf16 bit patterns, grouped by magnitude (each row spans a narrow range, so every code of
    every binade appears) and shuffled (each row mixes magnitudes)."""
    x = bf16_to_f32(np.arange(1 << 16, dtype=np.uint32).astype(np.uint16))
    x = x[np.isfinite(x)]
    pad = (-x.size) % 128
    x = np.concatenate([x, np.zeros(pad, np.float32)])
    by_mag = x[np.argsort(np.abs(x), kind="stable")].reshape(-1, 128)
    shuffled = x[np.random.default_rng(0).permutation(x.size)].reshape(-1, 128)
    for rows in (by_mag, shuffled):
        kc, ks, vc, vs = append_rows(rows, device)
        wc, ws, _, _ = expected_codes(rows[:, None], rows[:, None])
        assert np.array_equal(kc, wc) and np.array_equal(vc, wc)
        assert np.array_equal(ks, ws) and np.array_equal(vs, ws)


@pytest.mark.parametrize("name", ["c1", "c3"])
def test_cache_bytes_match_oracle(device, name):
    w = DECODE[name]
    if name == "c3":   # the ragged outlier workload at 6 sequences
        w = dataclasses.replace(w, batch=6, name="c3-small")
    inp = decode_inputs(w, seed=0)
    cache, table, lens = device_cache(inp, w.kv_heads, device)
    for b in range(w.batch):
        n = int(inp["ctx_lens"][b])
        got = read_sequence(cache, table, b, n + 1)
        k = np.concatenate([f32(inp["k_cache"][b, :n]), f32(inp["k_new"][b])])
        v = np.concatenate([f32(inp["v_cache"][b, :n]), f32(inp["v_new"][b])])
        for g, e in zip(got, expected_codes(k, v)):
            assert np.array_equal(g, e)


def test_config1_golden_bytes(device):
    want = np.load(GOLDEN / "config1.npz")
    inp = decode_inputs(DECODE["c1"], seed=0)
    cache, table, _ = device_cache(inp, 6, device)
    kc, ks, vc, vs = read_sequence(cache, table, 0, 1025)
    assert np.array_equal(kc, want["k_codes"]) and np.array_equal(ks, want["k_scale"])
    assert np.array_equal(vc, want["v_codes"]) and np.array_equal(vs, want["v_scale"])


@pytest.mark.parametrize("Hq,Hkv,theta", [(8, 2, 1e4), (6, 6, 1e6), (16, 4, 1e4)])
def test_fused_norm_rope_append(device, Hq, Hkv, theta):
    B, T = 3, 37
    gen = torch.Generator().manual_seed(Hq * 100 + Hkv)
    qkv = (torch.randn(B, T, (Hq + 2 * Hkv) * 128, generator=gen) * 2).to(torch.bfloat16)
    qg = 1 + 0.1 * torch.randn(128, generator=gen)
    kg = 1 + 0.1 * torch.randn(128, generator=gen)
    start = torch.tensor([0, 5, 100], dtype=torch.int32)
    cos, sin = rotary_tables(256, theta)
    mp = (100 + T + 15) // 16
    table = permuted_block_table(B, mp, gen, device)
    cache = PagedKVCache(B * mp, Hkv, device)
    q = qk_norm_rope_append(qkv.to(device), Hq, cache, table, start.to(device), qg.to(device), kg.to(device),
                            cos.to(device), sin.to(device))
    torch.cuda.synchronize()
    x = f32(qkv).reshape(B, T, Hq + 2 * Hkv, 128)
    for b in range(B):
        pos = int(start[b]) + np.arange(T)
        c, s = cos.numpy()[pos][:, None], sin.numpy()[pos][:, None]
        wq = qk_norm_rope(x[b, :, :Hq], qg.numpy(), c, s)
        assert np.array_equal(bf16_bits(wq), q[b].view(torch.int16).cpu().numpy().view(np.uint16))
        wk = qk_norm_rope(x[b, :, Hq:Hq + Hkv], kg.numpy(), c, s)
        got = read_sequence(cache, table, b, int(pos[-1]) + 1)
        got = [a[pos] for a in got]
        for g, e in zip(got, expected_codes(wk, x[b, :, Hq + Hkv:])):
            assert np.array_equal(g, e)


def test_qk_forward_matches_oracle(device):
    B, T, H = 2, 33, 6
    gen = torch.Generator().manual_seed(3)
    qkv = torch.randn(B, T, 3, H, 128, generator=gen).to(torch.bfloat16).to(device)
    qg = (1 + 0.1 * torch.randn(128, generator=gen)).to(device)
    kg = (1 + 0.1 * torch.randn(128, generator=gen)).to(device)
    cos, sin = rotary_tables(T, 1e6, device)
    q, k = qkv[:, :, 0], qkv[:, :, 1]
    qo, ko = qk_forward(q, k, qg, kg, cos, sin)
    torch.cuda.synchronize()
    c, s = cos.cpu().numpy()[None, :, None], sin.cpu().numpy()[None, :, None]
    for got, x, g in ((qo, q, qg), (ko, k, kg)):
        want = qk_norm_rope(f32(x), g.cpu().numpy(), c, s)
        assert np.array_equal(bf16_bits(want), got.view(torch.int16).cpu().numpy().view(np.uint16))


def test_golden_rope_vectors(device):
    """The committed q/k-norm + rotation vectors (tests/golden/rope.npz): each row appended as the q head of its own
    sequence at its position (the fused append, the product's rotary tables) and, as the k head, through the training
    prologue at the same position, gives the committed bf16 bits."""
    want = np.load(GOLDEN / "rope.npz")
    x = torch.from_numpy(want["x_bf16"].view(np.int16)).view(torch.bfloat16)
    pos = want["row_positions"]
    n = x.shape[0]
    gain = torch.from_numpy(want["gain"]).to(device)
    cos, sin = rotary_tables(int(pos.max()) + 1, 1e6, device)
    # fused append: sequence i holds row i as its q head (and as k and v) at position pos[i]
    qkv = x.view(n, 1, 1, 128).expand(n, 1, 3, 128).reshape(n, 1, 3 * 128).contiguous().to(device)
    mp = int(pos.max()) // 16 + 1
    table = contiguous_block_table(n, mp, device)
    cache = PagedKVCache(n * mp, 1, device)
    q = qk_norm_rope_append(qkv, 1, cache, table, torch.from_numpy(pos.astype(np.int32)).to(device), gain, gain,
                            cos, sin)
    torch.cuda.synchronize()
    assert np.array_equal(q.view(torch.int16).cpu().numpy().view(np.uint16).reshape(n, 128), want["y_bf16"])
    # training prologue: one sequence of pos.max() + 1 tokens, row i placed at token pos[i] of head 0 of k
    T = int(pos.max()) + 1
    for i in range(n):
        fused = torch.zeros(1, T, 3, 1, 128, dtype=torch.bfloat16)
        fused[0, pos[i], 1, 0] = x[i]
        fused = fused.to(device)
        _, ko = qk_forward(fused[:, :, 0], fused[:, :, 1], gain, gain, cos, sin)
        torch.cuda.synchronize()
        assert np.array_equal(ko[0, pos[i], 0].view(torch.int16).cpu().numpy().view(np.uint16), want["y_bf16"][i]), i


def test_append_skips_out_of_range_pages(device):
    """A position past the block table, or a table entry outside the pool, writes nothing."""
    cache = PagedKVCache(2, 1, device)
    table = torch.tensor([[1, 7]], dtype=torch.int32, device=device)     # page 7 is outside the pool
    x = torch.ones(1, 3, 1, 128, dtype=torch.bfloat16, device=device)
    cache.append(x, x, torch.tensor([15], dtype=torch.int32, device=device), table)   # positions 15, 16, 17
    torch.cuda.synchronize()
    assert cache.k_scale[1, 0, 15].item() == pytest.approx(1 / 448)
    assert int(cache.k_pages[0].count_nonzero()) == 0 and cache.k_scale[0].abs().sum().item() == 0
    assert int(cache.k_pages[1].count_nonzero()) == 128


@pytest.mark.parametrize("B,T,H", [(2, 33, 6), (4, 512, 6), (1, 1, 1)])
def test_qk_backward_matches_oracle(device, B, T, H):
    """dq, dk within one bf16 rounding of the float64 backward plus fp32 error; the gains' gradients within the
    rigorous bound of their fp32 summation depth; bitwise repeatable; the v third of the gradient buffer untouched."""
    from nanochat_amd.qk_prologue import qk_backward
    from oracle.rope import qk_norm_rope_backward

    gen = torch.Generator().manual_seed(B * 100 + T + H)
    qkv = torch.randn(B, T, 3, H, 128, generator=gen).to(torch.bfloat16)
    dout = torch.randn(2, B, T, H, 128, generator=gen).to(torch.bfloat16)
    gains = 1 + 0.1 * torch.randn(2, 128, generator=gen)
    cos, sin = rotary_tables(T, 1e4, device)
    qkv_d, dout_d, g_d = qkv.to(device), dout.to(device), gains.to(device)

    def run():
        dqkv = torch.full_like(qkv_d, 7.0)
        dgq, dgk = qk_backward(qkv_d[:, :, 0], qkv_d[:, :, 1], g_d[0], g_d[1], dout_d[0], dout_d[1], cos, sin,
                               dqkv[:, :, 0], dqkv[:, :, 1])
        torch.cuda.synchronize()
        return dqkv.cpu(), dgq.cpu(), dgk.cpu()

    dqkv, dgq, dgk = run()
    again = run()
    assert all(torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a, b.view(torch.int16) if
                           b.dtype == torch.bfloat16 else b) for a, b in zip((dqkv, dgq, dgk), again))
    assert bool((dqkv[:, :, 2] == 7.0).all())
    rows = B * T * H
    c = cos.cpu().numpy()[None, :, None].astype(np.float64)
    s = sin.cpu().numpy()[None, :, None].astype(np.float64)
    for j, dg in ((0, dgq), (1, dgk)):
        x = qkv[:, :, j].double().numpy()
        dy = dout[j].double().numpy()
        dx, want_dg = qk_norm_rope_backward(x, gains[j].double().numpy(), c, s, dy)
        got = dqkv[:, :, j].double().numpy()
        row_scale = np.abs(dx).max(axis=-1, keepdims=True)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(dx), 2.0 ** -126))) - 7)
        assert np.all(np.abs(got - dx) <= ulp + 1e-5 * row_scale)
        # |dm n| summed over rows: the scale of the fp32 summation error, depth rows/2048 + 4 + QKB_BLOCKS
        d1, d2 = dy[..., :64], dy[..., 64:]
        dm = np.concatenate([d1 * c - d2 * s, d1 * s + d2 * c], axis=-1)
        n = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 2.0 ** -23)
        mag = np.abs(dm * n).reshape(-1, 128).sum(axis=0)
        depth = rows // 2048 + 4 + 512
        assert np.all(np.abs(dg.double().numpy() - want_dg) <= depth * 2.0 ** -24 * mag + 1e-30)


def test_partial_pages_keep_the_other_slots(device):
    """Appends that start and end inside pages (misaligned starts, num_new shorter than T, new positions filling part
    of one page, a V block's four slots split between old and new) change exactly the new positions' codes and
    scales: the whole pool after the append, every other slot's bytes included, equals the pool before it with the
    oracle's codes and scales put at the new positions."""
    gen = torch.Generator().manual_seed(5)
    B, Hkv, mp, T = 3, 2, 6, 20
    table = permuted_block_table(B, mp, gen, device)
    cache = PagedKVCache(B * mp, Hkv, device)
    old = (torch.randn(B, 90, Hkv, 128, generator=gen) * 3).to(torch.bfloat16)
    cache.append(old.to(device), old.flip(3).contiguous().to(device), torch.zeros(B, dtype=torch.int32, device=device),
                 table)
    torch.cuda.synchronize()
    kp, vp, sc = (t.cpu().numpy().copy() for t in (cache.k_pages, cache.v_pages, cache.kv_scale))
    k = torch.randn(B, T, Hkv, 128, generator=gen).to(torch.bfloat16)
    v = (torch.randn(B, T, Hkv, 128, generator=gen) * 0.01).to(torch.bfloat16)
    start, num_new = [37, 5, 66], [13, 20, 3]
    cache.append(k.to(device), v.to(device), torch.tensor(start, dtype=torch.int32, device=device), table,
                 torch.tensor(num_new, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    kc, ks, vc, vs = expected_codes(f32(k).reshape(B * T, Hkv, 128), f32(v).reshape(B * T, Hkv, 128))
    tab = table.cpu().numpy()
    for b in range(B):
        for t in range(num_new[b]):
            p = start[b] + t
            page, slot, r = tab[b, p // PAGE], p % PAGE, b * T + t
            kp[page, :, K_OFF[slot]] = kc[r].T
            vp[page, :, V_OFF[slot]] = vc[r].T
            sc[page, :, 0, slot], sc[page, :, 1, slot] = ks[r], vs[r]
    assert np.array_equal(cache.k_pages.cpu().numpy(), kp)
    assert np.array_equal(cache.v_pages.cpu().numpy(), vp)
    assert np.array_equal(cache.kv_scale.cpu().numpy(), sc)


def test_prefill_append_runs_with_value_embeddings(device):
    """The decoder's prefill append (dec_debug_append_runs) over runs of rows: misaligned starts, two runs of one slot
    writing the two halves of one page (a V block split between them), a width C that is not a multiple of 64. q rows
    and K codes equal the oracle's norm + rotation bit for bit; V codes and scales equal the value-embedding mix with
    the gate in the append's fixed fp32 order (oracle/ve_gate.py:cache_gate), quantized; every other byte of the pool
    keeps its value."""
    from nanochat_amd.native import hip_library, pointer, stream
    from oracle import ve_gate as ove

    Hq, Hkv, C, vocab, mp, pool = 4, 2, 300, 23, 4, 16
    runs = [(1, 5, 20), (0, 37, 3), (2, 0, 38), (1, 25, 7)]          # (slot, start, count)
    rows = sum(r[2] for r in runs)
    gen = torch.Generator().manual_seed(21)
    qkv = (torch.randn(rows, (Hq + 2 * Hkv) * 128, generator=gen) * 2).to(torch.bfloat16)
    qg = 1 + 0.1 * torch.randn(128, generator=gen)
    kg = 1 + 0.1 * torch.randn(128, generator=gen)
    h = torch.randn(rows, C, generator=gen).to(torch.bfloat16)
    table = torch.randn(vocab, C, generator=gen).to(torch.bfloat16)
    gate = (0.05 * torch.randn(Hkv, C, generator=gen)).float()
    tokens = torch.randint(0, vocab, (rows,), generator=gen, dtype=torch.int32)
    bt = torch.randperm(pool, generator=gen)[:3 * mp].view(3, mp).to(torch.int32)
    cos, sin = rotary_tables(64, 1e4)
    k_pages = torch.randint(0, 256, (pool, Hkv, 2048), generator=gen, dtype=torch.uint8)
    v_pages = torch.randint(0, 256, (pool, Hkv, 2048), generator=gen, dtype=torch.uint8)
    scales = torch.rand(pool, Hkv, 2, 16, generator=gen)
    row0 = np.cumsum([0] + [r[2] for r in runs[:-1]]).astype(np.int32)
    meta = [torch.tensor(x, dtype=torch.int32) for x in (row0, [r[2] for r in runs], [r[1] for r in runs],
                                                         [r[0] for r in runs])]
    d = {k: t.to(device) for k, t in dict(qkv=qkv, qg=qg, kg=kg, h=h, table=table, gate=gate, tokens=tokens, bt=bt,
                                          cos=cos, sin=sin, kp=k_pages, vp=v_pages, sc=scales).items()}
    dm = [t.to(device) for t in meta]
    q_out = torch.zeros(rows, Hq, 128, dtype=torch.bfloat16, device=device)
    rc = hip_library("decode").dec_debug_append_runs(
        pointer(d["qkv"]), (Hq + 2 * Hkv) * 128, len(runs), max(r[2] for r in runs), *(pointer(t) for t in dm), Hq, Hkv,
        pointer(d["qg"]), pointer(d["kg"]), pointer(d["cos"]), pointer(d["sin"]), 64, pointer(q_out), pointer(d["bt"]),
        mp, pointer(d["kp"]), pointer(d["vp"]), pointer(d["sc"]), pool, pointer(d["h"]), pointer(d["table"]),
        pointer(d["gate"]), pointer(d["tokens"]), C, stream())
    assert rc == 0, rc
    torch.cuda.synchronize()

    x = f32(qkv).reshape(rows, Hq + 2 * Hkv, 128)
    pos = np.concatenate([np.arange(r[1], r[1] + r[2]) for r in runs])
    slot = np.concatenate([np.full(r[2], r[0]) for r in runs])
    c, s = cos.numpy()[pos][:, None], sin.numpy()[pos][:, None]
    wq = qk_norm_rope(x[:, :Hq], qg.numpy(), c, s)
    assert np.array_equal(bf16_bits(wq), q_out.view(torch.int16).cpu().numpy().view(np.uint16))
    wk = qk_norm_rope(x[:, Hq:Hq + Hkv], kg.numpy(), c, s)
    g = ove.cache_gate(f32(h), gate.numpy())                                            # (rows, Hkv)
    v = ove.mix(x[:, Hq + Hkv:].reshape(rows, Hkv * 128), g, tokens.numpy(), f32(table)[:, :Hkv * 128])
    kc, ks, vc, vs = expected_codes(wk, v.reshape(rows, Hkv, 128))
    kp, vp, sc = k_pages.numpy().copy(), v_pages.numpy().copy(), scales.numpy().copy()
    tab = bt.numpy()
    for r in range(rows):
        page, sl = tab[slot[r], pos[r] // PAGE], pos[r] % PAGE
        kp[page, :, K_OFF[sl]] = kc[r].T
        vp[page, :, V_OFF[sl]] = vc[r].T
        sc[page, :, 0, sl], sc[page, :, 1, sl] = ks[r], vs[r]
    assert np.array_equal(d["kp"].cpu().numpy(), kp)
    assert np.array_equal(d["vp"].cpu().numpy(), vp)
    assert np.array_equal(d["sc"].cpu().numpy(), sc)
