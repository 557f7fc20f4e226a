"""Pins of oracle/cpu_step.py (the PyTorch CPU baseline) against the float64 oracle: the quantizer's codes equal
oracle.quant's, the norm + rotation is within one bf16 step of oracle.rope's (only the sum's order differs), the
stored cache dequantizes to the oracle cache's values, and a decode step and a prefill step match
oracle.attention's decode and prefill attention on the same cache within fp32 accumulation error."""
import numpy as np
import torch

from oracle import cpu_step as cs
from oracle.attention import decode_attention, prefill_attention
from oracle.layout import PagedCache
from oracle.quant import quantize_rows
from oracle.rope import qk_norm_rope, rotary_tables


def bf16_randn(gen, *shape):
    return torch.randn(*shape, generator=gen).to(torch.bfloat16).float()


def test_quantize_matches_oracle():
    gen = torch.Generator().manual_seed(0)
    x = bf16_randn(gen, 300, 128) * torch.exp(torch.randn(300, 1, generator=gen) * 3)
    x[5] = 0
    codes, scale = cs.quantize(x)
    want_c, want_s = quantize_rows(x.numpy())
    assert np.array_equal(codes.numpy(), want_c)
    assert np.array_equal(scale.numpy(), want_s)


def test_norm_rope_within_a_bf16_step_of_oracle():
    gen = torch.Generator().manual_seed(1)
    x = bf16_randn(gen, 64, 4, 128)
    gain = 1 + 0.1 * torch.randn(128, generator=gen)
    cos, sin = rotary_tables(64, 1e6)
    c, s = torch.tensor(cos)[:, None, :], torch.tensor(sin)[:, None, :]
    got = cs.norm_rope(x, gain, c, s).numpy()
    want = qk_norm_rope(x.numpy(), gain.numpy(), cos[:, None, :], sin[:, None, :])
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.maximum(np.abs(want), 1e-3))


def make_case(B=3, Hq=8, Hkv=2, ctx=(40, 17, 90), T=1, seed=2):
    gen = torch.Generator().manual_seed(seed)
    L = max(ctx) + T
    mp = (L + 15) // 16
    table = torch.randperm(B * mp, generator=gen).to(torch.int32).view(B, mp)
    k = bf16_randn(gen, B, max(ctx), Hkv, 128)
    v = bf16_randn(gen, B, max(ctx), Hkv, 128)
    qkv = bf16_randn(gen, B, T, (Hq + 2 * Hkv) * 128)
    gains = 1 + 0.1 * torch.randn(128, generator=gen), 1 + 0.1 * torch.randn(128, generator=gen)
    cos, sin = rotary_tables(L, 1e6)
    cache, ocache = cs.PagedCpuCache(B * mp, Hkv), PagedCache(B * mp, Hkv)
    for b in range(B):
        pos = torch.arange(ctx[b])
        cache.store(table, b, pos, k[b, :ctx[b]], v[b, :ctx[b]])
        ocache.append(table.numpy(), b, pos.numpy(), k[b, :ctx[b]].numpy(), v[b, :ctx[b]].numpy())
    return dict(table=table, qkv=qkv, gains=gains, cos=torch.tensor(cos), sin=torch.tensor(sin), cache=cache,
                ocache=ocache, start=torch.tensor(ctx), Hq=Hq, Hkv=Hkv, T=T)


def oracle_rows(c):
    """The step's q rows and appended cache through the float64 oracle's own functions."""
    B, T = c["qkv"].shape[:2]
    x = c["qkv"].numpy().reshape(B, T, c["Hq"] + 2 * c["Hkv"], 128)
    pos = c["start"].numpy()[:, None] + np.arange(T)[None, :]
    cos, sin = c["cos"].numpy()[pos][:, :, None], c["sin"].numpy()[pos][:, :, None]
    q = qk_norm_rope(x[:, :, :c["Hq"]], c["gains"][0].numpy(), cos, sin)
    k = qk_norm_rope(x[:, :, c["Hq"]:c["Hq"] + c["Hkv"]], c["gains"][1].numpy(), cos, sin)
    v = x[:, :, c["Hq"] + c["Hkv"]:]
    for b in range(B):
        c["ocache"].append(c["table"].numpy(), b, pos[b], k[b], v[b])
    return q


def test_decode_step_matches_oracle():
    c = make_case()
    got = cs.step(c["cache"], c["table"], c["qkv"], c["start"], c["Hq"], c["Hkv"], *c["gains"], c["cos"], c["sin"])
    q = oracle_rows(c)
    want = decode_attention(q[:, 0], c["ocache"], c["table"].numpy(), c["start"].numpy() + 1)
    # the q and k rows may differ by a bf16 rounding of the norm (summation order), so the tolerance is that of a
    # relative 2^-7 perturbation of the scores, not fp32 accumulation alone
    assert np.abs(got[:, 0].numpy() - want).max() <= 2e-2 * np.abs(want).max()
    # the cache: every stored value dequantizes like the oracle's
    for b in range(3):
        n = int(c["start"][b]) + 1
        K, V = c["cache"].gather(c["table"][b:b + 1], torch.tensor([n]))
        Ko, Vo = c["ocache"].gather_values(c["table"].numpy(), b, n)
        assert np.abs(K[0].permute(1, 0, 2).numpy()[:n - 1] - Ko[:n - 1]).max() == 0
        assert np.abs(V[0].permute(1, 0, 2).numpy() - Vo).max() == 0


def test_prefill_step_matches_oracle():
    c = make_case(ctx=(33, 64, 5), T=20, seed=3)
    got = cs.step(c["cache"], c["table"], c["qkv"], c["start"], c["Hq"], c["Hkv"], *c["gains"], c["cos"], c["sin"],
                  window=25)
    q = oracle_rows(c)
    want = prefill_attention(q, c["ocache"], c["table"].numpy(), c["start"].numpy(), window=25)
    assert np.abs(got.numpy() - want).max() <= 2e-2 * np.abs(want).max()
