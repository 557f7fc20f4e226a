"""Pins oracle/ve_gate.py: forward and gradients against torch autograd of the float64 expression
out = v + 2 sigmoid(n w^T)[head] * e, the mix's fp32 roundings against torch's CPU float32 ops, and the special
cases (zero gate weights give gate 1; a token outside the table mixes in nothing and gets no gradient)."""
import numpy as np
import torch

from oracle import ve_gate as ov
from oracle.numerics import bf16_round

HEAD_DIM = 128


def bf16(x):
    return bf16_round(np.asarray(x, np.float32))


def bf16_ulp(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def case(rows=96, H=3, vocab=40, seed=0):
    rng = np.random.default_rng(seed)
    C = H * HEAD_DIM
    n = bf16(rng.standard_normal((rows, C)))
    v = bf16(rng.standard_normal((rows, C)))
    table = bf16(rng.standard_normal((vocab, C)))          # already bf16: bf16(table) = table
    w = (rng.standard_normal((H, C)) * 0.05).astype(np.float32)
    idx = rng.integers(0, vocab, rows)
    dout = bf16(rng.standard_normal((rows, C)))
    return n, v, table, w, idx, dout


def autograd(n, v, table, w, idx, dout):
    H = w.shape[0]
    tn = torch.tensor(n, dtype=torch.float64, requires_grad=True)
    tw = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    tt = torch.tensor(table, dtype=torch.float64, requires_grad=True)
    z = tn @ tw.T
    z.retain_grad()
    g = 2 * torch.sigmoid(z)
    e = tt[torch.tensor(idx)]
    out = torch.tensor(v, dtype=torch.float64) + (g[:, :, None] * e.view(-1, H, HEAD_DIM)).view(e.shape)
    (out * torch.tensor(dout, dtype=torch.float64)).sum().backward()
    return (out.detach().numpy(), g.detach().numpy(), z.grad.numpy(), tn.grad.numpy(), tw.grad.numpy(),
            tt.grad.numpy())


def test_forward_and_gradients_match_autograd():
    n, v, table, w, idx, dout = case()
    out64, g64, dz64, dn64, dw64, dtab64 = autograd(n, v, table, w, idx, dout)
    out, g = ov.ve_forward(n, v, idx, table, w)
    assert np.allclose(g, g64, rtol=1e-13, atol=0)
    assert np.all(np.abs(out - out64) <= bf16_ulp(out64) * 0.5 + 2.0 ** -23 * np.abs(out64))

    order = np.argsort(idx, kind="stable")
    ids = idx[order]
    g32 = g.astype(np.float32)
    dz, dn, dtab = ov.ve_backward(dout, ids, order, table, w, g32)
    # the oracle's s is the fp32 gate / 2: relative 2^-24 on s and 1 - s
    assert np.allclose(dz, dz64, rtol=1e-6, atol=1e-12)
    assert np.all(np.abs(dn - dn64) <= (np.abs(dz64) * 1e-6) @ np.abs(w).astype(np.float64) + 1e-12)
    # each table term is bf16(g dout): at most half a bf16 ulp (2^-9 relative) from the exact product
    tok_terms = np.abs(np.repeat(g32, HEAD_DIM, axis=1) * dout).astype(np.float64)
    bound = np.zeros_like(dtab)
    np.add.at(bound, idx, tok_terms)
    assert np.all(np.abs(dtab - dtab64) <= bound * 2.0 ** -8 + 1e-12)
    dzb = bf16(dz.astype(np.float32))
    dw = ov.weight_grad(dzb, n)
    assert np.all(np.abs(dw - dw64) <= (np.abs(dz).T @ np.abs(n)) * 2.0 ** -8 + 1e-9)


def test_mix_rounding_matches_torch_float32():
    n, v, table, w, idx, _ = case(seed=1)
    g = ov.gate(n, w).astype(np.float32)
    ref = (torch.tensor(v) + torch.tensor(np.repeat(g, HEAD_DIM, axis=1)) *
           torch.tensor(table[idx]).bfloat16().float()).bfloat16().float().numpy()
    assert np.array_equal(ov.mix(v, g, idx, table), ref)


def test_zero_weights_give_gate_one():
    n, v, table, w, idx, _ = case(seed=2)
    out, g = ov.ve_forward(n, v, idx, table, np.zeros_like(w))
    assert np.all(g == 1.0)
    assert np.array_equal(out, bf16((v + table[idx]).astype(np.float32)))


def test_token_outside_table_mixes_nothing():
    n, v, table, w, idx, dout = case(seed=3)
    idx = idx.copy()
    idx[::7] = table.shape[0] + 5
    idx[1::7] = -1
    out, g = ov.ve_forward(n, v, idx, table, w)
    bad = (idx < 0) | (idx >= table.shape[0])
    assert np.array_equal(out[bad], v[bad])
    order = np.argsort(idx, kind="stable")
    dz, dn, dtab = ov.ve_backward(dout, idx[order], order, table, w, g.astype(np.float32))
    assert np.all(dz[bad] == 0) and np.all(dn[bad] == 0)
    good = ~bad
    ref = np.zeros_like(dtab)
    np.add.at(ref, idx[good], bf16((np.repeat(g.astype(np.float32), HEAD_DIM, axis=1) * dout).astype(np.float32))[good])
    assert np.array_equal(dtab, ref)


def rn32(x):
    """The fp32 value nearest the rational x (ties to an even significand)."""
    from fractions import Fraction
    f = np.float32(float(x))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - x), int(np.array(c).view(np.uint32)) & 1))
    return np.float32(best)


def test_fma32_is_one_rounding_of_the_exact_value():
    """Random operands over many exponents, and the constructed midpoint cases: 205 x 5,237,765 = 2^30 + 1, so
    a = 205 / 128 (bf16) times b = 5,237,765 / 2^22 (fp32) is 2^1 + 2^-29, and 2^25 + a b lies 2^-29 above the
    midpoint of the floats 2^25 and 2^25 + 4 while its float64 sum is that midpoint (the sum's error is 2^-29)."""
    from fractions import Fraction
    rng = np.random.default_rng(3)
    a = bf16(rng.standard_normal(4000) * 2.0 ** rng.integers(-20, 20, 4000))
    b = (rng.standard_normal(4000) * 2.0 ** rng.integers(-20, 20, 4000)).astype(np.float32)
    c = (rng.standard_normal(4000) * 2.0 ** rng.integers(-30, 30, 4000)).astype(np.float32)
    ta, tb = np.float32(205 / 128), np.float32(5237765 / 2 ** 22)
    assert float(ta) * float(tb) == 2.0 + 2.0 ** -29
    a = np.concatenate([a, [ta, -ta, ta, ta]]).astype(np.float32)
    b = np.concatenate([b, [tb, tb, -tb, tb]]).astype(np.float32)
    c = np.concatenate([c, [2.0 ** 25, -2.0 ** 25, 2.0 ** 25, 0.0]]).astype(np.float32)
    got = ov.fma32(a, b, c)
    for x, y, z, g in zip(a, b, c, got):
        want = rn32(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)))
        assert g == want, (x, y, z, g, want)
    assert got[-4] == np.float32(2.0 ** 25 + 4) and got[-3] == np.float32(-(2.0 ** 25 + 4))
    # plain float64-then-float32 rounding lands on the even neighbour, 2^25: the case the correction exists for
    assert np.float32(float(ta) * float(tb) + 2.0 ** 25) == np.float32(2.0 ** 25)


def test_cache_gate_is_the_gate_within_its_fp32_error():
    """cache_gate against the float64 gate: each FMA chain, butterfly add, exponential, add, divide and scale rounds
    once to fp32, so |g - g64| <= 0.5 (C / 64 + 6) 2^-24 sum |n w| + 10 2^-24 (sigmoid' <= 1/4, times 2; g <= 2);
    widths that are and are not multiples of 64; zero weights give exactly 1."""
    rng = np.random.default_rng(4)
    for C in (768, 1664, 200, 64, 1):
        n = bf16(rng.standard_normal((37, C)))
        w = (rng.standard_normal((5, C)) * rng.choice([0.01, 0.05, 0.3])).astype(np.float32)
        g = ov.cache_gate(n, w)
        assert g.dtype == np.float32 and g.shape == (37, 5)
        g64 = ov.gate(n, w)
        mag = np.abs(n.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
        tol = 0.5 * (C / 64 + 6) * 2.0 ** -24 * mag + 10 * 2.0 ** -24
        assert (np.abs(g - g64) <= tol).all(), (C, float(np.abs(g - g64).max()))
        assert (ov.cache_gate(n, np.zeros_like(w)) == 1.0).all()
