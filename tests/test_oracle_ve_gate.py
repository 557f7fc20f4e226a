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
