"""Pins oracle/flash.py: the forward against torch's scaled_dot_product_attention and logsumexp in float64 with an
explicit causal/window mask, the backward against torch autograd of that forward, and the window special cases."""
import numpy as np
import torch

from oracle import flash as of


def case(lengths, H=2, D=128, seed=0):
    rng = np.random.default_rng(seed)
    total = sum(lengths)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    q, k, v, do = (rng.standard_normal((total, H, D)) for _ in range(4))
    return q, k, v, do, cu


def torch_reference(q, k, v, cu, window):
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    outs, lses = [], []
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        mask = torch.tensor(of.visible(b - a, window))
        qs, ks, vs = (t[a:b].transpose(0, 1) for t in (tq, tk, tv))        # (H, n, D)
        outs.append(torch.nn.functional.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask).transpose(0, 1))
        sc = (qs @ ks.transpose(1, 2)) * q.shape[-1] ** -0.5
        lses.append(torch.logsumexp(sc.masked_fill(~mask, -torch.inf), dim=-1))
    return tq, tk, tv, torch.cat(outs), torch.cat(lses, dim=1)


def test_forward_and_backward_match_torch():
    for window in (-1, 5, 40):
        q, k, v, do, cu = case([1, 7, 33, 64], seed=window + 2)
        tq, tk, tv, out, lse = torch_reference(q, k, v, cu, window)
        o, l = of.varlen_forward(q, k, v, cu, window)
        assert np.allclose(o, out.detach().numpy(), atol=1e-12)
        assert np.allclose(l, lse.detach().numpy(), atol=1e-12)
        (out * torch.tensor(do)).sum().backward()
        dq, dk, dv = of.varlen_backward(q, k, v, do, cu, window)
        for mine, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
            assert np.allclose(mine, ref.numpy(), atol=1e-11)


def test_window_special_cases():
    q, k, v, _, cu = case([50, 13], seed=9)
    full, lf = of.varlen_forward(q, k, v, cu, -1)
    wide, lw = of.varlen_forward(q, k, v, cu, 49)
    assert np.array_equal(full, wide) and np.array_equal(lf, lw)
    own, _ = of.varlen_forward(q, k, v, cu, 0)
    assert np.allclose(own, v)
