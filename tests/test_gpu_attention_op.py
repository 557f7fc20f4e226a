"""The registered training attention op (nanochat_amd.attention_op) against torch autograd of the same block in float64
on the CPU: the q/k RMS norm with gains and the -theta rotation, the value-embedding mix (gate 2 sigmoid(n w^T) per
head, table rows rounded to bf16), causal attention inside each document segment (window: keys at distance <= window),
the output projection plus residual, and the rstd of the sum. Forward outputs and every gradient (qkv, both norm
weights, n, the gate weight, the table through table.grad, o_proj's weight through o_grad, the residual) are compared
at bf16 tolerances: max error within 2 % of the largest reference value and mean error within 1 % of the mean
magnitude (the training kernels' own tolerance, tests/test_gpu_flash_attn.py)."""
import numpy as np
import pytest
import torch

from nanochat_amd.attention_op import attention
from nanochat_amd.rotary import rotary_tables

pytestmark = pytest.mark.gpu
EPS = torch.finfo(torch.float32).eps


def rel_check(got, ref, what, max_rel=2e-2, mean_rel=1e-2):
    got = got.detach().double().cpu().numpy()
    ref = ref.detach().double().cpu().numpy()
    err = np.abs(got - ref)
    scale = max(np.abs(ref).max(), 1e-3)
    assert err.max() <= max_rel * scale, (what, err.max(), scale)
    assert err.mean() <= mean_rel * max(np.abs(ref).mean(), 1e-4), (what, err.mean(), np.abs(ref).mean())


def reference(qkv, qnw, knw, cos, sin, window, bounds, o_weight, residual, ve):
    """Float64 forward of the block; bounds: the segments' token offsets over the flattened B*T tokens."""
    B, T, C3 = qkv.shape
    C = C3 // 3
    H = C // 128
    x = qkv.view(B, T, 3, H, 128)

    def norm_rope(t, gain):
        r = t / torch.sqrt(t.square().mean(-1, keepdim=True) + EPS) * gain
        a, b = r[..., :64], r[..., 64:]
        c, s = cos[:T, None, :], sin[:T, None, :]
        return torch.cat([a * c + b * s, b * c - a * s], -1)

    q, k, v = norm_rope(x[:, :, 0], qnw), norm_rope(x[:, :, 1], knw), x[:, :, 2]
    if ve is not None:
        n, ids, table, w = ve
        e = table + (table.to(torch.bfloat16).double() - table).detach()    # bf16 rows, gradient straight through
        g = 2 * torch.sigmoid(n @ w.t())                                        # (B, T, H)
        v = v + g[..., None] * e[ids.long()].view(B, T, H, 128)
    N = B * T
    seg = torch.zeros(N, dtype=torch.long)
    for s0 in bounds[1:-1]:
        seg[s0:] += 1
    i = torch.arange(N)
    ok = (seg[:, None] == seg[None, :]) & (i[None, :] <= i[:, None])
    if window < T:
        ok &= i[:, None] - i[None, :] <= window
    qf, kf, vf = q.reshape(N, H, 128), k.reshape(N, H, 128), v.reshape(N, H, 128)
    s = torch.einsum("ihd,jhd->hij", qf, kf) / 128 ** 0.5
    s = s.masked_fill(~ok, float("-inf"))
    lse = torch.logsumexp(s, -1)
    o = torch.einsum("hij,jhd->ihd", torch.softmax(s, -1), vf)
    h = residual.reshape(N, C) + o.reshape(N, C) @ o_weight.t()
    rstd = 1 / torch.sqrt(h.square().mean(-1) + EPS)
    return h.view(B, T, C), rstd, o.view(B, T, H, 128), lse, q, k


@pytest.mark.parametrize("with_table", [False, True])
@pytest.mark.parametrize("window", [1000, 24])
def test_attention_op_matches_float64_autograd(device, with_table, window):
    B, T, H, vocab = 2, 160, 2, 300
    C = H * 128
    gen = torch.Generator().manual_seed(3 + 2 * with_table + (window < T))
    bf = lambda *s, scale=1.0: (torch.randn(*s, generator=gen) * scale).bfloat16()
    qkv = bf(B, T, 3 * C)
    qnw = 1 + 0.1 * torch.randn(128, generator=gen)
    knw = 1 + 0.1 * torch.randn(128, generator=gen)
    o_weight = bf(C, C, scale=C ** -0.5)
    residual = bf(B, T, C)
    bounds = [0, 50, 160, 161, 250, 320]                  # ragged segments across the row boundary, one of length 1
    cu = torch.tensor(bounds + [320, 320], dtype=torch.int32)   # padded like the reference's buffer
    segments = torch.tensor(len(bounds) - 1)
    cos, sin = rotary_tables(T)
    dh = bf(B, T, C)
    n = bf(B, T, C)
    table = torch.randn(vocab, C, generator=gen)
    w_gate = 0.05 * torch.randn(H, C, generator=gen)
    input_ids = torch.randint(0, vocab, (B, T), generator=gen, dtype=torch.int32)

    # device op
    d = lambda t: t.to(device)
    qkv_d = d(qkv).requires_grad_()
    qnw_d, knw_d = d(qnw).requires_grad_(), d(knw).requires_grad_()
    res_d = d(residual).requires_grad_()
    o_grad = torch.zeros(C, C, device=device)
    if with_table:
        n_d, w_d, tab_d, ids_d = d(n).requires_grad_(), d(w_gate).requires_grad_(), d(table), d(input_ids)
        ve_d = (n_d, ids_d, tab_d, w_d, *torch.sort(ids_d.flatten()))
    else:
        ve_d = (None,) * 6
    outs = attention(qkv_d, qnw_d, knw_d, d(cos), d(sin), window, d(cu), d(segments), d(o_weight), o_grad, res_d,
                     *ve_d)
    h, rstd = outs[:2]
    h.backward(d(dh))
    torch.cuda.synchronize()

    # float64 reference
    dbl = lambda t: t.double().requires_grad_()
    r_qkv, r_qnw, r_knw, r_w, r_res = dbl(qkv), dbl(qnw), dbl(knw), dbl(o_weight), dbl(residual)
    r_ve = None
    if with_table:
        r_n, r_tab, r_wg = dbl(n), dbl(table), dbl(w_gate)
        r_ve = (r_n, input_ids, r_tab, r_wg)
    rh, rrstd, ro, rlse, rq, rk = reference(r_qkv, r_qnw, r_knw, cos.double(), sin.double(), window, bounds, r_w,
                                            r_res, r_ve)
    rh.backward(dh.double())

    rel_check(h, rh, "h")
    rel_check(rstd, rrstd, "rstd")
    rel_check(outs[2], ro, "out")
    assert (outs[3].cpu().double() - rlse).abs().max() <= 5e-2
    rel_check(outs[4], rq, "qn")
    rel_check(outs[5], rk, "kn")
    rel_check(qkv_d.grad, r_qkv.grad, "d qkv")
    rel_check(qnw_d.grad, r_qnw.grad, "d q_norm_weight")
    rel_check(knw_d.grad, r_knw.grad, "d k_norm_weight")
    rel_check(o_grad, r_w.grad, "o_grad")
    assert torch.equal(res_d.grad.cpu(), dh)
    if with_table:
        rel_check(n_d.grad, r_n.grad, "d n")
        rel_check(w_d.grad, r_wg.grad, "d w_gate")
        rel_check(tab_d.grad, r_tab.grad, "table.grad")
    else:
        assert outs[6].numel() == 0 and outs[7].numel() == 0
