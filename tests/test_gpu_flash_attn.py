"""Training attention forward (csrc/flash_attn.hip) against oracle/flash.py in float64: ragged segments (1 token up
to several 128-row tiles), full causal and windows (0, inside a tile, across tiles), strided q/v views of a fused
projection, max_seqlen above the longest segment, several heads. Tolerance: the north star's bf16 bound on outputs
(max abs 2e-2, mean abs 2e-3) and 1e-4 on the natural-log lse."""
import numpy as np
import pytest
import torch

from nanochat_amd.flash_attn import flash_attn_bwd, flash_attn_bwd_rows, flash_attn_fwd
from oracle import flash as of

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def make(lengths, H, seed, fused=False):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    if fused:   # q, k, v as views of one (total, 3 H 128) projection
        qkv = torch.randn(total, 3, H, 128, generator=gen).bfloat16()
        return qkv[:, 0], qkv[:, 1], qkv[:, 2], cu, qkv
    q, k, v = (torch.randn(total, H, 128, generator=gen).bfloat16() for _ in range(3))
    return q, k, v, cu, None


def run(device, q, k, v, cu, max_seqlen, window, base=None):
    if base is not None:
        b = base.to(device)
        qd, kd, vd = b[:, 0], b[:, 1], b[:, 2]
    else:
        qd, kd, vd = q.to(device), k.to(device), v.to(device)
    out, lse = flash_attn_fwd(qd, kd, vd, cu.to(device), max_seqlen, window_left=window)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), lse.cpu().numpy()


def check(q, k, v, cu, window, out, lse):
    ref, ref_lse = of.varlen_forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu.numpy(),
                                     -1 if window is None else window)
    err = np.abs(out - ref)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (err.max(), err.mean())
    assert np.abs(lse - ref_lse).max() <= 1e-4, np.abs(lse - ref_lse).max()


@pytest.mark.parametrize("window", [None, 0, 37, 200])
@pytest.mark.parametrize("lengths,H", [([1, 17, 128, 200, 513, 64], 3), ([300], 1), ([129, 127, 2, 256], 2)])
def test_forward_matches_oracle(device, lengths, H, window):
    q, k, v, cu, _ = make(lengths, H, seed=len(lengths) * 10 + H)
    out, lse = run(device, q, k, v, cu, max(lengths), window)
    check(q, k, v, cu, window, out, lse)


def test_fused_views_and_larger_max_seqlen(device):
    lengths = [70, 300, 5]
    q, k, v, cu, qkv = make(lengths, 4, seed=3, fused=True)
    out, lse = run(device, q, k, v, cu, 1024, None, base=qkv)
    check(q, k, v, cu, None, out, lse)


def test_training_shape_against_float32_sdpa(device):
    """One 2048-token segment (the training sequence length), 6 heads: outputs against float32 SDPA on the GPU."""
    gen = torch.Generator().manual_seed(11)
    T, H = 2048, 6
    q, k, v = (torch.randn(T, H, 128, generator=gen).bfloat16().to(device) for _ in range(3))
    cu = torch.tensor([0, T], dtype=torch.int32, device=device)
    out, lse = flash_attn_fwd(q, k, v, cu, T)
    ref = torch.nn.functional.scaled_dot_product_attention(*(t.float().transpose(0, 1) for t in (q, k, v)),
                                                           is_causal=True).transpose(0, 1)
    err = (out.float() - ref).abs()
    assert err.max().item() <= MAX_ABS and err.mean().item() <= MEAN_ABS


def rel_check(got, ref, max_rel=2e-2, mean_rel=1e-2):
    """bf16 gradients: max error against the largest reference value, mean error against the mean magnitude (floors
    of 1e-3 and 1e-4: with window 0 dq and dk are exactly zero and the device's are rounding noise)."""
    err = np.abs(got - ref)
    scale = max(np.abs(ref).max(), 1e-3)
    assert err.max() <= max_rel * scale, (err.max(), scale)
    assert err.mean() <= mean_rel * max(np.abs(ref).mean(), 1e-4), (err.mean(), np.abs(ref).mean())


@pytest.mark.parametrize("window", [None, 0, 37, 200])
@pytest.mark.parametrize("lengths,H", [([1, 17, 128, 200, 513, 64], 3), ([129, 127, 2, 256], 2)])
def test_backward_matches_oracle(device, lengths, H, window):
    q, k, v, cu, _ = make(lengths, H, seed=len(lengths) * 7 + H)
    gen = torch.Generator().manual_seed(99)
    dout = torch.randn(q.shape, generator=gen).bfloat16()
    qd, kd, vd, dod, cud = (t.to(device) for t in (q, k, v, dout, cu))
    out, lse = flash_attn_fwd(qd, kd, vd, cud, max(lengths), window_left=window)
    dq, dk, dv = flash_attn_bwd(qd, kd, vd, out, dod, lse, cud, max(lengths), window_left=window)
    torch.cuda.synchronize()
    w = -1 if window is None else window
    rdq, rdk, rdv = of.varlen_backward(q.float().numpy(), k.float().numpy(), v.float().numpy(), dout.float().numpy(),
                                       cu.numpy(), w)
    for got, ref in ((dq, rdq), (dk, rdk), (dv, rdv)):
        rel_check(got.float().cpu().numpy(), ref)


def test_backward_rows_and_strided_dv(device):
    """rows given (the reference passes D from the o_proj epilogue), dv written into the v block of a fused
    gradient, v a view of the fused projection."""
    lengths, H = [300, 40], 2
    q, k, v, cu, qkv = make(lengths, H, seed=4, fused=True)
    gen = torch.Generator().manual_seed(5)
    dout = torch.randn(q.shape, generator=gen).bfloat16().to(device)
    base = qkv.to(device)
    qd, kd, vd, cud = base[:, 0], base[:, 1], base[:, 2], cu.to(device)
    out, lse = flash_attn_fwd(qd, kd, vd, cud, 300)
    rows = flash_attn_bwd_rows(out, dout)
    ref_rows = (out.float() * dout.float()).sum(-1)
    assert torch.allclose(rows, ref_rows, rtol=1e-5, atol=1e-4)
    dqkv = torch.zeros_like(base)
    dq, dk, dv = flash_attn_bwd(qd, kd, vd, out, dout, lse, cud, 300, rows=rows, dv=dqkv[:, 2])
    torch.cuda.synchronize()
    assert dv.data_ptr() == dqkv[:, 2].data_ptr() and torch.equal(dqkv[:, 0], torch.zeros_like(dqkv[:, 0]))
    rdq, rdk, rdv = of.varlen_backward(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                       dout.float().cpu().numpy(), cu.numpy(), -1)
    for got, ref in ((dq, rdq), (dk, rdk), (dqkv[:, 2], rdv)):
        rel_check(got.float().cpu().numpy(), ref)


def test_backward_training_shape_against_autograd(device):
    """One 2048-token segment, 6 heads: gradients against float32 autograd of causal SDPA on the GPU."""
    gen = torch.Generator().manual_seed(12)
    T, H = 2048, 6
    q, k, v, do = (torch.randn(T, H, 128, generator=gen).bfloat16().to(device) for _ in range(4))
    cu = torch.tensor([0, T], dtype=torch.int32, device=device)
    out, lse = flash_attn_fwd(q, k, v, cu, T)
    dq, dk, dv = flash_attn_bwd(q, k, v, out, do, lse, cu, T)
    ref = [t.float().transpose(0, 1).contiguous().requires_grad_() for t in (q, k, v)]
    o = torch.nn.functional.scaled_dot_product_attention(*ref, is_causal=True)
    o.backward(do.float().transpose(0, 1))
    for got, r in ((dq, ref[0]), (dk, ref[1]), (dv, ref[2])):
        rel_check(got.float().cpu().numpy(), r.grad.transpose(0, 1).cpu().numpy())
