"""The value-embedding gate and mix (csrc/ve_gate.hip) against oracle/ve_gate.py: the gate within its fp32
accumulation bound of the exact float64 gate, the mix bit-exact given the device's gate, the backward's dz, dn, table
gradient and dw within their propagated fp32 bounds. Head counts 1..16 (6: the reference's shape), ragged row counts,
strided v / dout, long runs of one token across many waves, tokens outside the table, and the reference-signature
entry points against the general ones."""
import ctypes

import numpy as np
import pytest
import torch

from nanochat_amd.native import hip_library, pointer, stream
from nanochat_amd.ve_gate import ve_backward, ve_forward
from oracle import ve_gate as ov
from oracle.numerics import bf16_round

pytestmark = pytest.mark.gpu
HEAD_DIM = 128
U = 2.0 ** -24


def bf16_ulp(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def make(rows, H, vocab, seed, token_range=None, wscale=0.05):
    gen = torch.Generator().manual_seed(seed)
    C = H * HEAD_DIM
    qkv = torch.randn(rows, 3 * C, generator=gen).bfloat16()           # v = its last C columns (strided rows)
    n = torch.randn(rows, C, generator=gen).bfloat16()
    table = torch.randn(vocab, C, generator=gen)
    w = torch.randn(H, C, generator=gen) * wscale
    lo, hi = token_range or (0, vocab)
    idx = torch.randint(lo, hi, (rows,), generator=gen, dtype=torch.int32)
    dqkv = torch.randn(rows, 3 * C, generator=gen).bfloat16()
    dtable0 = torch.randn(vocab, C, generator=gen) * 0.1
    return qkv, n, table, w, idx, dqkv, dtable0


def np32(t):
    return t.float().cpu().numpy()


def run_forward(dev, qkv, n, table, w, idx, heads, ref_symbol=False):
    lib = hip_library()
    rows, C = n.shape
    qkv_d, n_d, table_d, w_d, idx_d = (t.to(dev) for t in (qkv, n, table, w, idx))
    v_d = qkv_d[:, 2 * C:]
    out = torch.empty(rows, C, dtype=torch.bfloat16, device=dev)
    gate = torch.empty(rows, heads, dtype=torch.float32, device=dev)
    if ref_symbol:
        lib.ve_forward(pointer(n_d), pointer(v_d), qkv_d.stride(0), pointer(idx_d), pointer(table_d), pointer(w_d),
                       pointer(out), pointer(gate), rows, stream())
        st = lib.nc_last_error()
    else:
        st = lib.nc_ve_forward(pointer(n_d), pointer(v_d), qkv_d.stride(0), pointer(idx_d), pointer(table_d),
                               table.shape[0], pointer(w_d), pointer(out), pointer(gate), rows, heads, stream())
    assert st == 0, st
    torch.cuda.synchronize()
    return np32(out), gate.cpu().numpy()


def run_backward(dev, dqkv, idx, table, w, gate, dtable0, heads, ref_symbol=False):
    lib = hip_library()
    rows, C = dqkv.shape[0], heads * HEAD_DIM
    ids, order = torch.sort(idx.to(torch.int64), stable=True)
    dqkv_d, table_d, w_d = dqkv.to(dev), table.to(dev), w.to(dev)
    dout_d = dqkv_d[:, 2 * C:]
    ids_d, order_d = ids.to(torch.int32).to(dev), order.to(dev)
    gate_d = torch.tensor(gate, device=dev)
    dn = torch.empty(rows, C, dtype=torch.bfloat16, device=dev)
    dz = torch.empty(rows, heads, dtype=torch.bfloat16, device=dev)
    dtable = dtable0.to(dev).clone()
    if ref_symbol:
        lib.ve_backward(pointer(dout_d), dqkv_d.stride(0), pointer(ids_d), pointer(order_d), pointer(table_d),
                        pointer(w_d), pointer(gate_d), pointer(dn), pointer(dtable), pointer(dz), rows, stream())
        st = lib.nc_last_error()
    else:
        st = lib.nc_ve_backward(pointer(dout_d), dqkv_d.stride(0), pointer(ids_d), pointer(order_d),
                                pointer(table_d), table.shape[0], pointer(w_d), pointer(gate_d), pointer(dn),
                                pointer(dtable), pointer(dz), rows, heads, stream())
    assert st == 0, st
    torch.cuda.synchronize()
    return np32(dn), np32(dz), dtable.cpu().numpy().astype(np.float64), ids.numpy(), order.numpy()


def check_forward(n, table, w, idx, v, out, gate):
    """gate within its fp32 bound of the exact gate; out bit-exact given the device's gate."""
    H = w.shape[0]
    nch = (H + 3) // 4
    g64 = ov.gate(n, w)
    z_abs = np.abs(n.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    bound = 0.5 * z_abs * U * (8 * nch + 8) + 4 * U * g64
    assert np.all(np.abs(gate - g64) <= bound), np.max(np.abs(gate - g64) - bound)
    assert np.array_equal(out, ov.mix(v, gate, idx, table, table.shape[0]))


def check_backward(dout, table, w, idx, gate, n, dtable0, dn, dz, dtable, ids, order, tol_runs):
    H = w.shape[0]
    vocab = table.shape[0]
    dz64, dn64, dtab_add = ov.ve_backward(dout, ids, order, table, w, gate, vocab)
    e = ov.table_rows(table, idx, vocab).astype(np.float64)
    de_abs = (np.abs(dout.astype(np.float64)) * np.abs(e)).reshape(len(idx), H, HEAD_DIM).sum(axis=2)
    s = gate.astype(np.float64) * 0.5
    ddz = 2 * (1 - s) * s * de_abs * U * 16 + 8 * U * np.abs(dz64)
    assert np.all(np.abs(dz - dz64) <= bf16_ulp(dz64) * 0.5 + ddz + 1e-30)
    w64 = np.abs(w.astype(np.float64))
    ddn = ddz @ w64 + (H + 1) * U * (np.abs(dz64) @ w64)
    assert np.all(np.abs(dn - dn64) <= bf16_ulp(dn64) * 0.5 + ddn + 1e-30)
    gd = np.abs(bf16_round((np.repeat(gate, HEAD_DIM, axis=1) * dout).astype(np.float32))).astype(np.float64)
    mag = np.zeros_like(dtable)
    ok = (idx >= 0) & (idx < vocab)
    np.add.at(mag, idx[ok], gd[ok])
    ref = dtable0.astype(np.float64) + dtab_add
    assert np.all(np.abs(dtable - ref) <= (mag + np.abs(dtable0)) * U * tol_runs + 1e-30)


@pytest.mark.parametrize("H,rows,vocab", [(6, 1000, 300), (13, 777, 50), (1, 65, 10), (3, 300, 40), (16, 513, 2000),
                                          (10, 1, 5)])
def test_forward_backward_match_oracle(device, H, rows, vocab):
    qkv, n, table, w, idx, dqkv, dtable0 = make(rows, H, vocab, seed=H * 100 + rows)
    C = H * HEAD_DIM
    out, gate = run_forward(device, qkv, n, table, w, idx, H)
    n_, table_, w_, idx_ = np32(n), table.numpy(), w.numpy(), idx.numpy().astype(np.int64)
    check_forward(n_, table_, w_, idx_, np32(qkv[:, 2 * C:]), out, gate)
    dn, dz, dtable, ids, order = run_backward(device, dqkv, idx, table, w, gate, dtable0, H)
    check_backward(np32(dqkv[:, 2 * C:]), table_, w_, idx_, gate, n_, dtable0.numpy(), dn, dz, dtable, ids, order,
                   tol_runs=rows + 2)


def test_one_token_across_many_waves(device):
    """Every row the same token (and a second token for a few rows): runs that span many waves' ranges meet at wave
    boundaries and are summed by atomics."""
    H, rows = 6, 20000
    qkv, n, table, w, idx, dqkv, dtable0 = make(rows, H, 3, seed=7)
    idx[:] = 1
    idx[::997] = 2
    C = H * HEAD_DIM
    out, gate = run_forward(device, qkv, n, table, w, idx, H)
    check_forward(np32(n), table.numpy(), w.numpy(), idx.numpy().astype(np.int64), np32(qkv[:, 2 * C:]), out, gate)
    dn, dz, dtable, ids, order = run_backward(device, dqkv, idx, table, w, gate, dtable0, H)
    check_backward(np32(dqkv[:, 2 * C:]), table.numpy(), w.numpy(), idx.numpy().astype(np.int64), gate, np32(n),
                   dtable0.numpy(), dn, dz, dtable, ids, order, tol_runs=rows + 2)


def test_tokens_outside_table(device):
    H, rows, vocab = 5, 400, 30
    qkv, n, table, w, idx, dqkv, dtable0 = make(rows, H, vocab, seed=11, token_range=(-3, vocab + 3))
    C = H * HEAD_DIM
    out, gate = run_forward(device, qkv, n, table, w, idx, H)
    v = np32(qkv[:, 2 * C:])
    bad = (idx.numpy() < 0) | (idx.numpy() >= vocab)
    assert bad.sum() > 10
    assert np.array_equal(out[bad], v[bad])
    check_forward(np32(n), table.numpy(), w.numpy(), idx.numpy().astype(np.int64), v, out, gate)
    dn, dz, dtable, ids, order = run_backward(device, dqkv, idx, table, w, gate, dtable0, H)
    assert np.all(dz[bad] == 0) and np.all(dn[bad] == 0)
    check_backward(np32(dqkv[:, 2 * C:]), table.numpy(), w.numpy(), idx.numpy().astype(np.int64), gate, np32(n),
                   dtable0.numpy(), dn, dz, dtable, ids, order, tol_runs=rows + 2)


def test_reference_symbols_match_general_entry_points(device):
    H, rows, vocab = 6, 700, 100
    qkv, n, table, w, idx, dqkv, dtable0 = make(rows, H, vocab, seed=3)
    out_a, gate_a = run_forward(device, qkv, n, table, w, idx, H)
    out_b, gate_b = run_forward(device, qkv, n, table, w, idx, H, ref_symbol=True)
    assert np.array_equal(out_a, out_b) and np.array_equal(gate_a, gate_b)
    dn_a, dz_a, dt_a, *_ = run_backward(device, dqkv, idx, table, w, gate_a, dtable0, H)
    dn_b, dz_b, dt_b, *_ = run_backward(device, dqkv, idx, table, w, gate_a, dtable0, H, ref_symbol=True)
    assert np.array_equal(dn_a, dn_b) and np.array_equal(dz_a, dz_b)
    assert np.allclose(dt_a, dt_b, rtol=1e-5, atol=1e-5)


def test_zero_rows_launch_nothing(device):
    lib = hip_library()
    assert lib.nc_ve_forward(None, None, 768, None, None, 1, None, None, None, 0, 6, stream()) == 0
    assert lib.nc_ve_backward(None, 768, None, None, None, 1, None, None, None, None, None, 0, 6, stream()) == 0


def test_torch_surface_matches_oracle(device):
    """The reference's Python surface (model/ops/ve_gate.py): (B, T) shapes, v a view of the fused projection,
    table.grad accumulated across two backward calls, dw = dz^T n by torch.mm."""
    B, T, H, vocab = 2, 300, 6, 500
    C = H * HEAD_DIM
    gen = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, T, 3 * C, generator=gen).bfloat16().to(device)
    n = torch.randn(B, T, C, generator=gen).bfloat16().to(device)
    table = torch.randn(vocab, C, generator=gen).to(device).requires_grad_()
    w = (torch.randn(H, C, generator=gen) * 0.05).to(device)
    input_ids = torch.randint(0, vocab, (B, T), generator=gen, dtype=torch.int32).to(device)
    v = qkv[..., 2 * C:].unflatten(-1, (H, HEAD_DIM))
    out, gate = ve_forward(n, v, input_ids, table.detach(), w)
    torch.cuda.synchronize()
    n_, idx_ = np32(n.view(-1, C)), input_ids.view(-1).cpu().numpy().astype(np.int64)
    check_forward(n_, table.detach().cpu().numpy(), w.cpu().numpy(), idx_, np32(v.reshape(-1, C)),
                  np32(out.view(-1, C)), gate.cpu().numpy())
    dqkv = torch.randn(B, T, 3 * C, generator=gen).bfloat16().to(device)
    dv = dqkv[..., 2 * C:].unflatten(-1, (H, HEAD_DIM))
    ids, order = torch.sort(input_ids.flatten())
    dn, dw = ve_backward(dv, n, ids, order, table, w, gate)
    dn2, dw2 = ve_backward(dv, n, ids, order, table, w, gate)
    torch.cuda.synchronize()
    assert torch.equal(dn, dn2) and torch.equal(dw, dw2)
    g = gate.cpu().numpy()
    dz64, dn64, dtab_add = ov.ve_backward(np32(dv.reshape(-1, C)), ids.cpu().numpy(), order.cpu().numpy(),
                                          table.detach().cpu().numpy(), w.cpu().numpy(), g)
    got = table.grad.cpu().numpy().astype(np.float64)
    assert np.allclose(got, 2 * dtab_add, rtol=1e-4, atol=1e-5)
    assert np.all(np.abs(np32(dn.view(-1, C)) - dn64) <= bf16_ulp(dn64) + 1e-3 * np.abs(dn64).max())
    # dw from the device's bf16 dz: torch.mm's fp32 accumulation over B*T rows
    dz_b = bf16_round(dz64.astype(np.float32))
    dw64 = ov.weight_grad(dz_b, n_)
    bound = (np.abs(dz_b).astype(np.float64).T @ np.abs(n_).astype(np.float64))
    assert np.all(np.abs(dw.cpu().numpy() - dw64) <= bound * 2.0 ** -7 + 1e-6)
