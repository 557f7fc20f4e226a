"""Varlen causal (optionally windowed) training attention, float64 — test infrastructure only (the checker of
nanochat_amd/csrc/flash_attn.hip; nothing in the product imports it).

Restates the semantics the reference gets from FlashAttention-4 (flash-attn-4 4.0.0b36, not vendored in the
reference) at its call sites model/ops/flash_attn.py:340-345 (forward: _flash_attn_fwd(q, k, v, cu_seqlens, cu_seqlens,
T, T, causal=True, window_size_left=window, return_lse=True)) and :381-383 (backward), with the window rule of
fa4_window_left (flash_attn.py:309-311): within segment s (tokens cu[s] .. cu[s+1]-1), row i attends keys j with
j <= i and i - j <= window (window < 0: all earlier keys).

    out_i = sum_j P_ij v_j,  P_i = softmax_j(scale q_i . k_j),  lse_i = ln sum_j exp(scale q_i . k_j)
    backward (dout): D_i = dout_i . out_i, dv_j = sum_i P_ij dout_i, dP_ij = dout_i . v_j,
                     dS_ij = P_ij (dP_ij - D_i), dq_i = scale sum_j dS_ij k_j, dk_j = scale sum_i dS_ij q_i

FA4's own bits cannot be reproduced here (CUDA only): parity unpinned against the library itself, pinned against the
mathematics. Pinned by tests/test_oracle_flash.py: the forward equals torch's scaled_dot_product_attention (float64,
explicit mask) and torch.logsumexp; the backward equals torch autograd of that forward; window >= length - 1 equals
plain causal; window 0 returns v.
"""
import numpy as np

HEAD_DIM = 128


def visible(n, window=-1):
    """(n, n) bool: row i sees key j."""
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    ok = j <= i
    if window >= 0:
        ok &= (i - j) <= window
    return ok


def varlen_forward(q, k, v, cu, window=-1, scale=None):
    """q, k, v (total, H, D) -> out (total, H, D) float64, lse (H, total) float64."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    total, H, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    out = np.zeros((total, H, D))
    lse = np.zeros((H, total))
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        if b <= a:
            continue
        ok = visible(b - a, window)
        for h in range(H):
            sc = np.where(ok, q[a:b, h] @ k[a:b, h].T * scale, -np.inf)
            m = sc.max(axis=1, keepdims=True)
            e = np.exp(sc - m)
            l = e.sum(axis=1, keepdims=True)
            out[a:b, h] = (e / l) @ v[a:b, h]
            lse[h, a:b] = (m + np.log(l))[:, 0]
    return out, lse


def varlen_backward(q, k, v, dout, cu, window=-1, scale=None):
    """-> dq, dk, dv (total, H, D) float64."""
    q, k, v, dout = (np.asarray(x, np.float64) for x in (q, k, v, dout))
    total, H, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        if b <= a:
            continue
        ok = visible(b - a, window)
        for h in range(H):
            sc = np.where(ok, q[a:b, h] @ k[a:b, h].T * scale, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            o = p @ v[a:b, h]
            do = dout[a:b, h]
            dv[a:b, h] = p.T @ do
            dp = do @ v[a:b, h].T
            ds = p * (dp - (do * o).sum(axis=1, keepdims=True))
            dq[a:b, h] = scale * ds @ k[a:b, h]
            dk[a:b, h] = scale * ds.T @ q[a:b, h]
    return dq, dk, dv
