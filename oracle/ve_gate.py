"""Value-embedding gate and mix of training — test infrastructure only (the checker of
nanochat_amd/csrc/ve_gate.hip; nothing in the product imports it).

Restates model/kernels/ve_gate.cu (ve_forward_kernel :36-88, ve_backward_kernel :101-194) and the host side
model/ops/ve_gate.py:13-33, for rows of the normed stream n (C = 128 H):

    gate[r][h]   = 2 sigmoid(sum_c n[r][c] w[h][c])                                     (ve_gate.cu:57-71)
    out[r][c]    = bf16(v[r][c] + gate[r][c / 128] * bf16(table[idx[r]][c]))            (ve_gate.cu:75-86)
    dg[h]        = sum over head h's columns of dout[r][c] bf16(table[t][c])            (ve_gate.cu:155-170)
    dz[r][h]     = 2 dg[h] (1 - s) s,  s = gate[r][h] / 2  (stored as bf16)             (ve_gate.cu:172-178)
    dn[r][c]     = sum_h dz[h] w[h][c]  (stored as bf16)                                (ve_gate.cu:179-190)
    dtable[t][c] += sum over rows of token t of bf16(gate[r][c / 128] dout[r][c])       (ve_gate.cu:90-99, 166)
    dw           = dz^T n  (the host's GEMM, ve_gate.py:33)

The sums the kernel accumulates in fp32 (gate logits, dg, dn, the table's runs) are computed here in float64;
the tests bound the device's fp32 accumulation error against them. The roundings the contract fixes (bf16 of the
table, the product and sum of the mix, the per-row bf16 of gate * dout) are reproduced exactly in fp32.

Pinned by tests/test_oracle_ve_gate.py: the forward and all four gradients equal torch autograd of the float64
expression v + 2 sigmoid(n w^T)[head] e (table values already bf16) within the stated roundings; a zero w gives
gate 1 (out = v + e rounded); a token outside the table mixes in nothing.

The cache append's gate (cache_gate) is the same gate in one fixed fp32 order, so its bits are fixed: fma32 is pinned
against exact rational arithmetic (random operands and constructed midpoint ties), and cache_gate against the
float64 gate within the fp32 chain's error bound, with a zero w giving exactly 1.
"""
import numpy as np

from oracle.numerics import bf16_round

HEAD_DIM = 128


def gate(n, w):
    """n (rows, C) bf16 values, w (H, C) fp32 -> the exact gate 2 sigmoid(n w^T) (rows, H) float64."""
    z = np.asarray(n, np.float64) @ np.asarray(w, np.float64).T
    return 2.0 / (1.0 + np.exp(-z))


def fma32(a, b, c):
    """a * b + c rounded once to fp32, elementwise, for fp32 arrays whose product a * b is exact in float64 (a holding
    bf16 values: 8 + 24 significant bits). The float64 sum s and its exact error e (Knuth's TwoSum) give the exact
    value s + e; rounding s to fp32 already rounds s + e correctly unless s is exactly the midpoint of two floats and
    e is not zero, where the exact value lies on e's side of it."""
    p = np.asarray(a, np.float32).astype(np.float64) * np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    s = p + c64
    pv = s - c64                       # the parts of s that came from p and from c
    e = (p - pv) + (c64 - (s - pv))
    f = s.astype(np.float32)
    f64 = f.astype(np.float64)
    toward = np.where(s > f64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
    other = np.nextafter(f, toward)
    tie = (f64 != s) & (s == (f64 + other.astype(np.float64)) * 0.5) & (e != 0)
    return np.where(tie, np.where(e > 0, np.maximum(f, other), np.minimum(f, other)), f).astype(np.float32)


def exp_rn(x):
    """e^x of fp32 values rounded once to fp32 (the float64 exponential rounded to float)."""
    return np.exp(np.asarray(x, np.float32).astype(np.float64)).astype(np.float32)


def cache_gate(n, w):
    """The cache append's gate in its fixed fp32 order (the append and the fused decode step alike; the reference's
    attn_prologue, model/kernels/decode.cu:481-494, fixes another fp32 order): per (row, head), 64 lanes each run an
    FMA chain d_l = fma(n[i], w[i], d_l) over i = l, l + 64, ... < C from 0; then an xor butterfly over offsets 32, 16,
    8, 4, 2, 1 (d_l + d_(l ^ o), fp32); then g = 2 (1 / (1 + exp_rn(-d))), each operation rounded to fp32.
    n (rows, C) bf16 values, w (H, C) fp32 -> (rows, H) fp32."""
    n = np.asarray(n, np.float32)
    w = np.asarray(w, np.float32)
    rows, C = n.shape
    H = w.shape[0]
    d = np.zeros((rows, H, 64), np.float32)
    for i0 in range(0, C, 64):
        k = min(64, C - i0)
        a = np.broadcast_to(n[:, None, i0:i0 + k], (rows, H, k))
        b = np.broadcast_to(w[None, :, i0:i0 + k], (rows, H, k))
        d[:, :, :k] = fma32(a, b, d[:, :, :k])
    lanes = np.arange(64)
    for o in (32, 16, 8, 4, 2, 1):
        d = (d + d[:, :, lanes ^ o]).astype(np.float32)
    one = np.float32(1.0)
    return (np.float32(2.0) * (one / (one + exp_rn(-d[:, :, 0])))).astype(np.float32)


def table_rows(table, idx, vocab=None):
    """bf16(table[idx]) as fp32 (rows, C); tokens outside [0, vocab) give zero rows."""
    table = np.asarray(table, np.float32)
    vocab = table.shape[0] if vocab is None else vocab
    idx = np.asarray(idx, np.int64)
    ok = (idx >= 0) & (idx < vocab)
    e = np.zeros((len(idx), table.shape[1]), np.float32)
    e[ok] = bf16_round(table[idx[ok]])
    return e


def mix(v, g, idx, table, vocab=None):
    """out = bf16(v + g[head] * bf16(table[idx])) with the product and the sum each rounded to fp32 (ve_gate.cu:84),
    for a given fp32 gate g (rows, H)."""
    v = np.asarray(v, np.float32)
    rows, C = v.shape
    gh = np.repeat(np.asarray(g, np.float32), HEAD_DIM, axis=1)          # (rows, C)
    prod = (gh * table_rows(table, idx, vocab)).astype(np.float32)
    return bf16_round((v + prod).astype(np.float32))


def ve_forward(n, v, idx, table, w, vocab=None):
    """-> (out (rows, C) fp32 holding bf16, gate (rows, H) float64 exact)."""
    g = gate(n, w)
    return mix(v, g.astype(np.float32), idx, table, vocab), g


def ve_backward(dout, ids, order, table, w, g, vocab=None):
    """dout (rows, C) bf16 values in row order; ids, order: the sorted tokens and their rows; g (rows, H) the forward's
    fp32 gate. -> dz (rows, H) float64 before its bf16 rounding, dn (rows, C) float64 from that dz, dtable_add
    (vocab, C) float64: the sum of the exactly rounded per-row terms bf16(g dout)."""
    dout = np.asarray(dout, np.float32)
    g = np.asarray(g, np.float32)
    w = np.asarray(w, np.float64)
    table = np.asarray(table, np.float32)
    rows, C = dout.shape
    H = C // HEAD_DIM
    vocab = table.shape[0] if vocab is None else vocab
    ids = np.asarray(ids, np.int64)
    order = np.asarray(order, np.int64)
    tok = np.empty(rows, np.int64)
    tok[order] = ids
    e = table_rows(table, tok, vocab).astype(np.float64)
    dg = (dout.astype(np.float64) * e).reshape(rows, H, HEAD_DIM).sum(axis=2)
    s = g.astype(np.float64) * 0.5
    dz = 2.0 * dg * (1.0 - s) * s
    dn = dz @ w
    terms = bf16_round((np.repeat(g, HEAD_DIM, axis=1) * dout).astype(np.float32)).astype(np.float64)
    dtable = np.zeros((table.shape[0], C), np.float64)
    ok = (tok >= 0) & (tok < vocab)
    np.add.at(dtable, tok[ok], terms[ok])
    return dz, dn, dtable


def weight_grad(dz_bf16, n):
    """dw = dz^T n in float64 from the stored bf16 dz (ve_gate.py:33)."""
    return np.asarray(dz_bf16, np.float64).T @ np.asarray(n, np.float64)
