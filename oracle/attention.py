"""Decode and chunked-prefill attention over the fp8 cache, float64 — test infrastructure only.

Decode restates model/kernels/decode.cu:567-675 (k_attn): the query of sequence b at position
p = seq_len - 1 attends keys [max(p - window, 0), p] (decode.cu:575; FA4's window_size_left,
model/ops/flash_attn.py:309-311), scores (q . k) * sm_scale, softmax, weighted sum of values. In the
build the current token's K/V are read back from the fp8 cache (append, then attend), where the
reference merges its bf16 k, v last (decode.cu:671-674). GQA: query head h reads KV head h // (Hq/Hkv).

Chunked prefill restates decode.cu:859-863 (every chunk row's k, v appended before any row attends):
row t of sequence b sits at position start[b] + t and attends keys [max(p - window, 0), p].

Both compute in float64 on the dequantized cache (fp32(code) * scale) from bf16 queries.

Pinned by tests/test_oracle_attention.py: a single key returns its value; equal scores give the mean
of the values; a window equals slicing the cache; GQA equals MHA with repeated KV heads; prefill rows
equal decode at each position; prefill equals torch's scaled_dot_product_attention (float64, explicit
mask) on the same dequantized cache.
"""
import numpy as np

PAGE = 16


def _softmax_rows(s):
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def decode_attention(q, cache, block_table, seq_lens, window=-1, sm_scale=None):
    """q (B, Hq, 128) bf16-valued -> (B, Hq, 128) float64. Sequences with seq_len <= 0 give zeros."""
    q = np.asarray(q, np.float64)
    B, Hq, D = q.shape
    hkv = cache.hkv
    G = Hq // hkv
    if sm_scale is None:
        sm_scale = D ** -0.5
    out = np.zeros((B, Hq, D), np.float64)
    for b in range(B):
        n = int(seq_lens[b])
        if n <= 0:
            continue
        p = n - 1
        begin = max(p - window, 0) if window >= 0 else 0
        K, V = cache.gather_values(block_table, b, n)
        K = K[begin:].astype(np.float64)
        V = V[begin:].astype(np.float64)
        for h in range(hkv):
            qs = q[b, h * G:(h + 1) * G]                       # (G, D)
            w = _softmax_rows(qs @ K[:, h].T * sm_scale)       # (G, n')
            out[b, h * G:(h + 1) * G] = w @ V[:, h]
    return out


def prefill_attention(q, cache, block_table, start, window=-1, sm_scale=None):
    """q (B, T, Hq, 128) bf16-valued; row t of sequence b at position start[b] + t -> (B, T, Hq, 128) float64."""
    q = np.asarray(q, np.float64)
    B, T, Hq, D = q.shape
    hkv = cache.hkv
    G = Hq // hkv
    if sm_scale is None:
        sm_scale = D ** -0.5
    out = np.zeros((B, T, Hq, D), np.float64)
    for b in range(B):
        n = int(start[b]) + T
        K, V = cache.gather_values(block_table, b, n)
        K = K.astype(np.float64)
        V = V.astype(np.float64)
        pos = int(start[b]) + np.arange(T)
        keys = np.arange(n)
        allowed = keys[None, :] <= pos[:, None]
        if window >= 0:
            allowed &= keys[None, :] >= pos[:, None] - window
        bias = np.where(allowed, 0.0, -np.inf)                # (T, n)
        for h in range(hkv):
            qs = q[b, :, h * G:(h + 1) * G]                    # (T, G, D)
            s = np.einsum("tgd,nd->tgn", qs, K[:, h]) * sm_scale + bias[:, None, :]
            out[b, :, h * G:(h + 1) * G] = np.einsum("tgn,nd->tgd", _softmax_rows(s), V[:, h])
    return out
