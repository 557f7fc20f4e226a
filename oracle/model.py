"""The decoder's body and head over an fp8 cache, numpy — test infrastructure only.

Restates the step of model/kernels/decode.cu (enqueue_body / enqueue_head, decode.cu:838-891) as the build computes
it, on rows (token, position, slot):

    EMBED       x0 = wte[token] * r                                   r = 1 / sqrt(mean v^2 + FLT_EPSILON) (fp32)
    per layer   v = fma(l1, h, x0 * l2), h = x (bf16) or x0 at layer 0;  xm = bf16(v);  hn = bf16(v * r)
                qkv = bf16(hn W_qkv^T)
                q, k = qk_norm_rope(q, k) at the row's position (oracle.rope); v = bf16(v + 2 sigmoid(w_gate . hn) ve)
                K, V cached as fp8 (oracle.quant) at (slot, position); every row's K, V before any row attends
                att = bf16(softmax over keys [max(p - window, 0), p] of the slot's dequantized cache)
                x = s + xm (s = att W_o^T);  xo = bf16(x);  rstd = 1 / sqrt(sum x^2 / C + FLT_EPSILON)
                u = bf16(relu(p) p), p = (xo W_fc^T) rstd;  x = bf16(u W_proj^T + xo)
    HEAD        hn = bf16(x * r);  logits = hn lm_head^T                                         (float64)

GEMM sums are float64 (the device: fp32 accumulation), each rounded where the device rounds; a prefill call's last
layer only caches K and V (decode.cu:859-863).

Pinned by tests/test_oracle_model.py: with zero o/proj weights the stream is the scaled embedding and the logits
equal lm_head applied to torch's rms_norm (float64); the MLP equals torch's relu(rms_norm(x) W_fc^T)^2 W_proj^T
(the rstd identity W (x r) = (W x) r); attention with one cached key returns its value; `attend` equals torch's
scaled_dot_product_attention (float64) under an explicit band mask for windows 0, 1, inside and past the context, and
through a one-layer model a token just outside a row's window leaves the row's output bit-identical while the one at
the window's edge changes it; a prompt prefilled in one call equals the same rows fed one at a time; the
value-embedding gate at zero weights adds exactly ve.
"""
from dataclasses import dataclass, field

import numpy as np

from .numerics import bf16_round
from .quant import dequantize_rows, quantize_rows
from .rope import qk_norm_rope

HEAD_DIM = 128
FLT_EPSILON = np.float32(np.finfo(np.float32).eps)


@dataclass
class LayerWeights:
    qkv: np.ndarray            # (3C, C) float32 holding bf16
    o: np.ndarray              # (C, C)
    fc: np.ndarray             # (F, C)
    proj: np.ndarray           # (C, F)
    q_gain: np.ndarray         # (128,) float32
    k_gain: np.ndarray
    resid: float
    x0: float
    window: int
    ve: np.ndarray | None = None        # (vocab, C) float32 holding bf16
    ve_gate: np.ndarray | None = None   # (H, C) float32


@dataclass
class ModelWeights:
    wte: np.ndarray            # (vocab, C) float32
    cos: np.ndarray            # (T, 64) float32
    sin: np.ndarray
    lm_head: np.ndarray        # (vocab, C) float32 holding bf16
    layers: list[LayerWeights] = field(default_factory=list)
    softcap: float = 15.0

    @property
    def C(self) -> int:
        return self.wte.shape[1]

    @property
    def H(self) -> int:
        return self.C // HEAD_DIM


def _f32(x):
    return np.asarray(x, np.float32)


def rms_scale(v, divide=True):
    """r = 1 / sqrt(sum v^2 / C + FLT_EPSILON) per row, fp32 (divide=False: sum v^2 * (1 / C), as the rstd)."""
    ss = np.sum(v.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    C = v.shape[-1]
    mean = ss / np.float32(C) if divide else ss * np.float32(1.0 / C)
    return (np.float32(1.0) / np.sqrt((mean + FLT_EPSILON).astype(np.float32))).astype(np.float32)


def attend(q, K, V, p, window):
    """One row's attention (decode.cu:567-675): q (H, 128) at position p over the cached K, V (T, H, 128) at positions
    [max(p - window, 0), p] (window < 0: from 0), scores scaled by 1/sqrt(128), softmax in float64 -> (H, 128)."""
    begin = max(p - window, 0) if window >= 0 else 0
    kk = K[begin:p + 1].astype(np.float64)                    # (m, H, 128)
    vv = V[begin:p + 1].astype(np.float64)
    s = np.einsum("hd,mhd->hm", q.astype(np.float64), kk) * HEAD_DIM ** -0.5
    s = np.exp(s - s.max(axis=-1, keepdims=True))
    return np.einsum("hm,mhd->hd", s / s.sum(axis=-1, keepdims=True), vv)


def matmul_t(x, w):
    """x (n, K) @ w (R, K)^T in float64."""
    return x.astype(np.float64) @ w.astype(np.float64).T


class DecoderOracle:
    """Per-slot fp8 caches (dequantized values) and the step's arithmetic."""

    def __init__(self, weights: ModelWeights, max_len: int):
        self.w = weights
        self.max_len = max_len
        L, H = len(weights.layers), weights.H
        self.k = {}   # slot -> (L, max_len, H, 128) float32 dequantized
        self.v = {}
        self.codes = {}   # slot -> dict of raw codes/scales per layer for byte comparisons
        self.L, self.H = L, H
        self._f64 = {}    # id(weight) -> its float64 copy, converted once

    def _mm(self, x, w):
        """x (n, K) @ w (R, K)^T in float64, w converted once per oracle."""
        key = id(w)
        if key not in self._f64:
            self._f64[key] = (w, w.astype(np.float64))
        return x.astype(np.float64) @ self._f64[key][1].T

    def _slot(self, b):
        if b not in self.k:
            shape = (self.L, self.max_len, self.H, HEAD_DIM)
            self.k[b] = np.zeros(shape, np.float32)
            self.v[b] = np.zeros(shape, np.float32)
            self.codes[b] = {
                "k": np.zeros(shape, np.uint8), "v": np.zeros(shape, np.uint8),
                "scale": np.zeros((self.L, self.max_len, self.H, 2), np.float32),
            }
        return self.k[b], self.v[b]

    def body(self, tokens, positions, slots, cache_only_last=False):
        """Rows through the layers; returns x (n, C) float32 holding bf16 (None when cache_only_last)."""
        w = self.w
        tokens = np.asarray(tokens, np.int64)
        positions = np.asarray(positions, np.int64)
        slots = np.asarray(slots, np.int64)
        n, C, H = len(tokens), w.C, w.H
        emb = _f32(w.wte[tokens])
        x0 = (emb * rms_scale(emb)).astype(np.float32)
        x = None
        for li, ly in enumerate(w.layers):
            h = x0 if x is None else x
            v = (np.float64(ly.resid) * h.astype(np.float64) + (x0 * np.float32(ly.x0)).astype(np.float64))
            v = v.astype(np.float32)
            xm = bf16_round(v)
            hn = bf16_round((v * rms_scale(v)).astype(np.float32))
            qkv = bf16_round(self._mm(hn, ly.qkv).astype(np.float32)).reshape(n, 3, H, HEAD_DIM)
            cos, sin = w.cos[positions][:, None, :], w.sin[positions][:, None, :]
            q = qk_norm_rope(qkv[:, 0], ly.q_gain, cos, sin)
            k = qk_norm_rope(qkv[:, 1], ly.k_gain, cos, sin)
            val = qkv[:, 2]
            if ly.ve is not None:
                d = self._mm(hn, ly.ve_gate)                              # (n, H)
                g = (2.0 / (1.0 + np.exp(-d))).astype(np.float32)[:, :, None]
                e = _f32(ly.ve[tokens]).reshape(n, H, HEAD_DIM)
                val = bf16_round((val + (g * e).astype(np.float32)).astype(np.float32))
            kc, ks = quantize_rows(k)
            vc, vs = quantize_rows(val)
            for r in range(n):
                K, V = self._slot(int(slots[r]))
                p = int(positions[r])
                K[li, p] = dequantize_rows(kc[r], ks[r])
                V[li, p] = dequantize_rows(vc[r], vs[r])
                c = self.codes[int(slots[r])]
                c["k"][li, p], c["v"][li, p] = kc[r], vc[r]
                c["scale"][li, p, :, 0], c["scale"][li, p, :, 1] = ks[r], vs[r]
            if cache_only_last and li == len(w.layers) - 1:
                return None
            att = np.zeros((n, H, HEAD_DIM), np.float64)
            for r in range(n):
                K, V = self.k[int(slots[r])][li], self.v[int(slots[r])][li]
                att[r] = attend(q[r], K, V, int(positions[r]), ly.window)
            att = bf16_round(att.astype(np.float32)).reshape(n, C)
            xs = (self._mm(att, ly.o) + xm.astype(np.float64)).astype(np.float32)
            xo = bf16_round(xs)
            rstd = rms_scale(xs, divide=False)
            p_ = (self._mm(xo, ly.fc).astype(np.float32) * rstd).astype(np.float32)
            u = bf16_round((np.maximum(p_, 0) * p_).astype(np.float32))
            x = bf16_round((self._mm(u, ly.proj) + xo.astype(np.float64)).astype(np.float32))
        return x

    def head(self, x):
        """Final norm and lm_head: logits (n, vocab) float64."""
        hn = bf16_round((x * rms_scale(x)).astype(np.float32))
        return self._mm(hn, self.w.lm_head)


def weights_from_tensors(model):
    """ModelWeights from a model given as tensors (attributes wte, cos, sin, lm_head, layers with qkv, o, fc,
    proj, q_norm, k_norm, ve, ve_gate, and per-layer resid_lambdas, x0_lambdas, windows, softcap), on any device."""
    def f32(t):
        return None if t is None else t.detach().float().cpu().numpy()

    layers = [LayerWeights(qkv=f32(ly.qkv), o=f32(ly.o), fc=f32(ly.fc), proj=f32(ly.proj), q_gain=f32(ly.q_norm),
                           k_gain=f32(ly.k_norm), resid=float(r), x0=float(x), window=int(w), ve=f32(ly.ve),
                           ve_gate=f32(ly.ve_gate))
              for ly, r, x, w in zip(model.layers, model.resid_lambdas, model.x0_lambdas, model.windows)]
    return ModelWeights(wte=f32(model.wte), cos=f32(model.cos), sin=f32(model.sin), lm_head=f32(model.lm_head),
                        layers=layers, softcap=float(model.softcap))
