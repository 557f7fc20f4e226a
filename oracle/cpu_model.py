"""The CPU baseline of the whole decode step (config 5): the decoder's body and head in PyTorch float32 on the host's
threads — measurement and test infrastructure only (bench.py's cpu_baseline leg and tests/; nothing in the product
imports it).

It is the arithmetic of oracle/model.py (which restates model/kernels/decode.cu:838-891, enqueue_body / enqueue_head)
with float32 GEMMs (torch.mm over the host's BLAS threads) in place of float64 ones, and the attention, norms and
rotation of oracle/cpu_step.py:

    EMBED       x0 = wte[token] * r,  r = 1 / sqrt(mean v^2 + FLT_EPSILON)
    per layer   v = l1 h + l2 x0 (h = x, or x0 at layer 0);  xm = bf16(v);  hn = bf16(v r)
                qkv = bf16(hn W_qkv^T);  q, k = bf16 of the q/k norm and rotation;  v = bf16(v + 2 sigmoid(w_gate . hn) ve)
                k, v quantized per (token, head) to e4m3fn (scale max|x| / 448) and cached as their decoded values
                att = bf16(softmax over keys [max(p - window, 0), p] of the slot's cache)
                xs = att W_o^T + xm;  xo = bf16(xs);  rstd = 1 / sqrt(sum xs^2 / C + FLT_EPSILON)
                u = bf16(relu(p) p), p = (xo W_fc^T) rstd;  x = bf16(u W_proj^T + xo)
    HEAD        logits = bf16(x r) lm_head^T

The cache holds each position's decoded fp8 values (fp32(code) * scale, exact), decoded once when stored, so a step
reads four bytes per cached element instead of decoding every code again. Every row of a call is appended before any
row attends (decode.cu:859-863). Pinned by tests/test_oracle_cpu_model.py against oracle/model.py (float64) on a small
model: logits, greedy tokens and the cache codes.
"""
import torch

from .cpu_step import EPS, HEAD_DIM, norm_rope, quantize


def _bf16(x):
    return x.to(torch.bfloat16).float()


def _rms(v, divide=True):
    """1 / sqrt(sum v^2 / C + FLT_EPSILON) per row (divide=False: sum v^2 * (1 / C))."""
    ss = (v * v).sum(-1, keepdim=True)
    C = v.shape[-1]
    return 1.0 / torch.sqrt((ss / C if divide else ss * (1.0 / C)) + EPS)


class CpuDecoder:
    """Weights as float32 host tensors (their bf16 values), a cache of decoded values [layers][slots][H][max_len][128]
    for K and V (a slot's head is contiguous, so slots attend through views), and the step's arithmetic."""

    def __init__(self, model, slots: int, max_len: int, keep_codes: bool = True):
        def f32(t):
            return None if t is None else t.detach().float().cpu().contiguous()

        self.wte, self.lm_head = f32(model.wte), f32(model.lm_head)
        self.cos, self.sin = f32(model.cos), f32(model.sin)
        self.layers = [dict(qkv=f32(ly.qkv), o=f32(ly.o), fc=f32(ly.fc), proj=f32(ly.proj), q_gain=f32(ly.q_norm),
                            k_gain=f32(ly.k_norm), ve=f32(ly.ve), ve_gate=f32(ly.ve_gate), resid=float(r),
                            x0=float(x), window=int(w))
                       for ly, r, x, w in zip(model.layers, model.resid_lambdas, model.x0_lambdas, model.windows)]
        self.C = self.wte.shape[1]
        self.H = self.C // HEAD_DIM
        shape = (len(self.layers), slots, self.H, max_len, HEAD_DIM)
        self.k = torch.zeros(shape)
        self.v = torch.zeros(shape)
        # (k, v) codes [layers][slots][max_len][H][2][128], for the tests
        self.codes = (torch.zeros((len(self.layers), slots, max_len, self.H, 2, HEAD_DIM), dtype=torch.uint8)
                      if keep_codes else None)

    def store(self, li, slots, positions, k, v):
        """Quantize rows' k, v (n, H, 128) and cache their decoded values at (slot, position)."""
        kc, ks = quantize(k)
        vc, vs = quantize(v)
        if self.codes is not None:
            self.codes[li, slots, positions, :, 0] = kc
            self.codes[li, slots, positions, :, 1] = vc
        kd = kc.view(torch.float8_e4m3fn).float() * ks[..., None]
        vd = vc.view(torch.float8_e4m3fn).float() * vs[..., None]
        for r in range(len(slots)):
            self.k[li, slots[r], :, positions[r]] = kd[r]
            self.v[li, slots[r], :, positions[r]] = vd[r]

    def attend(self, li, q, slots, positions, window):
        """Each row (q (n, H, 128) at its slot and position) over its slot's keys [max(p - window, 0), p]. Rows of a
        run of consecutive slots, one row each, attend as one batch through views of the cache; other rows by
        slot."""
        n = q.shape[0]
        s0 = int(slots[0])
        if torch.equal(slots, torch.arange(s0, s0 + n)):
            groups = [(slice(s0, s0 + n), torch.arange(n))]
        else:
            groups = [(int(b), (slots == b).nonzero()[:, 0]) for b in torch.unique(slots)]
        out = torch.empty_like(q)
        for sel, idx in groups:
            pos = positions[idx]
            L = int(pos.max()) + 1
            K, V = self.k[li, sel, :, :L], self.v[li, sel, :, :L]              # (n, H, L, 128) or (H, L, 128)
            if isinstance(sel, slice):
                s = torch.matmul(q[idx][:, :, None, :], K.transpose(-1, -2))[:, :, 0] * HEAD_DIM ** -0.5  # (n, H, L)
            else:
                s = torch.matmul(q[idx].transpose(0, 1), K.transpose(-1, -2)).transpose(0, 1) * HEAD_DIM ** -0.5
            p = pos[:, None, None]
            j = torch.arange(L)
            ok = j <= p
            if window >= 0:
                ok = ok & (j >= p - window)
            w = torch.softmax(s.masked_fill(~ok, float("-inf")), dim=-1)       # (rows, H, L)
            if isinstance(sel, slice):
                out[idx] = torch.matmul(w[:, :, None, :], V)[:, :, 0]
            else:
                out[idx] = torch.matmul(w.transpose(0, 1), V).transpose(0, 1)
        return out

    def body(self, tokens, positions, slots, cache_only_last=False):
        """Rows (token, position, slot) through the layers -> x (n, C) float32 holding bf16 (None when
        cache_only_last: the last layer only caches its K and V)."""
        tokens = torch.as_tensor(tokens, dtype=torch.long)
        positions = torch.as_tensor(positions, dtype=torch.long)
        slots = torch.as_tensor(slots, dtype=torch.long)
        n, C, H = len(tokens), self.C, self.H
        emb = self.wte[tokens]
        x0 = emb * _rms(emb)
        x = None
        cos, sin = self.cos[positions][:, None, :], self.sin[positions][:, None, :]
        for li, ly in enumerate(self.layers):
            h = x0 if x is None else x
            v = ly["resid"] * h + x0 * ly["x0"]
            xm = _bf16(v)
            hn = _bf16(v * _rms(v))
            qkv = _bf16(hn @ ly["qkv"].T).view(n, 3, H, HEAD_DIM)
            q = norm_rope(qkv[:, 0], ly["q_gain"], cos, sin)
            k = norm_rope(qkv[:, 1], ly["k_gain"], cos, sin)
            val = qkv[:, 2]
            if ly["ve"] is not None:
                g = 2.0 * torch.sigmoid(hn @ ly["ve_gate"].T)[:, :, None]
                val = _bf16(val + g * self.ve_rows(ly, tokens))
            self.store(li, slots, positions, k, val)
            if cache_only_last and li == len(self.layers) - 1:
                return None
            att = _bf16(self.attend(li, q, slots, positions, ly["window"])).reshape(n, C)
            xs = att @ ly["o"].T + xm
            xo = _bf16(xs)
            p = (xo @ ly["fc"].T) * _rms(xs, divide=False)
            u = _bf16(torch.relu(p) * p)
            x = _bf16(u @ ly["proj"].T + xo)
        return x

    def ve_rows(self, ly, tokens):
        return ly["ve"][tokens].view(len(tokens), self.H, HEAD_DIM)

    def head(self, x):
        """Final norm and lm_head: logits (n, vocab) float32."""
        return _bf16(x * _rms(x)) @ self.lm_head.T
