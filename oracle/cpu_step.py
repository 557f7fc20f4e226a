"""The CPU baseline of the fp8-KV hot path: a PyTorch (float32, all host threads) restatement of one decode step and
one chunked-prefill step — test and measurement infrastructure only (bench.py's cpu_baseline leg and tests/; nothing
in the product imports it).

A decode step, as the GPU step does it (the reference's k_prologue + k_attn, model/kernels/decode.cu:551-675):
  1. the step's token row: q and k RMS-normed (eps FLT_EPSILON), times the gains, rotated by -theta at the token's
     position, rounded to bf16 (model/kernels/qk_row.cuh:26-41; inference/modeling_nanochat.py:37-45);
  2. k and v quantized per (token, KV head): scale = max|x| / 448 (1 for a zero row), code = e4m3fn(x / scale), and
     stored into the sequence's page at the token's position;
  3. attention of the query over keys [max(p - window, 0), p] gathered through the block table and dequantized
     (fp32(code) * scale), scores (q . k) / sqrt(128), softmax, values (decode.cu:567-675), GQA by head groups.
A prefill step does the same for a chunk of rows per sequence, every row appended before any attends
(decode.cu:859-863), each row attending causally.

Layout is the natural one (pages [num_pages][Hkv][16][128] of codes, scales [num_pages][Hkv][16]): the baseline
restates the arithmetic, not the GPU's tiling. The norm sums in torch's order rather than the device's butterfly, so
its bits may differ from the device's by rounding; tests/test_oracle_cpu_step.py pins it against the float64 oracle
(oracle.rope, oracle.quant, oracle.attention).
"""
import statistics
import time

import torch

PAGE = 16
HEAD_DIM = 128
FP8_MAX = 448.0
EPS = torch.finfo(torch.float32).eps


def norm_rope(x, gain, cos, sin):
    """x (..., 128) float32 holding bf16 values; cos, sin (..., 64) broadcast over heads -> bf16-rounded float32."""
    r = 1.0 / torch.sqrt((x * x).sum(-1, keepdim=True) / HEAD_DIM + EPS)
    n = x * r * gain
    n1, n2 = n[..., :64], n[..., 64:]
    y = torch.cat([n1 * cos + n2 * sin, n2 * cos - n1 * sin], dim=-1)
    return y.to(torch.bfloat16).float()


def quantize(x):
    """x (..., 128) float32 -> (codes uint8 (..., 128) e4m3fn, scale float32 (...))."""
    amax = x.abs().amax(-1)
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    codes = (x / scale[..., None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return codes.view(torch.uint8), scale


def dequantize(codes, scale):
    return codes.view(torch.float8_e4m3fn).float() * scale[..., None]


class PagedCpuCache:
    """Codes [num_pages, Hkv, 16, 128] uint8, scales [num_pages, Hkv, 16] float32; position p of sequence b in page
    table[b, p // 16], slot p % 16."""

    def __init__(self, num_pages, hkv):
        self.k = torch.zeros(num_pages, hkv, PAGE, HEAD_DIM, dtype=torch.uint8)
        self.v = torch.zeros_like(self.k)
        self.ks = torch.zeros(num_pages, hkv, PAGE)
        self.vs = torch.zeros_like(self.ks)

    def store(self, table, b, positions, k, v):
        """k, v (n, Hkv, 128) float32 for positions (n,) of sequence b: quantize and store."""
        pages = table[b, positions // PAGE].long()
        slots = positions % PAGE
        kc, ks = quantize(k)
        vc, vs = quantize(v)
        self.k[pages, :, slots] = kc
        self.v[pages, :, slots] = vc
        self.ks[pages, :, slots] = ks
        self.vs[pages, :, slots] = vs

    def gather(self, table, lengths):
        """Dequantized K, V (B, Hkv, Lmax, 128) of the sequences' positions [0, length) (zeros past each length)."""
        Lmax = int(max(lengths))
        pages = table[:, : (Lmax + PAGE - 1) // PAGE].long()                 # (B, P)
        B, P = pages.shape

        def one(codes, scales):
            c = codes[pages]                                                   # (B, P, Hkv, 16, 128)
            s = scales[pages]                                                  # (B, P, Hkv, 16)
            x = dequantize(c, s).permute(0, 2, 1, 3, 4).reshape(B, c.shape[2], P * PAGE, HEAD_DIM)
            return x[:, :, :Lmax]

        return one(self.k, self.ks), one(self.v, self.vs)


def attend(q, K, V, positions, lengths, window=-1):
    """q (B, T, Hq, 128) float32 at positions (B, T); K, V (B, Hkv, L, 128); row (b, t) sees keys
    [max(p - window, 0), p] below lengths[b] -> (B, T, Hq, 128) float32."""
    B, T, Hq, D = q.shape
    hkv, L = K.shape[1], K.shape[2]
    G = Hq // hkv
    qg = q.view(B, T, hkv, G, D).permute(0, 2, 1, 3, 4).reshape(B, hkv, T * G, D)
    s = torch.matmul(qg, K.transpose(-1, -2)) * D ** -0.5                   # (B, Hkv, T G, L)
    j = torch.arange(L)
    p = positions.repeat_interleave(G, dim=1)[:, None, :, None]              # (B, 1, T G, 1)
    ok = (j <= p) & (j < lengths.view(B, 1, 1, 1))
    if window >= 0:
        ok &= j >= p - window
    s = s.masked_fill(~ok, float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), V)                          # (B, Hkv, T G, D)
    return o.view(B, hkv, T, G, D).permute(0, 2, 1, 3, 4).reshape(B, T, Hq, D)


def step(cache, table, qkv, start, hq, hkv, q_gain, k_gain, cos, sin, window=-1):
    """One step: qkv (B, T, (Hq + 2 Hkv) 128) float32 holding bf16 rows at positions start[b] + t; appends the rows'
    k, v, then attends -> (B, T, Hq, 128). T = 1 is a decode step."""
    B, T, _ = qkv.shape
    pos = start[:, None] + torch.arange(T)[None, :]                         # (B, T)
    c, s = cos[pos][:, :, None, :], sin[pos][:, :, None, :]                  # (B, T, 1, 64)
    x = qkv.view(B, T, hq + 2 * hkv, HEAD_DIM)
    q = norm_rope(x[:, :, :hq], q_gain, c, s)
    k = norm_rope(x[:, :, hq:hq + hkv], k_gain, c, s)
    v = x[:, :, hq + hkv:]
    for b in range(B):
        cache.store(table, b, pos[b], k[b], v[b])
    lengths = start + T
    K, V = cache.gather(table, lengths)
    return attend(q, K, V, pos, lengths, window)


def time_median(fn, runs=5, warmup=1):
    """Median seconds of `runs` calls after `warmup` calls."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_model():
    """The host CPU's model name (Linux), or 'unknown'."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"
