"""Rotary tables and the fused QK-norm + rotation — test infrastructure only.

rotary_tables restates model/modeling.py:169-176 (CausalLM.init_buffers) and
inference/modeling_nanochat.py:29-34: angles t * theta^(-2i/D) in float64, cos/sin rounded once to fp32.

qk_norm_rope restates model/kernels/qk_row.cuh:26-41 (qk_rstd, qk_rotate) and
inference/modeling_nanochat.py:37-45 (qk_norm_rope) with the build's fixed fp32 order, every
operation rounded and nothing contracted into an FMA:

    part[l] = x[l]*x[l] + x[l+64]*x[l+64]             l = 0..63 (one wave lane each)
    for o in 32, 16, 8, 4, 2, 1: part[l] = part[l] + part[l ^ o]   (xor butterfly; all lanes equal)
    r  = 1 / sqrt(part[0] / 128 + FLT_EPSILON)          (correctly rounded sqrt, then division)
    n1 = (x[l] * r) * g[l];  n2 = (x[l+64] * r) * g[l+64]
    y[l] = n1*cos[l] + n2*sin[l];  y[l+64] = n2*cos[l] - n1*sin[l]     (the -theta rotation)
    out = bf16_rne(y)

The reference's rsqrtf is an approximation whose bits cannot be reproduced here (nvcc is absent), so
the correctly rounded 1/sqrt is the build's choice; the HF restatement's torch.rsqrt is the same
division of a correctly rounded sqrt.

qk_norm_rope_backward restates the backward of model/kernels/qk_prologue.cu:36-97 (k_backward, k_gain_sum) exactly
(float64): n = x r, dm1 = dy1 cos - dy2 sin, dm2 = dy1 sin + dy2 cos, dgain = sum over rows of dm n,
dn = dm gain, dx = r (dn - n mean(dn n)).

Pinned by tests/test_oracle_rope.py: cos^2+sin^2 ~ 1 and t = 0 -> (1, 0); the position-0 case with unit
gains reduces to the textbook RMS norm (torch.nn.functional.rms_norm, fp64) within half a bf16 ulp;
a 90-degree rotation swaps the halves with a sign; a zero row gives zeros; the butterfly sum equals
math.fsum within fp32 accumulation error; and float64 brute force within one bf16 ulp everywhere. The backward
equals torch autograd of the float64 forward (rms_norm, gain, rotation) within 1e-12.
"""
import numpy as np

from .numerics import bf16_round

HEAD_DIM = 128
HALF = HEAD_DIM // 2
FLT_EPSILON = np.float32(np.finfo(np.float32).eps)


def rotary_tables(T, theta, head_dim=HEAD_DIM):
    """cos, sin (T, head_dim/2) fp32 of t * theta^(-2i/head_dim), computed in float64."""
    exponent = np.arange(0, head_dim, 2, dtype=np.float64) / head_dim
    freqs = np.outer(np.arange(T, dtype=np.float64), np.float64(theta) ** -exponent)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def butterfly_sum(part):
    """(..., 64) fp32 lane partials -> (..., 1) their wave-64 xor-butterfly sum (offsets 32..1)."""
    part = np.ascontiguousarray(part, dtype=np.float32)
    lanes = np.arange(part.shape[-1])
    o = part.shape[-1] // 2
    while o >= 1:
        part = (part + part[..., lanes ^ o]).astype(np.float32)
        o //= 2
    return part[..., :1]


def qk_norm_rope(x, gain, cos, sin):
    """x (..., 128) fp32 holding bf16; gain (128,) fp32; cos, sin broadcastable to (..., 64) -> (..., 128)
    fp32 holding the bf16 result."""
    x = np.asarray(x, dtype=np.float32)
    g = np.asarray(gain, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)
    s = np.asarray(sin, dtype=np.float32)
    x1, x2 = x[..., :HALF], x[..., HALF:]
    part = (x1 * x1 + x2 * x2).astype(np.float32)
    ss = butterfly_sum(part)
    v = (ss / np.float32(HEAD_DIM) + FLT_EPSILON).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt(v)).astype(np.float32)
    n1 = ((x1 * r) * g[:HALF]).astype(np.float32)
    n2 = ((x2 * r) * g[HALF:]).astype(np.float32)
    y1 = (n1 * c + n2 * s).astype(np.float32)
    y2 = (n2 * c - n1 * s).astype(np.float32)
    return bf16_round(np.concatenate([y1, y2], axis=-1))


def qk_norm_rope_backward(x, gain, cos, sin, dy):
    """x (rows, 128) bf16 values, gain (128,), cos, sin broadcastable to (rows, 64), dy (rows, 128) -> (dx float64
    (rows, 128), dgain float64 (128,)), exact float64 math."""
    x = np.asarray(x, np.float64)
    g = np.asarray(gain, np.float64)
    c = np.asarray(cos, np.float64)
    s = np.asarray(sin, np.float64)
    dy = np.asarray(dy, np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + float(FLT_EPSILON))
    n = x * r
    d1, d2 = dy[..., :HALF], dy[..., HALF:]
    dm = np.concatenate([d1 * c - d2 * s, d1 * s + d2 * c], axis=-1)
    dgain = np.sum(dm * n, axis=tuple(range(dm.ndim - 1)))
    dn = dm * g
    b = np.mean(dn * n, axis=-1, keepdims=True)
    return r * (dn - n * b), dgain
