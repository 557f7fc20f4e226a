"""Training attention (csrc/flash_attn.hip): the varlen causal, optionally windowed, attention the reference runs
through FlashAttention-4 at model/ops/flash_attn.py:340-345 (`_flash_attn_fwd(q, k, v, cu_seqlens, cu_seqlens, T, T,
causal=True, window_size_left=window, return_lse=True)`) and differentiates at :367-391 (`_flash_attn_bwd` with the
precomputed row statistics, or `bwd_bf16dq` for window layers), with FA4's window rule (fa4_window_left,
flash_attn.py:309-311: None, i.e. no limit, when the window spans the sequence)."""

import math

import torch
from torch import Tensor

from .config import HEAD_DIM
from .native import NativeError, check, hip_library, pointer, stream


def _heads(t: Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16 or not t.is_cuda:
        raise NativeError(f"{name} must be a bf16 device tensor")
    if t.dim() != 3 or t.size(-1) != HEAD_DIM or t.stride(-1) != 1 or t.stride(-2) != HEAD_DIM:
        raise NativeError(f"{name} must be (total, H, {HEAD_DIM}) with contiguous heads")


def fa4_window_left(window_left: int, T: int) -> int | None:
    """None (plain causal) when the window spans T, else the window (the reference's flash_attn.py:309-311)."""
    return None if window_left >= T else window_left


def flash_attn_fwd(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: int,
                   window_left: int | None = None, softmax_scale: float | None = None) -> tuple[Tensor, Tensor]:
    """q, k, v (total, H, 128) bf16 (contiguous heads, any token stride), cu_seqlens int32 (segments + 1) ->
    (out (total, H, 128) bf16, lse (H, total) fp32, natural log)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        _heads(t, name)
    if k.shape != q.shape or v.shape != q.shape:
        raise NativeError("q, k and v must have the same shape")
    if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_contiguous() or not cu_seqlens.is_cuda:
        raise NativeError("cu_seqlens must be a contiguous int32 device tensor")
    total, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    out = torch.empty(total, H, D, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(H, total, dtype=torch.float32, device=q.device)
    window = -1 if window_left is None else window_left
    check(hip_library().nc_flash_attn_fwd(pointer(q), pointer(k), pointer(v), q.stride(0), k.stride(0), v.stride(0),
                                          pointer(cu_seqlens), cu_seqlens.numel() - 1, max_seqlen, H, window, scale,
                                          pointer(out), pointer(lse), total, stream()))
    return out, lse


def flash_attn_bwd_rows(out: Tensor, dout: Tensor) -> Tensor:
    """D = dout . out per (token, head): (total, H) fp32, the reference's `rows`."""
    _heads(out, "out")
    _heads(dout, "dout")
    total, H, _ = out.shape
    rows = torch.empty(total, H, dtype=torch.float32, device=out.device)
    check(hip_library().nc_flash_attn_bwd_rows(pointer(out), out.stride(0), pointer(dout), dout.stride(0), total, H,
                                               pointer(rows), stream()))
    return rows


def flash_attn_bwd(q: Tensor, k: Tensor, v: Tensor, out: Tensor, dout: Tensor, lse: Tensor, cu_seqlens: Tensor,
                   max_seqlen: int, window_left: int | None = None, softmax_scale: float | None = None,
                   rows: Tensor | None = None, dv: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """Gradients of flash_attn_fwd: -> (dq, dk, dv), bf16 (total, H, 128); dv, when given (any token stride with
    contiguous heads, e.g. the v block of a fused projection's gradient), is written in place. rows: D = dout . out
    (total, H) fp32, computed from out and dout when None."""
    for name, t in (("q", q), ("k", k), ("v", v), ("dout", dout)):
        _heads(t, name)
    if lse.dtype != torch.float32 or lse.dim() != 2 or lse.stride(1) != 1:
        raise NativeError("lse must be (H, total) fp32 with contiguous rows")
    if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_contiguous() or not cu_seqlens.is_cuda:
        raise NativeError("cu_seqlens must be a contiguous int32 device tensor")
    total, H, D = q.shape
    if rows is None:
        rows = flash_attn_bwd_rows(out, dout)
    if rows.dtype != torch.float32 or not rows.is_contiguous() or tuple(rows.shape) != (total, H):
        raise NativeError("rows must be (total, H) contiguous fp32")
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    dq, dk = torch.empty_like(q, memory_format=torch.contiguous_format), torch.empty(total, H, D, dtype=q.dtype,
                                                                                     device=q.device)
    if dv is None:
        dv = torch.empty(total, H, D, dtype=q.dtype, device=q.device)
    _heads(dv, "dv")
    window = -1 if window_left is None else window_left
    check(hip_library().nc_flash_attn_bwd(
        pointer(q), pointer(k), pointer(v), pointer(dout), q.stride(0), k.stride(0), v.stride(0), dout.stride(0),
        pointer(lse), lse.stride(0), pointer(rows), pointer(cu_seqlens), cu_seqlens.numel() - 1, max_seqlen, H, window,
        scale, pointer(dq), pointer(dk), pointer(dv), dq.stride(0), dk.stride(0), dv.stride(0), stream()))
    return dq, dk, dv
