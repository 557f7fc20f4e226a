"""The training attention block as two registered torch ops, `nanochat_amd::attention` and
`nanochat_amd::attention_bwd`, with the argument lists, returned tensors and autograd wiring of the reference's
`nanochat::attention` / `nanochat::attention_bwd` (model/ops/flash_attn.py:325-391), so the reference's model swaps
its import (model/modeling.py:15) and calls `attention(...)` unchanged (model/modeling.py:86-87).

One block: the q/k prologue (qk_prologue.qk_forward), the value-embedding mix when a table is given
(ve_gate.ve_forward), varlen causal attention over the first `segments` document segments of cu_seqlens, windowed by
`window_left` unless the window spans the sequence (flash_attn.flash_attn_fwd, the HIP kernel of csrc/flash_attn.hip),
and the output projection with the residual: h = bf16(residual + out W^T), summed in fp32 and rounded once, and
rstd = 1 / sqrt(mean(h^2) + FLT_EPSILON) of the fp32 sum (the reference's residual_rms, model/ops/linear.py:93-100).
The projection and its two gradient products are plain library GEMMs (torch.mm, bf16 operands, fp32 sums); the
per-(token, head) row statistic the attention backward needs, dout . out, comes from the HIP kernel
`nc_flash_attn_bwd_rows` rather than from a GEMM epilogue.

The backward returns the gradients of qkv, of the two norm weights, of the normed stream n and of the gate weight
(the last two empty without value embeddings), adds o_proj's weight gradient into `o_grad` (fp32, in place) and the
table's gradient into `table.grad`; autograd passes dh through as the residual's gradient."""

import torch
from torch import Tensor
from torch.autograd.function import FunctionCtx

from .config import HEAD_DIM
from .flash_attn import fa4_window_left, flash_attn_bwd, flash_attn_bwd_rows, flash_attn_fwd
from .qk_prologue import qk_backward, qk_forward
from .ve_gate import ve_backward, ve_forward

EPS = torch.finfo(torch.float32).eps


def _block(qkv: Tensor, i: int) -> Tensor:
    """Block i (0 q, 1 k, 2 v) of the fused (B, T, 3C) projection, viewed as (B, T, H, 128)."""
    C = qkv.size(-1) // 3
    return qkv[..., i * C:(i + 1) * C].unflatten(-1, (-1, HEAD_DIM))


def _segments(cu_seqlens: Tensor, segments: Tensor) -> Tensor:
    """The offsets of the real segments: the first `segments` + 1 entries (the rest of the buffer is padding)."""
    return cu_seqlens[:int(segments) + 1]


def _project(out: Tensor, o_weight: Tensor, residual: Tensor) -> tuple[Tensor, Tensor]:
    """out (M, K) bf16, o_weight (N, K) bf16, residual (M, N) bf16 -> (bf16(residual + out W^T), rstd (M,) fp32)."""
    s = torch.mm(out, o_weight.t(), out_dtype=torch.float32).add_(residual)
    rstd = torch.sqrt(s.square().mean(-1).add_(EPS)).reciprocal_()
    return s.to(torch.bfloat16), rstd


@torch.library.custom_op("nanochat_amd::attention", mutates_args=(), device_types="cuda")
def attention(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor, sin: Tensor, window_left: int,
              cu_seqlens: Tensor, segments: Tensor, o_weight: Tensor, o_grad: Tensor | None, residual: Tensor,
              n: Tensor | None, input_ids: Tensor | None, table: Tensor | None, w_gate: Tensor | None,
              ids: Tensor | None,
              order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """qkv (B, T, 3C) bf16 fused projection, residual (B, T, C) bf16; with value embeddings n (B, T, C) bf16,
    input_ids (B, T) int32, table (V, C) and w_gate (H, C) fp32 (else None). Returns (h (B, T, C), rstd (B*T,) fp32,
    then what the backward reads: out (B, T, H, 128), lse (H, B*T) fp32, the normed and rotated q and k, the mixed v
    (empty without a table) and the gates (B*T, H) fp32 (empty without a table)). ids, order and o_grad are only
    saved for the backward."""
    T = qkv.size(1)
    cu = _segments(cu_seqlens, segments)
    qn, kn = qk_forward(_block(qkv, 0), _block(qkv, 1), q_norm_weight, k_norm_weight, cos, sin)
    if table is None:
        v, vmix, gate = _block(qkv, 2), qkv.new_empty(0), qkv.new_empty(0, dtype=torch.float32)
    else:
        vmix, gate = ve_forward(n, _block(qkv, 2), input_ids, table, w_gate)
        v = vmix
    out, lse = flash_attn_fwd(qn.flatten(0, 1), kn.flatten(0, 1), v.flatten(0, 1), cu, T,
                              window_left=fa4_window_left(window_left, T))
    h, rstd = _project(out.flatten(1), o_weight, residual.flatten(0, 1))
    return h.view(residual.shape), rstd, out.view(qn.shape), lse, qn, kn, vmix, gate


@attention.register_fake
def _attention_fake(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor, sin: Tensor,
                    window_left: int, cu_seqlens: Tensor, segments: Tensor, o_weight: Tensor, o_grad: Tensor | None,
                    residual: Tensor, n: Tensor | None, input_ids: Tensor | None, table: Tensor | None,
                    w_gate: Tensor | None, ids: Tensor | None,
                    order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    q = _block(qkv, 0)
    B, T, H = q.shape[:3]
    rows = B * T
    vmix = qkv.new_empty(0) if table is None else q.new_empty(q.shape)
    gate = qkv.new_empty((0,) if table is None else (rows, H), dtype=torch.float32)
    return (residual.new_empty(residual.shape), q.new_empty(rows, dtype=torch.float32), q.new_empty(q.shape),
            q.new_empty((H, rows), dtype=torch.float32), q.new_empty(q.shape), q.new_empty(q.shape), vmix, gate)


@torch.library.custom_op("nanochat_amd::attention_bwd", mutates_args=("o_grad",), device_types="cuda")
def attention_bwd(dh: Tensor, qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor, sin: Tensor,
                  out: Tensor, lse: Tensor, qn: Tensor, kn: Tensor, vmix: Tensor, gate: Tensor, window_left: int,
                  cu_seqlens: Tensor, segments: Tensor, o_weight: Tensor, o_grad: Tensor, n: Tensor | None,
                  table: Tensor | None, w_gate: Tensor | None, ids: Tensor | None,
                  order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """-> (d qkv, d q_norm_weight, d k_norm_weight, d n, d w_gate), the last two empty without a table; o_proj's
    weight gradient is added into o_grad and the table's into table.grad."""
    T = qkv.size(1)
    cu = _segments(cu_seqlens, segments)
    dh2 = dh.flatten(0, 1)
    x = out.flatten(2).flatten(0, 1)
    dout = torch.mm(dh2, o_weight).view(out.shape)
    o_grad.add_(torch.mm(dh2.t(), x, out_dtype=torch.float32))
    o3, do3 = out.flatten(0, 1), dout.flatten(0, 1)
    rows = flash_attn_bwd_rows(o3, do3)
    dqkv = torch.empty_like(qkv)
    dv = _block(dqkv, 2)
    v = _block(qkv, 2) if table is None else vmix
    dqn, dkn, _ = flash_attn_bwd(qn.flatten(0, 1), kn.flatten(0, 1), v.flatten(0, 1), o3, do3, lse, cu, T,
                                 window_left=fa4_window_left(window_left, T), rows=rows, dv=dv.flatten(0, 1))
    dqnw, dknw = qk_backward(_block(qkv, 0), _block(qkv, 1), q_norm_weight, k_norm_weight, dqn.view(qn.shape),
                             dkn.view(kn.shape), cos, sin, _block(dqkv, 0), _block(dqkv, 1))
    if table is None:
        return dqkv, dqnw, dknw, qkv.new_empty(0), qkv.new_empty(0)
    dn, dw = ve_backward(dv, n, ids, order, table, w_gate, gate)
    return dqkv, dqnw, dknw, dn, dw


@attention_bwd.register_fake
def _attention_bwd_fake(dh: Tensor, qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor,
                        sin: Tensor, out: Tensor, lse: Tensor, qn: Tensor, kn: Tensor, vmix: Tensor, gate: Tensor,
                        window_left: int, cu_seqlens: Tensor, segments: Tensor, o_weight: Tensor, o_grad: Tensor,
                        n: Tensor | None, table: Tensor | None, w_gate: Tensor | None, ids: Tensor | None,
                        order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    with_table = table is not None
    return (torch.empty_like(qkv), torch.empty_like(q_norm_weight), torch.empty_like(k_norm_weight),
            torch.empty_like(n) if with_table else qkv.new_empty(0),
            torch.empty_like(w_gate) if with_table else qkv.new_empty(0))


def _save(ctx: FunctionCtx, inputs: tuple, output: tuple[Tensor, ...]) -> None:
    (qkv, q_norm_weight, k_norm_weight, cos, sin, ctx.window_left, cu_seqlens, segments, o_weight, o_grad, _, n, _,
     table, w_gate, ids, order) = inputs
    # rstd is differentiated by the next block's norm, not here; the rest are the backward's operands
    ctx.mark_non_differentiable(*output[1:])
    ctx.save_for_backward(qkv, q_norm_weight, k_norm_weight, cos, sin, *output[2:], cu_seqlens, segments, o_weight,
                          o_grad, n, table, w_gate, ids, order)


def _grad(ctx: FunctionCtx, dh: Tensor, *_: Tensor) -> tuple:
    """Gradients in input order: qkv, the two norm weights, (cos, sin, window, cu_seqlens, segments, o_weight,
    o_grad: none), the residual (= dh), n, (input_ids, table: none), w_gate, (ids, order: none)."""
    (qkv, qnw, knw, cos, sin, out, lse, qn, kn, vmix, gate, cu_seqlens, segments, o_weight, o_grad, n, table, w_gate,
     ids, order) = ctx.saved_tensors
    dqkv, dqnw, dknw, dn, dw = attention_bwd(dh, qkv, qnw, knw, cos, sin, out, lse, qn, kn, vmix, gate,
                                             ctx.window_left, cu_seqlens, segments, o_weight, o_grad, n, table,
                                             w_gate, ids, order)
    with_table = table is not None
    return (dqkv, dqnw, dknw, None, None, None, None, None, None, None, dh, dn if with_table else None, None, None,
            dw if with_table else None, None, None)


attention.register_autograd(_grad, setup_context=_save)
