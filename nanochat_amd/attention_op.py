"""The training attention block as two registered torch ops, `nanochat_amd::attention` and
`nanochat_amd::attention_bwd`.

Interface: the argument lists, the eight returned tensors and the gradient positions are those of the reference's
`nanochat::attention` / `nanochat::attention_bwd` (model/ops/flash_attn.py:325-391), so the reference's model swaps
its import (model/modeling.py:15) and calls `attention(...)` unchanged (model/modeling.py:86-87).

What one call computes, on the fused (B, T, 3C) projection split into q, k and v heads:

1. q and k through the RMS norm, their gains and the -theta rotation (qk_prologue.qk_forward);
2. with a value-embedding table, v mixed with its gated table rows (ve_gate.ve_forward);
3. varlen causal attention inside each of the first `segments` document segments of cu_seqlens, limited to
   `window_left` keys back unless that spans the sequence (flash_attn.flash_attn_fwd, csrc/flash_attn.hip);
4. the output projection added to the residual in fp32 and rounded once, h = bf16(residual + out W^T), with
   rstd = 1 / sqrt(mean(h^2) + FLT_EPSILON) of the fp32 sum (the reference's residual_rms, model/ops/linear.py:93-100).

The projection's three products are library GEMMs (bf16 operands, fp32 sums). The attention backward's per-(token,
head) statistic dout . out comes from the HIP kernel `nc_flash_attn_bwd_rows`.

Layout of this module: every tensor the ops return is described once by a spec (shape and dtype as functions of the
inputs); the eager ops allocate their placeholders from it and the fake (meta) implementations return it whole. The
autograd wiring names what it keeps and what it differentiates against the op's input list, so the saved operands
and the gradient tuple follow from those names."""

from typing import NamedTuple

import torch
from torch import Tensor
from torch.autograd.function import FunctionCtx

from .config import HEAD_DIM
from .flash_attn import fa4_window_left, flash_attn_bwd, flash_attn_bwd_rows, flash_attn_fwd
from .qk_prologue import qk_backward, qk_forward
from .ve_gate import ve_backward, ve_forward

EPS = torch.finfo(torch.float32).eps
BF16, F32 = torch.bfloat16, torch.float32

# The forward op's inputs, positionally (model/modeling.py:86-87 passes them in this order).
FORWARD_INPUTS = ("qkv", "q_norm_weight", "k_norm_weight", "cos", "sin", "window_left", "cu_seqlens", "segments",
                  "o_weight", "o_grad", "residual", "n", "input_ids", "table", "w_gate", "ids", "order")
# The forward op's outputs: the block's result, then what the backward reads back.
FORWARD_OUTPUTS = ("h", "rstd", "out", "lse", "qn", "kn", "vmix", "gate")
# The backward op's inputs: dh, then forward inputs and outputs by name.
BACKWARD_INPUTS = ("dh", "qkv", "q_norm_weight", "k_norm_weight", "cos", "sin", "out", "lse", "qn", "kn", "vmix",
                   "gate", "window_left", "cu_seqlens", "segments", "o_weight", "o_grad", "n", "table", "w_gate",
                   "ids", "order")
# The backward op's outputs, each the gradient of the named forward input.
BACKWARD_OUTPUTS = ("qkv", "q_norm_weight", "k_norm_weight", "n", "w_gate")
# Only h carries a gradient out of the forward; rstd is differentiated by the next block's norm.
DIFFERENTIABLE_OUTPUTS = ("h",)
# The residual's gradient is dh itself.
PASSED_THROUGH = {"residual": "dh"}

# What the autograd context keeps: the tensors among the backward's inputs (window_left rides on ctx as an int).
SAVED = tuple(name for name in BACKWARD_INPUTS if name not in ("dh", "window_left"))


class Heads(NamedTuple):
    """The fused projection's three (B, T, H, 128) views (token stride 3C), and the sizes they fix."""
    q: Tensor
    k: Tensor
    v: Tensor
    B: int
    T: int
    H: int

    @classmethod
    def of(cls, qkv: Tensor) -> "Heads":
        B, T, width = qkv.shape
        H = width // (3 * HEAD_DIM)
        q, k, v = qkv.unflatten(-1, (3, H, HEAD_DIM)).unbind(2)
        return cls(q, k, v, B, T, H)


def forward_spec(qkv: Tensor, residual: Tensor, with_table: bool) -> dict[str, tuple[tuple[int, ...], torch.dtype]]:
    """Shape and dtype of each forward output. Without a table the mix and the gates are empty."""
    s = Heads.of(qkv)
    tokens, head = s.B * s.T, (s.B, s.T, s.H, HEAD_DIM)
    return {"h": (tuple(residual.shape), residual.dtype), "rstd": ((tokens,), F32), "out": (head, BF16),
            "lse": ((s.H, tokens), F32), "qn": (head, BF16), "kn": (head, BF16),
            "vmix": (head if with_table else (0,), BF16), "gate": ((tokens, s.H) if with_table else (0,), F32)}


def backward_spec(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, n: Tensor | None,
                  w_gate: Tensor | None) -> dict[str, tuple[tuple[int, ...], torch.dtype]]:
    """Shape and dtype of each backward output (the gradient of the input of the same name)."""
    like = {"qkv": qkv, "q_norm_weight": q_norm_weight, "k_norm_weight": k_norm_weight, "n": n, "w_gate": w_gate}
    return {name: ((0,), qkv.dtype) if t is None else (tuple(t.shape), t.dtype) for name, t in like.items()}


def allocate(template: Tensor, spec: dict, names=None) -> dict[str, Tensor]:
    """Uninitialized tensors for the named entries of a spec (all of them by default), on template's device."""
    return {name: template.new_empty(spec[name][0], dtype=spec[name][1]) for name in (names or spec)}


def real_segments(cu_seqlens: Tensor, segments: Tensor) -> Tensor:
    """cu_seqlens is a padded buffer; the document offsets are its leading segments + 1 entries."""
    return cu_seqlens.narrow(0, 0, int(segments) + 1)


@torch.library.custom_op("nanochat_amd::attention", mutates_args=(), device_types="cuda")
def attention(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor, sin: Tensor, window_left: int,
              cu_seqlens: Tensor, segments: Tensor, o_weight: Tensor, o_grad: Tensor | None, residual: Tensor,
              n: Tensor | None, input_ids: Tensor | None, table: Tensor | None, w_gate: Tensor | None,
              ids: Tensor | None,
              order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """qkv (B, T, 3C) bf16 and residual (B, T, C) bf16. Value embeddings, when used: n (B, T, C) bf16, input_ids
    (B, T) int32, table (V, C) fp32, w_gate (H, C) fp32. o_grad, ids and order are read by the backward only.
    Returns the tensors FORWARD_OUTPUTS names, shaped as forward_spec says."""
    s = Heads.of(qkv)
    res = {}
    res["qn"], res["kn"] = qk_forward(s.q, s.k, q_norm_weight, k_norm_weight, cos, sin)
    if table is not None:
        res["vmix"], res["gate"] = ve_forward(n, s.v, input_ids, table, w_gate)
    else:
        res.update(allocate(qkv, forward_spec(qkv, residual, False), ("vmix", "gate")))
    values = s.v if table is None else res["vmix"]
    out, res["lse"] = flash_attn_fwd(res["qn"].flatten(0, 1), res["kn"].flatten(0, 1), values.flatten(0, 1),
                                     real_segments(cu_seqlens, segments), s.T,
                                     window_left=fa4_window_left(window_left, s.T))
    res["out"] = out.view(s.B, s.T, s.H, HEAD_DIM)
    total = torch.mm(out.flatten(1), o_weight.t(), out_dtype=F32)
    total += residual.flatten(0, 1)
    res["rstd"] = (total.square().mean(-1) + EPS).sqrt().reciprocal()    # correctly rounded sqrt, then 1/x
    res["h"] = total.to(BF16).view(residual.shape)
    return tuple(res[name] for name in FORWARD_OUTPUTS)


@attention.register_fake
def _(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor, sin: Tensor, window_left: int,
      cu_seqlens: Tensor, segments: Tensor, o_weight: Tensor, o_grad: Tensor | None, residual: Tensor,
      n: Tensor | None, input_ids: Tensor | None, table: Tensor | None, w_gate: Tensor | None, ids: Tensor | None,
      order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    made = allocate(qkv, forward_spec(qkv, residual, table is not None))
    return tuple(made[name] for name in FORWARD_OUTPUTS)


@torch.library.custom_op("nanochat_amd::attention_bwd", mutates_args=("o_grad",), device_types="cuda")
def attention_bwd(dh: Tensor, qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor, sin: Tensor,
                  out: Tensor, lse: Tensor, qn: Tensor, kn: Tensor, vmix: Tensor, gate: Tensor, window_left: int,
                  cu_seqlens: Tensor, segments: Tensor, o_weight: Tensor, o_grad: Tensor, n: Tensor | None,
                  table: Tensor | None, w_gate: Tensor | None, ids: Tensor | None,
                  order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The gradients BACKWARD_OUTPUTS names (those of n and w_gate empty without a table). o_proj's weight gradient is
    added into o_grad (fp32), the table's into table.grad."""
    s = Heads.of(qkv)
    grads = allocate(qkv, backward_spec(qkv, q_norm_weight, k_norm_weight, n, w_gate), ("qkv", "n", "w_gate"))
    dq_in, dk_in, dv = Heads.of(grads["qkv"])[:3]
    # o_proj: out's gradient, and the weight's, from the block result's gradient dh
    tokens_dh = dh.flatten(0, 1)
    out_rows = out.flatten(0, 1)
    o_grad += torch.mm(tokens_dh.t(), out_rows.flatten(1), out_dtype=F32)
    dout = torch.mm(tokens_dh, o_weight).view(out_rows.shape)
    # attention: the value gradient lands straight in its block of d qkv
    values = s.v if table is None else vmix
    dqn, dkn, _ = flash_attn_bwd(qn.flatten(0, 1), kn.flatten(0, 1), values.flatten(0, 1), out_rows, dout, lse,
                                 real_segments(cu_seqlens, segments), s.T,
                                 window_left=fa4_window_left(window_left, s.T),
                                 rows=flash_attn_bwd_rows(out_rows, dout), dv=dv.flatten(0, 1))
    # the prologue writes q's and k's input gradients into their blocks of d qkv
    grads["q_norm_weight"], grads["k_norm_weight"] = qk_backward(
        s.q, s.k, q_norm_weight, k_norm_weight, dqn.view(qn.shape), dkn.view(kn.shape), cos, sin, dq_in, dk_in)
    if table is not None:
        grads["n"], grads["w_gate"] = ve_backward(dv, n, ids, order, table, w_gate, gate)
    return tuple(grads[name] for name in BACKWARD_OUTPUTS)


@attention_bwd.register_fake
def _(dh: Tensor, qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor, sin: Tensor, out: Tensor,
      lse: Tensor, qn: Tensor, kn: Tensor, vmix: Tensor, gate: Tensor, window_left: int, cu_seqlens: Tensor,
      segments: Tensor, o_weight: Tensor, o_grad: Tensor, n: Tensor | None, table: Tensor | None,
      w_gate: Tensor | None, ids: Tensor | None, order: Tensor | None) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    with_table = table is not None
    made = allocate(qkv, backward_spec(qkv, q_norm_weight, k_norm_weight, n if with_table else None,
                                       w_gate if with_table else None))
    return tuple(made[name] for name in BACKWARD_OUTPUTS)


def _setup_context(ctx: FunctionCtx, inputs: tuple, output: tuple) -> None:
    named = dict(zip(FORWARD_INPUTS, inputs)) | dict(zip(FORWARD_OUTPUTS, output))
    ctx.window_left = named["window_left"]
    ctx.mark_non_differentiable(*(named[o] for o in FORWARD_OUTPUTS if o not in DIFFERENTIABLE_OUTPUTS))
    ctx.save_for_backward(*(named[name] for name in SAVED))


def _backward(ctx: FunctionCtx, dh: Tensor, *_: Tensor) -> tuple:
    named = dict(zip(SAVED, ctx.saved_tensors), dh=dh, window_left=ctx.window_left)
    got = dict(zip(BACKWARD_OUTPUTS, attention_bwd(*(named[name] for name in BACKWARD_INPUTS))))
    if named["table"] is None:                      # no value embeddings: n and w_gate took no part
        del got["n"], got["w_gate"]
    got.update({name: named[source] for name, source in PASSED_THROUGH.items()})
    return tuple(got.get(name) for name in FORWARD_INPUTS)


attention.register_autograd(_backward, setup_context=_setup_context)
