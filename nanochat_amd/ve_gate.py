"""Training-side value embeddings on MI355X (csrc/ve_gate.hip), drop-in for the reference's model/ops/ve_gate.py:13-33
(same function names, arguments and returned tensors) at any head count 1 <= H <= 16 (the reference's kernel is fixed
at H = 6).

Each token row's value heads receive its embedding-table row scaled by a per-head gate: out = v + g * bf16(table[id])
with g = 2 * sigmoid(w_head . n) from the row's normed stream n. The gate logits are fp32 dot products and the sum is
rounded to bf16 once. The backward returns the gradients of n and w and accumulates the table's gradient into
table.grad, creating it as zeros when absent."""

import ctypes

import torch
from torch import Tensor

from .native import NativeError, check, hip_library, pointer, stream


def ve_forward(n: Tensor, v: Tensor, input_ids: Tensor, table: Tensor, w: Tensor) -> tuple[Tensor, Tensor]:
    """Mix value embeddings into v. Shapes: n (B, T, C) bf16; v (B, T, H, 128) bf16 with contiguous heads and one row
    stride; input_ids (B, T) int32; table (V, C) and w (H, C) fp32. Returns the mixed values as a new contiguous
    tensor shaped like v, and the gates (B*T, H) fp32 the backward needs. Ids outside [0, V) add nothing."""
    if v.stride(-1) != 1 or v.stride(-2) != v.size(-1) or v.stride(0) != v.size(1) * v.stride(1):
        raise NativeError("v must be (B, T, H, 128) with contiguous heads and evenly spaced rows")
    if not (n.is_contiguous() and input_ids.is_contiguous() and table.is_contiguous() and w.is_contiguous()):
        raise NativeError("n, input_ids, table and w must be contiguous")
    out, gate = v.new_empty(v.shape), v.new_empty((input_ids.numel(), w.size(0)), dtype=torch.float32)
    check(hip_library().nc_ve_forward(pointer(n), pointer(v), ctypes.c_longlong(v.stride(1)),
                                      pointer(input_ids), pointer(table), table.size(0), pointer(w),
                                      pointer(out), pointer(gate), input_ids.numel(), w.size(0), stream()))
    return out, gate


def ve_backward(dv: Tensor, n: Tensor, ids: Tensor, order: Tensor, table: Tensor, w: Tensor,
                gate: Tensor) -> tuple[Tensor, Tensor]:
    """Gradients of ve_forward. dv is the output's gradient, laid out like v; ids (B*T,) int32 are the input ids sorted
    (equal ids adjacent) and order (B*T,) int64 the row each came from; gate is ve_forward's. Returns (dn like n,
    dw like w); the table's gradient is added into table.grad (allocated as zeros when it is None)."""
    if table.grad is None:
        table.grad = torch.zeros_like(table)
    if dv.stride(-1) != 1 or dv.stride(-2) != dv.size(-1) or dv.stride(0) != dv.size(1) * dv.stride(1):
        raise NativeError("dv must be (B, T, H, 128) with contiguous heads and evenly spaced rows")
    dn, dz = torch.empty_like(n), torch.empty_like(gate, dtype=torch.bfloat16)
    check(hip_library().nc_ve_backward(pointer(dv), ctypes.c_longlong(dv.stride(1)), pointer(ids), pointer(order),
                                       pointer(table), table.size(0), pointer(w), pointer(gate), pointer(dn),
                                       pointer(table.grad), pointer(dz), ids.numel(), w.size(0), stream()))
    return dn, torch.mm(dz.t().contiguous(), n.view(-1, n.size(-1)), out_dtype=w.dtype)
