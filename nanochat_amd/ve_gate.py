"""Value-embedding gate and mix of training (csrc/ve_gate.hip): v + 2 sigmoid(n W^T) per head x bf16(table[input_ids]);
gate logits in fp32, the mix rounded once. The backward adds the table's gradient into table.grad (a leaf requiring
grad). Same functions, arguments and results as the reference's model/ops/ve_gate.py:13-33, for any head count
1 <= H <= 16 (the reference kernel is built for H = 6)."""

import ctypes

import torch
from torch import Tensor

from .native import NativeError, check, hip_library, pointer, stream


def ve_forward(n: Tensor, v: Tensor, input_ids: Tensor, table: Tensor, w: Tensor) -> tuple[Tensor, Tensor]:
    """n (B, T, C) bf16, input_ids (B, T) int32, v (B, T, H, 128) bf16 evenly spaced rows, table (V, C) and w (H, C)
    fp32 -> (mixed v contiguous, gate (B*T, H) fp32). A token outside [0, V) mixes in nothing."""
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
    """dv laid out as v, ids (B*T,) int32 sorted input_ids, order int64 their rows -> (dn, dw); the table's gradient
    added into table.grad (zeros when None)."""
    if table.grad is None:
        table.grad = torch.zeros_like(table)
    if dv.stride(-1) != 1 or dv.stride(-2) != dv.size(-1) or dv.stride(0) != dv.size(1) * dv.stride(1):
        raise NativeError("dv must be (B, T, H, 128) with contiguous heads and evenly spaced rows")
    dn, dz = torch.empty_like(n), torch.empty_like(gate, dtype=torch.bfloat16)
    check(hip_library().nc_ve_backward(pointer(dv), ctypes.c_longlong(dv.stride(1)), pointer(ids), pointer(order),
                                       pointer(table), table.size(0), pointer(w), pointer(gate), pointer(dn),
                                       pointer(table.grad), pointer(dz), ids.numel(), w.size(0), stream()))
    return dn, torch.mm(dz.t().contiguous(), n.view(-1, n.size(-1)), out_dtype=w.dtype)
