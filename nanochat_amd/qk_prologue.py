"""Fused q/k prologue, training form: drop-in for the reference's model/ops/qk_prologue.py (qk_forward :13-21,
qk_backward :24-36).

Per (token, head) row of q and k: RMS norm (eps FLT_EPSILON), fp32 per-dimension gain and the -theta
rotation (reference model/kernels/qk_row.cuh:26-41), fp32 math and one bf16 rounding. q, k are
(B, T, H, 128) bf16 views of the fused projection (token stride 3*H*128); cos, sin fp32 [T, 64].
"""
import torch
from torch import Tensor

from .config import HEAD_DIM
from .native import NativeError, hip_library, pointer, stream


def qk_forward(q: Tensor, k: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor,
               sin: Tensor) -> tuple[Tensor, Tensor]:
    """New contiguous tensors holding q and k after the norm, the gain and the rotation (same shape, bf16)."""
    B, T, H = q.shape[:3]
    for name, t in (("q", q), ("k", k)):
        if not t.is_cuda or t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be a bf16 device tensor")
        if t.shape != (B, T, H, HEAD_DIM) or t.stride() != (T * 3 * H * HEAD_DIM, 3 * H * HEAD_DIM, HEAD_DIM, 1):
            raise ValueError(f"{name} must be a (B, T, H, {HEAD_DIM}) view of the fused qkv projection")
    for name, t in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight), ("cos", cos), ("sin", sin)):
        if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous fp32 device tensor")
    if cos.shape[0] < T or sin.shape[0] < T:
        raise ValueError(f"cos/sin need {T} positions")
    q_out, k_out = q.new_empty(q.shape), k.new_empty(k.shape)
    lib = hip_library()
    lib.qkp_forward(pointer(q), pointer(k), pointer(q_norm_weight), pointer(k_norm_weight), pointer(q_out),
                    pointer(k_out), pointer(cos), pointer(sin), B * T * H, H, T, stream())
    status = lib.nc_last_error()
    if status:
        raise NativeError(f"qkp_forward: {lib.nc_status_string(status).decode()}")
    return q_out, k_out


def qk_backward(q: Tensor, k: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, dq_out: Tensor, dk_out: Tensor,
                cos: Tensor, sin: Tensor, dq: Tensor, dk: Tensor) -> tuple[Tensor, Tensor]:
    """Backward of qk_forward. dq_out, dk_out (contiguous) are the gradients of its two outputs; the inputs' gradients
    are stored into dq, dk (bf16 views with q's and k's shape and strides), and the two gain gradients (fp32, HEAD_DIM)
    are returned. The gain gradients are reduced over rows in one fixed order, so repeated calls agree bit for bit."""
    B, T, H, D = q.shape
    for name, t in (("q", q), ("k", k), ("dq", dq), ("dk", dk)):
        if not t.is_cuda or t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be a bf16 device tensor")
        if t.shape != (B, T, H, HEAD_DIM) or t.stride() != (T * 3 * H * HEAD_DIM, 3 * H * HEAD_DIM, HEAD_DIM, 1):
            raise ValueError(f"{name} must be a (B, T, H, {HEAD_DIM}) view of a fused qkv tensor")
    for name, t in (("dq_out", dq_out), ("dk_out", dk_out)):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.shape != q.shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 device tensor shaped like q")
    for name, t in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight), ("cos", cos), ("sin", sin)):
        if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous fp32 device tensor")
    if cos.shape[0] < T or sin.shape[0] < T:
        raise ValueError(f"cos/sin need {T} positions")
    dq_norm_weight, dk_norm_weight = torch.empty_like(q_norm_weight), torch.empty_like(k_norm_weight)
    lib = hip_library()
    part = q_norm_weight.new_empty((2 * lib.qkp_backward_blocks(), D))
    lib.qkp_backward(pointer(q), pointer(k), pointer(q_norm_weight), pointer(k_norm_weight), pointer(dq_out),
                     pointer(dk_out), pointer(dq), pointer(dk), pointer(dq_norm_weight), pointer(dk_norm_weight),
                     pointer(part), pointer(cos), pointer(sin), B * T * H, H, T, stream())
    status = lib.nc_last_error()
    if status:
        raise NativeError(f"qkp_backward: {lib.nc_status_string(status).decode()}")
    return dq_norm_weight, dk_norm_weight
