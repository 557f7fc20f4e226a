"""RoPE angle tables for the kernels: position t, frequency column i (i < head_dim / 2) holds cos and sin of
t * theta^(-2 i / head_dim), the angle evaluated in float64 and each value rounded once to fp32 — the same numbers
the reference's model builds (model/modeling.py:169-176, inference/modeling_nanochat.py:29-34). Host torch on the CPU;
callers move the tables to the device."""
import torch

from .config import HEAD_DIM, ROPE_THETA


def rotary(positions: torch.Tensor, head_dim: int = HEAD_DIM, theta: float = ROPE_THETA):
    """(cos, sin) of every position in `positions` (any shape) times the head's frequencies: two fp32 tensors shaped
    (*positions.shape, head_dim // 2)."""
    inv_freq = theta ** -(torch.arange(0, head_dim, 2, dtype=torch.float64, device=positions.device) / head_dim)
    angle = positions.to(torch.float64).unsqueeze(-1) * inv_freq
    return torch.cos(angle).to(torch.float32), torch.sin(angle).to(torch.float32)


def rotary_tables(length: int, theta: float = ROPE_THETA, device=None, head_dim: int = HEAD_DIM):
    """Contiguous fp32 tables (length, head_dim // 2) of cos and sin for positions 0 .. length - 1, on `device`."""
    cos, sin = rotary(torch.arange(length, dtype=torch.float64), head_dim, theta)
    return cos.contiguous().to(device), sin.contiguous().to(device)
