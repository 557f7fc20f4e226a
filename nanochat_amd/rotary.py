"""Rotary tables, computed in float64 and rounded once to fp32 (reference model/modeling.py:169-176,
CausalLM.init_buffers; inference/modeling_nanochat.py:29-34, rotary)."""
import torch

from .config import HEAD_DIM, ROPE_THETA


def rotary(positions: torch.Tensor, head_dim: int = HEAD_DIM, theta: float = ROPE_THETA):
    """cos, sin (*positions.shape, head_dim / 2) fp32 of the angles t theta^(-2i/D)."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.float64, device=positions.device) / head_dim
    freqs = positions.double()[..., None] * theta ** -exponent
    return freqs.cos().float(), freqs.sin().float()


def rotary_tables(length: int, theta: float = ROPE_THETA, device=None, head_dim: int = HEAD_DIM):
    """cos, sin (length, head_dim / 2) fp32 for positions 0..length-1, contiguous."""
    cos, sin = rotary(torch.arange(length, dtype=torch.float64), head_dim, theta)
    return cos.contiguous().to(device), sin.contiguous().to(device)
