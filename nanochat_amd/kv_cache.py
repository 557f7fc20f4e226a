"""The paged fp8 KV cache in HBM and its block tables.

The reference keeps one contiguous bf16 cache per slot, `[L][max_len][C]` (model/kernels/decode.cu:726,
740-763). Here one layer's cache is a pool of pages shared by all sequences:

    k_pages, v_pages  uint8 [num_pages, Hkv, 2048]   e4m3fn codes of 16 tokens of one KV head, in the MFMA
                                                     tiling of nanochat_amd/csrc/nc_device.h
    kv_scale          fp32  [num_pages, Hkv, 2, 16]  one absmax/448 scale per (token, KV head): K, then V
                                                     (k_scale and v_scale are views of its two halves)

and a sequence reaches its pages through an int32 block table row (position p -> page
table[b, p // 16], slot p % 16). A contiguous cache is the identity table.
"""
import torch

from .config import HEAD_DIM, PAGE_BYTES, PAGE_SIZE
from .native import check, hip_library, pointer, stream


def _require(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor (the fp8 KV path has no CPU implementation)")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def pages_for(length: int) -> int:
    """Pages holding `length` positions."""
    return (length + PAGE_SIZE - 1) // PAGE_SIZE


def contiguous_block_table(batch: int, max_pages: int, device=None) -> torch.Tensor:
    """Identity table: sequence b owns pages b*max_pages .. (b+1)*max_pages - 1."""
    return torch.arange(batch * max_pages, dtype=torch.int32, device=device).view(batch, max_pages)


def permuted_block_table(batch: int, max_pages: int, generator: torch.Generator, device=None) -> torch.Tensor:
    """A random permutation of the batch*max_pages pages, assigned in order (drawn on the CPU generator)."""
    perm = torch.randperm(batch * max_pages, generator=generator).to(torch.int32)
    return perm.view(batch, max_pages).to(device)


class PagedKVCache:
    """One layer's page pool. Pages start zeroed (codes 0, scales 0)."""

    def __init__(self, num_pages: int, num_kv_heads: int, device):
        self.num_pages, self.num_kv_heads = num_pages, num_kv_heads
        self.k_pages = torch.zeros(num_pages, num_kv_heads, PAGE_BYTES, dtype=torch.uint8, device=device)
        self.v_pages = torch.zeros_like(self.k_pages)
        self.kv_scale = torch.zeros(num_pages, num_kv_heads, 2, PAGE_SIZE, dtype=torch.float32, device=device)
        self.k_scale, self.v_scale = self.kv_scale[:, :, 0], self.kv_scale[:, :, 1]
        for name in ("k_pages", "v_pages", "kv_scale"):
            t = getattr(self, name)
            _require(t, name, t.dtype)

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.k_pages, self.v_pages, self.kv_scale))

    def check_table(self, block_table: torch.Tensor) -> None:
        _require(block_table, "block_table", torch.int32)
        if block_table.dim() != 2:
            raise ValueError("block_table must be [B, max_pages]")

    def append(self, k: torch.Tensor, v: torch.Tensor, start_pos: torch.Tensor, block_table: torch.Tensor,
               num_new: torch.Tensor | None = None) -> None:
        """Quantize and store k, v (bf16 [B, T, Hkv, 128], inner dims contiguous) at positions start_pos[b] + t."""
        B, T, H, D = k.shape
        if v.shape != k.shape or H != self.num_kv_heads or D != HEAD_DIM:
            raise ValueError(f"k, v must be [B, T, {self.num_kv_heads}, {HEAD_DIM}], got {tuple(k.shape)}, "
                             f"{tuple(v.shape)}")
        for name, t in (("k", k), ("v", v)):
            if t.dtype != torch.bfloat16 or not t.is_cuda:
                raise TypeError(f"{name} must be a bf16 device tensor")
            if t.stride(3) != 1 or t.stride(2) != HEAD_DIM or t.stride(0) != T * t.stride(1):
                raise ValueError(f"{name} must have contiguous heads and a uniform token stride")
        if k.stride() != v.stride():
            raise ValueError("k and v must share strides")
        _require(start_pos, "start_pos", torch.int32)
        if num_new is not None:
            _require(num_new, "num_new", torch.int32)
        self.check_table(block_table)
        check(hip_library().nc_kv_append_fp8(
            pointer(k), pointer(v), k.stride(1), B, T, H, pointer(start_pos),
            pointer(num_new) if num_new is not None else None, pointer(block_table), block_table.size(1),
            pointer(self.k_pages), pointer(self.v_pages), pointer(self.kv_scale), self.num_pages, stream()))
