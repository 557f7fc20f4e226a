"""Helpers shared by the GPU parity tests: build the device cache through the product path and the matching
oracle state on the host, and read the device pages back in logical (position, head, dim) order."""
import numpy as np
import torch

from nanochat_amd.kv_cache import PagedKVCache
from oracle.layout import K_OFF, PAGE, V_OFF, PagedCache
from oracle.quant import quantize_rows


def f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def device_cache(inp: dict, kv_heads: int, device) -> tuple:
    """Append the generated cache contents and the step's new token through nc_kv_append_fp8.
    Returns (cache, block_table, seq_lens) on the device; seq_lens = ctx_lens + 1."""
    cache = PagedKVCache(inp["num_pages"], kv_heads, device)
    table = inp["block_table"].to(device)
    ctx = inp["ctx_lens"].to(device)
    zeros = torch.zeros_like(ctx)
    if inp["k_cache"].shape[1]:
        cache.append(inp["k_cache"].to(device), inp["v_cache"].to(device), zeros, table, num_new=ctx)
    cache.append(inp["k_new"].to(device), inp["v_new"].to(device), ctx, table)
    torch.cuda.synchronize()
    return cache, table, ctx + 1


def oracle_cache(inp: dict, kv_heads: int, seqs) -> tuple:
    """A compact oracle cache holding sequences `seqs` (identity pages): (cache, table, seq_lens)."""
    seqs = list(seqs)
    lens = [int(inp["ctx_lens"][b]) + 1 for b in seqs]
    mp = (max(lens) + PAGE - 1) // PAGE
    table = np.arange(len(seqs) * mp, dtype=np.int32).reshape(len(seqs), mp)
    cache = PagedCache(table.size, kv_heads)
    for i, b in enumerate(seqs):
        n = lens[i] - 1
        if n:
            cache.append(table, i, np.arange(n), f32(inp["k_cache"][b, :n]), f32(inp["v_cache"][b, :n]))
        cache.append(table, i, np.array([n]), f32(inp["k_new"][b]), f32(inp["v_new"][b]))
    return cache, table, np.array(lens)


def read_sequence(cache: PagedKVCache, table: torch.Tensor, b: int, n: int):
    """Device codes and scales of positions 0..n-1 of sequence b -> (kc, ks, vc, vs) host arrays, codes
    (n, Hkv, 128)."""
    pages = table[b, : (n + PAGE - 1) // PAGE].long()
    kp = cache.k_pages.index_select(0, pages).cpu().numpy()
    vp = cache.v_pages.index_select(0, pages).cpu().numpy()
    ks = cache.k_scale.index_select(0, pages).cpu().numpy()
    vs = cache.v_scale.index_select(0, pages).cpu().numpy()
    pos = np.arange(n)
    pi, slots = pos // PAGE, pos % PAGE
    kc = np.take_along_axis(kp[pi], K_OFF[slots][:, None, :], axis=2)
    vc = np.take_along_axis(vp[pi], V_OFF[slots][:, None, :], axis=2)
    return kc, ks[pi, :, slots], vc, vs[pi, :, slots]


def expected_codes(k_rows: np.ndarray, v_rows: np.ndarray):
    kc, ks = quantize_rows(k_rows)
    vc, vs = quantize_rows(v_rows)
    return kc, ks, vc, vs


def attn_errors(got: torch.Tensor, want: np.ndarray) -> tuple[float, float]:
    d = np.abs(got.float().cpu().numpy().astype(np.float64) - want)
    return float(d.max()), float(d.mean())


def magnitude_cache(cache: PagedCache) -> PagedCache:
    """The same cache with every V code's sign cleared: attention over it gives sum_j p_j |v_j|."""
    mag = PagedCache(cache.k.shape[0], cache.hkv)
    mag.k, mag.ks, mag.vs = cache.k, cache.ks, cache.vs
    mag.v = cache.v & np.uint8(0x7F)
    return mag


# Per-element bound relative to the attention-weighted magnitude sum_j p_j |v_j|: the kernel's bf16 rounding of
# p * v_scale (2^-9), of q k products (none: fp32 accumulation of exact products) and of the output (2^-9)
# stay far inside 2^-7; a dequantization error of one e4m3 mantissa step (2^-3) does not.
REL_BOUND = 2.0 ** -7


def check_relative(got: torch.Tensor, want: np.ndarray, want_mag: np.ndarray) -> None:
    err = np.abs(got.float().cpu().numpy().astype(np.float64) - want)
    worst = float((err - REL_BOUND * want_mag).max())
    assert worst <= 1e-4, f"error exceeds 2^-7 of sum p|v| by {worst}"
