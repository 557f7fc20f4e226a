"""The paged fp8 cache's physical layout, scatter and gather — test infrastructure only.

The reference cache is contiguous bf16 `[slot][L][max_len][C]` (model/kernels/decode.cu:726, 740-763)
with a head's keys at stride C (decode.cu:577-579). The build's cache is paged:

    K, V pages    uint8 [num_pages][Hkv][2048]   one 16-token page of one KV head, fp8 codes
    K, V scales   fp32  [num_pages][Hkv][16]     one scale per (token, KV head); on the device the two are
                                                 interleaved as kv_scale [num_pages][Hkv][2][16] (K, then V)
    block table   int32 [B][max_pages]           position p of sequence b lives in page
                                                 table[b][p // 16], slot p % 16

Inside a 2048-byte page the codes are tiled for the gfx950 MFMA operands (the kernels' loads are
two 1 KiB-contiguous 16-byte-per-lane reads per page):

    K (slot k, dim d): g = d // 32, h = (d % 32) // 16        -> h*1024 + (g*16 + k)*16 + d % 16
    V (slot k, dim d): t = d // 16, r = d % 16, g = k // 4    -> (t//4)*1024 + (g*16 + r)*16 + (t%4)*4 + k%4

A contiguous cache is the identity block table (page = b * max_pages + p // 16).

Pinned by tests/test_oracle_layout.py: both maps are bijections onto 0..2047; a gather through a random
permutation block table is byte-identical to the identity table's; scatter-then-gather returns the
written codes; brute force over a tiny cache with Python loops.
"""
import numpy as np

from .quant import dequantize_rows, quantize_rows

PAGE = 16
HEAD_DIM = 128
PAGE_BYTES = PAGE * HEAD_DIM


def k_offset(slot, dim):
    g, h, j = dim // 32, (dim % 32) // 16, dim % 16
    return h * 1024 + (g * 16 + slot) * 16 + j


def v_offset(slot, dim):
    t, r = dim // 16, dim % 16
    g, kk = slot // 4, slot % 4
    return (t // 4) * 1024 + (g * 16 + r) * 16 + (t % 4) * 4 + kk


_slots, _dims = np.meshgrid(np.arange(PAGE), np.arange(HEAD_DIM), indexing="ij")
K_OFF = k_offset(_slots, _dims).astype(np.int64)   # (16, 128)
V_OFF = v_offset(_slots, _dims).astype(np.int64)


class PagedCache:
    """Host model of the device cache (same arrays, same bytes)."""

    def __init__(self, num_pages, hkv):
        self.hkv = hkv
        self.k = np.zeros((num_pages, hkv, PAGE_BYTES), np.uint8)
        self.v = np.zeros((num_pages, hkv, PAGE_BYTES), np.uint8)
        self.ks = np.zeros((num_pages, hkv, PAGE), np.float32)
        self.vs = np.zeros((num_pages, hkv, PAGE), np.float32)

    def scatter(self, pages, slots, kcodes, kscale, vcodes, vscale):
        """Store n tokens: pages, slots (n,); codes (n, Hkv, 128) uint8; scales (n, Hkv)."""
        pages = np.asarray(pages, np.int64)
        slots = np.asarray(slots, np.int64)
        hk = np.arange(self.hkv)[None, :, None]
        p3 = pages[:, None, None]
        self.k[p3, hk, K_OFF[slots][:, None, :]] = kcodes
        self.v[p3, hk, V_OFF[slots][:, None, :]] = vcodes
        h2 = np.arange(self.hkv)[None, :]
        self.ks[pages[:, None], h2, slots[:, None]] = kscale
        self.vs[pages[:, None], h2, slots[:, None]] = vscale

    def append(self, block_table, b, positions, k, v):
        """Quantize and store tokens of sequence b: positions (n,), k, v (n, Hkv, 128) fp32 holding bf16."""
        positions = np.asarray(positions, np.int64)
        pages = np.asarray(block_table)[b, positions // PAGE]
        kc, ks = quantize_rows(k)
        vc, vs = quantize_rows(v)
        self.scatter(pages, positions % PAGE, kc, ks, vc, vs)

    def gather(self, block_table, b, n):
        """Positions 0..n-1 of sequence b -> (kcodes, kscale, vcodes, vscale), codes (n, Hkv, 128)."""
        pos = np.arange(n)
        pages = np.asarray(block_table)[b, pos // PAGE].astype(np.int64)
        slots = pos % PAGE
        kc = np.take_along_axis(self.k[pages], K_OFF[slots][:, None, :], axis=2)
        vc = np.take_along_axis(self.v[pages], V_OFF[slots][:, None, :], axis=2)
        return kc, self.ks[pages, :, slots], vc, self.vs[pages, :, slots]

    def gather_values(self, block_table, b, n):
        """Dequantized K, V (n, Hkv, 128) fp32 of positions 0..n-1 of sequence b."""
        kc, ks, vc, vs = self.gather(block_table, b, n)
        return dequantize_rows(kc, ks), dequantize_rows(vc, vs)
