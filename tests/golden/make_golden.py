"""Writes the committed fixtures of tests/golden (run from the repository root: python tests/golden/make_golden.py).

- e4m3fn_codes.npy: torch's CPU float8_e4m3fn code of every finite bf16 value in [-448, 448], ascending
  bf16 bit pattern order (the library routine the oracle's encoder is pinned to).
- config1.npz: BASELINE config 1 (B=1, 6/6 heads, 1024 cached tokens + 1 appended, seed 0): the SHA-256 of
  the generated inputs, the oracle's fp8 codes and scales of all 1025 positions (logical [pos][head][dim]
  order), and the oracle's attention output rounded to bf16.
- rope.npz: a slice of the rotary tables (positions 0, 1, 2, 3, 1000, 2047, 4096, 8192; all 64 columns) at
  theta 1e6 (the model's) and 1e4 (config 4's), written from torch's float64 cos / sin rounded to fp32, and tiny
  q/k-norm + rotation vectors: 12 bf16 rows of 128 (seeded N(0,1), one all-zero row, one with a 2^10 outlier)
  at positions up to 8192 (theta 1e6) with a seeded fp32 gain, and the oracle's bf16 result bits.
"""
import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from nanochat_amd.workloads import DECODE, decode_inputs  # noqa: E402
from oracle.attention import decode_attention  # noqa: E402
from oracle.layout import PagedCache  # noqa: E402
from oracle.numerics import bf16_bits, bf16_to_f32  # noqa: E402

OUT = Path(__file__).resolve().parent


def f32(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


def input_digest(inputs: dict) -> str:
    h = hashlib.sha256()
    for name in ("q", "k_cache", "v_cache", "k_new", "v_new", "block_table", "ctx_lens"):
        t = inputs[name]
        h.update(name.encode())
        h.update((t.view(torch.int16) if t.dtype == torch.bfloat16 else t).numpy().tobytes())
    return h.hexdigest()


def config1():
    inp = decode_inputs(DECODE["c1"], seed=0)
    table = inp["block_table"].numpy()
    cache = PagedCache(inp["num_pages"], DECODE["c1"].kv_heads)
    n = DECODE["c1"].ctx
    cache.append(table, 0, np.arange(n), f32(inp["k_cache"][0]), f32(inp["v_cache"][0]))
    cache.append(table, 0, np.array([n]), f32(inp["k_new"][0]), f32(inp["v_new"][0]))
    kc, ks, vc, vs = cache.gather(table, 0, n + 1)
    out = decode_attention(f32(inp["q"]), cache, table, np.array([n + 1]))
    return dict(input_sha256=np.array(input_digest(inp)), k_codes=kc, k_scale=ks, v_codes=vc, v_scale=vs,
                out_bf16=bf16_bits(out.astype(np.float32)), out_f64=out)


ROPE_POSITIONS = [0, 1, 2, 3, 1000, 2047, 4096, 8192]


def rope_slice(theta):
    """cos, sin [len(ROPE_POSITIONS)][64] fp32 from torch float64: t * theta^(-2i/128)."""
    t = torch.tensor(ROPE_POSITIONS, dtype=torch.float64)[:, None]
    ang = t * torch.tensor(float(theta), dtype=torch.float64) ** (-torch.arange(0, 128, 2, dtype=torch.float64) / 128)
    return torch.cos(ang).float().numpy(), torch.sin(ang).float().numpy()


def rope_vectors():
    from oracle.rope import qk_norm_rope
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(12, 128, generator=gen)
    x[3] = 0.0
    x[7, 5] = 1024.0
    x = x.to(torch.bfloat16).float().numpy()
    gain = (1 + 0.1 * torch.randn(128, generator=gen)).numpy()
    pos = np.array([0, 1, 17, 1000, 2047, 8192, 0, 5, 4096, 3, 100, 2047])
    ang = torch.tensor(pos, dtype=torch.float64)[:, None] * \
        torch.tensor(1e6, dtype=torch.float64) ** (-torch.arange(0, 128, 2, dtype=torch.float64) / 128)
    c, s = torch.cos(ang).float().numpy(), torch.sin(ang).float().numpy()
    y = qk_norm_rope(x, gain, c, s)
    return dict(x_bf16=bf16_bits(x), gain=gain, row_positions=pos, y_bf16=bf16_bits(y))


def rope_fixture():
    c6, s6 = rope_slice(1e6)
    c4, s4 = rope_slice(1e4)
    return dict(positions=np.array(ROPE_POSITIONS), cos_1e6=c6, sin_1e6=s6, cos_1e4=c4, sin_1e4=s4, **rope_vectors())


def e4m3_table():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = bf16_to_f32(bits)
    x = x[np.isfinite(x) & (np.abs(x) <= 448)]
    return torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


if __name__ == "__main__":
    np.save(OUT / "e4m3fn_codes.npy", e4m3_table())
    np.savez_compressed(OUT / "config1.npz", **config1())
    np.savez_compressed(OUT / "rope.npz", **rope_fixture())
    for f in sorted(OUT.glob("*.np*")):
        print(f.name, f.stat().st_size)
