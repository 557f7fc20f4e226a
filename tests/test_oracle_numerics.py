"""Pins oracle/numerics.py: bf16 rounding and the e4m3fn encoder/decoder against torch's CPU casts (library
routines), the closed form of e4m3fn values, and the committed exhaustive code table."""
from pathlib import Path

import numpy as np
import torch

from oracle.numerics import bf16_bits, bf16_round, bf16_to_f32, e4m3_decode, e4m3_encode

GOLDEN = Path(__file__).parent / "golden"


def all_bf16_values():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = bf16_to_f32(bits)
    return x[np.isfinite(x)]


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) < 3e38)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16_bits(x), ref)
    ties = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8)], np.float32)
    assert np.array_equal(bf16_round(ties), np.array([1.0, 1.0 + 2.0 ** -6, -1.0], np.float32))


def test_e4m3_encode_matches_torch_on_every_bf16_in_range():
    x = all_bf16_values()
    x = x[np.abs(x) <= 448]
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(e4m3_encode(x), ref)


def test_e4m3_encode_matches_torch_on_random_fp32():
    rng = np.random.default_rng(1)
    mags = np.exp2(rng.uniform(-14, np.log2(448), size=1 << 20)).astype(np.float32)
    x = (mags * rng.choice([-1, 1], size=mags.size)).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 448.0, -448.0, 2 ** -6, 2 ** -9, 2 ** -10, 3 * 2 ** -10, 1e-30])])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(e4m3_encode(x), ref)


def test_e4m3_decode_closed_form_and_torch():
    codes = np.arange(256, dtype=np.uint8)
    finite = (codes & 0x7F) != 0x7F
    vals = e4m3_decode(codes)
    for c in codes[finite]:
        s = -1.0 if c & 0x80 else 1.0
        e, m = (int(c) >> 3) & 15, int(c) & 7
        want = s * (2.0 ** (e - 7) * (1 + m / 8) if e else m * 2.0 ** -9)
        assert vals[c] == np.float32(want)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(vals[finite], ref[finite])
    assert np.array_equal(e4m3_encode(vals[finite]), codes[finite])  # round trip of every finite code


def test_committed_e4m3_table():
    """tests/golden/e4m3fn_codes.npy: the e4m3fn code of every finite bf16 value in [-448, 448] (torch's cast)."""
    table = np.load(GOLDEN / "e4m3fn_codes.npy")
    x = all_bf16_values()
    x = x[np.abs(x) <= 448]
    assert table.shape == x.shape
    assert np.array_equal(e4m3_encode(x), table)
