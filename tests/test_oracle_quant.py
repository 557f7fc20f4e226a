"""Pins oracle/quant.py: the absmax element maps to +-448, the half-ulp error bound, zero rows, clamping."""
import numpy as np

from oracle.numerics import bf16_round, e4m3_decode
from oracle.quant import dequantize_rows, quantize_rows


def rows(seed, n=4096, outliers=0.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 128)).astype(np.float32)
    if outliers:
        m = rng.random(x.shape) < outliers
        x[m] = 8 * np.sign(x[m])
    return bf16_round(x)


def test_amax_element_maps_to_448():
    for seed in range(3):
        x = rows(seed)
        codes, scale = quantize_rows(x)
        i = np.argmax(np.abs(x), axis=1)
        top = codes[np.arange(len(x)), i]
        want = np.where(x[np.arange(len(x)), i] > 0, 0x7E, 0xFE)
        assert np.array_equal(top, want)
        assert np.array_equal(scale, (np.max(np.abs(x), axis=1) / np.float32(448)).astype(np.float32))


def test_error_within_half_ulp():
    for seed, out in ((0, 0.0), (1, 0.01)):
        x = rows(seed, outliers=out)
        codes, scale = quantize_rows(x)
        y = x.astype(np.float64) / scale[:, None].astype(np.float64)   # exact quotient
        back = e4m3_decode(codes).astype(np.float64)
        normal = np.abs(back) >= 2 ** -6
        err = np.abs(back - np.clip(y, -448, 448))
        # half an e4m3 ulp (2^-4 relative) plus the fp32 rounding of x / scale
        assert np.all(err[normal] <= np.abs(y[normal]) * (2 ** -4 + 2 ** -22))
        assert np.all(err[~normal] <= 2 ** -10 * (1 + 2 ** -20))
        deq = dequantize_rows(codes, scale)
        assert np.all(np.abs(deq - x) <= np.abs(x) * 2 ** -4 * 1.001 + scale[:, None] * 2 ** -10)


def test_zero_row_and_single_value():
    x = np.zeros((2, 128), np.float32)
    x[1, 5] = -3.0
    codes, scale = quantize_rows(x)
    assert scale[0] == 1.0 and not codes[0].any()
    assert scale[1] == np.float32(3.0 / 448) and codes[1, 5] == 0xFE and not np.delete(codes[1], 5).any()


def test_quotient_above_448_clamps():
    # amax / (amax / 448) can round above 448 in fp32; the clamp keeps the code at 0x7E, never NaN (0x7F)
    rng = np.random.default_rng(7)
    x = bf16_round(rng.uniform(-1000, 1000, (20000, 128)).astype(np.float32))
    codes, _ = quantize_rows(x)
    assert not np.any((codes & 0x7F) == 0x7F)
