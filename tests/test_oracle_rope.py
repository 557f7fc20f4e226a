"""Pins oracle/rope.py against closed forms and textbook routines: table identities, the RMS-norm special
case (torch rms_norm in float64), a quarter-turn rotation, zero rows, the butterfly sum, and a float64 brute
force within one bf16 ulp; plus the product's torch rotary tables against the oracle's."""
import math

import numpy as np
import pytest
import torch

from oracle.numerics import bf16_round
from oracle.rope import butterfly_sum, qk_norm_rope, rotary_tables


def bf16_rows(seed, n, scale=1.0):
    rng = np.random.default_rng(seed)
    return bf16_round((rng.standard_normal((n, 128)) * scale).astype(np.float32))


def test_tables_identities():
    cos, sin = rotary_tables(4097, 1e6)
    assert cos.dtype == np.float32 and cos.shape == (4097, 64)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    assert np.allclose(cos.astype(np.float64) ** 2 + sin.astype(np.float64) ** 2, 1, atol=2e-7)
    # column 0 is the angle t itself
    t = np.arange(4097, dtype=np.float64)
    assert np.array_equal(cos[:, 0], np.cos(t).astype(np.float32))


def test_product_tables_match_oracle():
    from nanochat_amd.rotary import rotary_tables as product_tables

    for theta in (1e4, 1e6):
        c, s = product_tables(8193, theta)
        oc, os_ = rotary_tables(8193, theta)
        for a, b in ((c.numpy(), oc), (s.numpy(), os_)):
            # the fp64 angle may differ in its last bit (pow): equal except within 2^-24 absolute near a zero
            assert np.all(np.abs(a.astype(np.float64) - b) <= 2 ** -24) and (a != b).mean() < 1e-4


def test_position_zero_is_rms_norm():
    x = bf16_rows(0, 2048, 3.0)
    g = np.ones(128, np.float32)
    y = qk_norm_rope(x, g, np.ones(64, np.float32), np.zeros(64, np.float32))
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (128,), eps=float(np.finfo(np.float32).eps))
    ref = ref.numpy()
    # one bf16 rounding of a value within a few fp32 ulps of the exact norm
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2 ** -8 * 1.01 + 1e-30)


def test_quarter_turn_swaps_halves():
    x = bf16_rows(1, 256)
    g = np.ones(128, np.float32)
    plain = qk_norm_rope(x, g, np.ones(64, np.float32), np.zeros(64, np.float32))
    turned = qk_norm_rope(x, g, np.zeros(64, np.float32), np.ones(64, np.float32))
    assert np.array_equal(turned[:, :64], plain[:, 64:])      # y1 = m2
    assert np.array_equal(turned[:, 64:], -plain[:, :64])     # y2 = -m1 (the -theta sign)


def test_zero_row_gives_zero():
    y = qk_norm_rope(np.zeros((1, 128), np.float32), np.full(128, 2, np.float32), np.full(64, .5, np.float32),
                     np.full(64, .5, np.float32))
    assert not np.any(y)


def test_butterfly_sum_close_to_exact():
    rng = np.random.default_rng(2)
    part = rng.random((1000, 64)).astype(np.float32)
    got = butterfly_sum(part)[:, 0].astype(np.float64)
    exact = np.array([math.fsum(r.astype(np.float64)) for r in part])
    assert np.all(np.abs(got - exact) <= exact * 6 * 2 ** -24)


def test_brute_force_float64():
    x = bf16_rows(3, 512, 2.0)
    rng = np.random.default_rng(4)
    g = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    cos, sin = rotary_tables(512, 1e4)
    y = qk_norm_rope(x, g, cos, sin)
    xd = x.astype(np.float64)
    m = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + np.finfo(np.float32).eps) * g
    c, s = cos.astype(np.float64), sin.astype(np.float64)
    ref = np.concatenate([m[:, :64] * c + m[:, 64:] * s, m[:, 64:] * c - m[:, :64] * s], -1)
    # one bf16 rounding (half an ulp) plus fp32 arithmetic error: within one bf16 ulp of the exact value
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    assert np.all(np.abs(y - ref) <= ulp + 1e-6)


def test_backward_equals_torch_autograd():
    """oracle.rope.qk_norm_rope_backward against autograd of the float64 forward: rms_norm (eps FLT_EPSILON), gain,
    the -theta rotation of halves (reference qk_row.cuh:33-41)."""
    import torch

    from oracle.rope import FLT_EPSILON, qk_norm_rope_backward, rotary_tables

    rng = np.random.default_rng(0)
    rows, T = 40, 16
    x = rng.standard_normal((rows, 128))
    g = 1 + 0.2 * rng.standard_normal(128)
    dy = rng.standard_normal((rows, 128))
    cos, sin = rotary_tables(T, 10000.0)
    pos = np.arange(rows) % T
    c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
    xt = torch.tensor(x, requires_grad=True)
    gt = torch.tensor(g, requires_grad=True)
    n = torch.nn.functional.rms_norm(xt, (128,), eps=float(FLT_EPSILON)) * gt
    ct, st = torch.tensor(c), torch.tensor(s)
    y = torch.cat([n[:, :64] * ct + n[:, 64:] * st, n[:, 64:] * ct - n[:, :64] * st], dim=1)
    y.backward(torch.tensor(dy))
    dx, dg = qk_norm_rope_backward(x, g, c, s, dy)
    assert np.abs(dx - xt.grad.numpy()).max() <= 1e-12 * max(1.0, np.abs(dx).max())
    assert np.abs(dg - gt.grad.numpy()).max() <= 1e-12 * max(1.0, np.abs(dg).max())


@pytest.mark.parametrize("theta,column,omega", [
    (1e4, 32, 0.01), (1e4, 16, 0.1), (1e4, 48, 0.001),
    (1e6, 16, 10 ** -1.5), (1e6, 32, 1e-3), (1e6, 48, 10 ** -4.5), (1e6, 8, 10 ** -0.75)])
def test_interior_columns_have_the_closed_form_frequency(theta, column, omega):
    """Column i's angle is t theta^(-2i/128): for these (theta, i) the frequency is a power of ten written out here
    (theta^(-1/2) = 0.01 for theta = 1e4, i = 32, ...), so an exponent of i/D or (2i+1)/D, a swapped sin/cos or a
    wrong theta fails. The table is the fp32 rounding of the float64 cos / sin: within one fp32 ulp of math.cos / sin
    (a different libm), and equal almost everywhere."""
    cos, sin = rotary_tables(8193, theta)
    t = np.arange(8193)
    want_c = np.array([math.cos(omega * x) for x in t], np.float32)
    want_s = np.array([math.sin(omega * x) for x in t], np.float32)
    for got, want in ((cos[:, column], want_c), (sin[:, column], want_s)):
        ulp = np.spacing(np.abs(want)).astype(np.float64)
        assert np.all(np.abs(got.astype(np.float64) - want) <= ulp), (theta, column)
        assert (got != want).mean() < 1e-3


@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_column_frequencies_fall_by_theta_to_the_minus_one_64th(theta):
    """The frequencies recovered from the table (atan2 of sin / cos at a position where the angle is below pi) form
    the geometric series omega_i = theta^(-i/64): omega_0 = 1 and each column's over the previous is theta^(-1/64)."""
    cos, sin = rotary_tables(8193, theta)
    omegas = []
    for i in range(64):
        t = 1
        while t * 2 < 8193 and np.arctan2(sin[t * 2, i], cos[t * 2, i]) > 0 and t * 2 * np.arctan2(sin[1, i], cos[1, i]) < 3.0:
            t *= 2
        omegas.append(np.arctan2(float(sin[t, i]), float(cos[t, i])) / t)
    omegas = np.array(omegas)
    assert abs(omegas[0] - 1.0) < 1e-6
    ratio = theta ** (-1.0 / 64)
    assert np.allclose(omegas[1:] / omegas[:-1], ratio, rtol=2e-4), (omegas[1:] / omegas[:-1])[:4]
