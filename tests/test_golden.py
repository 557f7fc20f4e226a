"""The committed config-1 fixture: the generator still produces the same inputs (SHA-256), and the oracle
still produces the committed cache bytes, scales and output."""
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).parent / "golden"


def test_config1_fixture():
    from tests.golden.make_golden import config1

    want = np.load(GOLDEN / "config1.npz")
    got = config1()
    assert str(got["input_sha256"]) == str(want["input_sha256"])
    for name in ("k_codes", "k_scale", "v_codes", "v_scale", "out_bf16"):
        assert np.array_equal(got[name], want[name]), name
    assert np.allclose(got["out_f64"], want["out_f64"], rtol=0, atol=1e-12)
    assert want["k_codes"].shape == (1025, 6, 128) and want["out_bf16"].shape == (1, 6, 128)


def test_rope_fixture():
    """The committed rotary slice and q/k-norm vectors regenerate bit for bit; the oracle's and the product's
    rotary tables agree with the slice (float64 angles in numpy or torch, one fp32 rounding: within one fp32 ulp,
    equal almost everywhere); the oracle's row math reproduces the committed result bits."""
    from nanochat_amd.rotary import rotary_tables as product_tables
    from oracle.numerics import bf16_bits, bf16_to_f32
    from oracle.rope import qk_norm_rope, rotary_tables
    from tests.golden.make_golden import rope_fixture

    want = np.load(GOLDEN / "rope.npz")
    got = rope_fixture()
    for name in want.files:
        assert np.array_equal(got[name], want[name]), name
    pos = want["positions"]
    for theta, key in ((1e6, "1e6"), (1e4, "1e4")):
        oc, os_ = rotary_tables(int(pos.max()) + 1, theta)
        pc, ps = (t.numpy() for t in product_tables(int(pos.max()) + 1, theta))
        for tabs in ((oc, os_), (pc, ps)):
            for got_t, name in zip(tabs, ("cos_", "sin_")):
                w = want[name + key]
                g = got_t[pos]
                assert np.all(np.abs(g.astype(np.float64) - w) <= np.spacing(np.abs(w))), (theta, name)
                assert (g != w).mean() < 0.01
    x = bf16_to_f32(want["x_bf16"])
    p = want["row_positions"]
    c, s = rotary_tables(int(p.max()) + 1, 1e6)
    y = qk_norm_rope(x, want["gain"], c[p], s[p])
    assert np.array_equal(bf16_bits(y), want["y_bf16"])
