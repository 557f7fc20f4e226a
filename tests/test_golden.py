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
