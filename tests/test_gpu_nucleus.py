"""The decoder's nucleus threshold (choose_kernel's top-p cut, through dec_debug_nucleus_cut) against the oracle's
restatement of the same integer rule (oracle/sampling.py:nucleus_cut_fixed): the threshold's bit pattern must be
equal for every row. Rows cover the config-5 vocabulary and a ragged one, temperatures that make the distribution
flat or peaked, top_p from 0 to just under 1, masked rows, exact ties, rows that weigh nothing, a row with nothing
allowed, and a peaked row whose nucleus is one token."""
import numpy as np
import pytest
import torch

from nanochat_amd.native import hip_library, pointer, stream
from oracle import sampling

pytestmark = pytest.mark.gpu


def probabilities(rng, vocab, T, spread, allowed_frac):
    z = sampling.capped((rng.standard_normal(vocab) * spread).astype(np.float32), 15.0)
    allowed = rng.random(vocab) < allowed_frac
    if allowed_frac > 0:
        allowed[int(rng.integers(vocab))] = True
    zt = np.where(allowed, z / np.float32(T), -np.inf).astype(np.float32)
    if not allowed.any():
        return np.zeros(vocab, np.float32)
    return np.where(allowed, np.exp(zt - zt[allowed].max()), 0).astype(np.float32)


def device_cuts(e_rows, top_p, device):
    e = torch.from_numpy(np.ascontiguousarray(e_rows)).to(device)
    p = torch.tensor(top_p, dtype=torch.float32, device=device)
    cut = torch.empty(e.size(0), dtype=torch.int32, device=device)
    lib = hip_library("decode")
    assert lib.dec_debug_nucleus_cut(pointer(e), e.size(0), e.size(1), pointer(p), pointer(cut), stream()) == 0
    torch.cuda.synchronize()
    return cut.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("vocab", [65536, 50000])
def test_nucleus_cut_bits_equal_the_oracle(device, vocab):
    rng = np.random.default_rng(vocab)
    rows, top_p = [], []
    for T, spread, frac, p in ((1.0, 2.0, 1.0, 0.9), (0.7, 3.0, 1.0, 0.5), (1.3, 1.0, 0.9, 0.99),
                               (0.5, 4.0, 1.0, 0.999999), (1.0, 2.0, 0.5, 0.0), (2.0, 0.5, 1.0, 0.95),
                               (0.9, 8.0, 1.0, 0.8), (1.0, 2.0, 0.01, 0.7), (1.0, 1.0, 1.0, 1e-7),
                               (0.3, 6.0, 1.0, 0.9)):
        rows.append(probabilities(rng, vocab, T, spread, frac))
        top_p.append(p)
    tied = np.full(vocab, 0.25, np.float32)                     # every row equal but a few at the maximum
    tied[rng.choice(vocab, 5, replace=False)] = 1.0
    rows += [tied, tied]
    top_p += [0.5, 1e-4]
    light = np.zeros(vocab, np.float32)                         # weights at the fixed-point floor
    light[: vocab // 2] = np.float32(2.0 ** -39)
    light[: vocab // 4] = np.float32(2.0 ** -38)
    light[7] = 1.0
    rows.append(light)
    top_p.append(0.9999999)
    rows.append(np.zeros(vocab, np.float32))                    # nothing allowed
    top_p.append(0.9)
    peaked = np.zeros(vocab, np.float32)
    peaked[123] = 1.0
    peaked[5:40] = 1e-6
    rows.append(peaked)
    top_p.append(0.9)
    e_rows = np.stack(rows)
    got = device_cuts(e_rows, top_p, device)
    want = np.array([sampling.nucleus_cut_fixed(e, p) for e, p in zip(e_rows, top_p)], np.uint32)
    assert (got == want).all(), [(i, hex(g), hex(w)) for i, (g, w) in enumerate(zip(got, want)) if g != w]
    assert want[-2] == 0xFFFFFFFF
    assert (e_rows[-1].view(np.uint32) >= want[-1]).sum() == 1

