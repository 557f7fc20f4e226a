"""The float32 PyTorch model step (oracle/cpu_model.py, config 5's CPU baseline) against the float64 oracle
(oracle/model.py) on a small model with a value-embedding layer and a 9-key window: the cache codes of a prefill,
then the logits and greedy tokens of decode steps; and a prompt fed in one call equals the same rows fed one at a
time."""
import numpy as np
import torch

from nanochat_amd.workloads import model_tensors
from oracle import model as om
from oracle.cpu_model import CpuDecoder


def small_model():
    return model_tensors(2, 256, 1024, 512, 64, seed=3, std=0.05, ve_layers=(1,), windows=[64, 9], device="cpu")


def prompts():
    rng = np.random.default_rng(5)
    return [[0] + [int(t) for t in rng.integers(1, 512, n - 1)] for n in (10, 17, 5)]


def test_cpu_model_matches_float64_oracle():
    m = small_model()
    orc = om.DecoderOracle(om.weights_from_tensors(m), 64)
    cpu = CpuDecoder(m, 4, 64)
    ids = prompts()
    rows = [(t, p, b) for b, q in enumerate(ids) for p, t in enumerate(q[:-1])]
    tk, ps, sl = map(list, zip(*rows))
    orc.body(tk, ps, sl, cache_only_last=True)
    assert cpu.body(tk, ps, sl, cache_only_last=True) is None
    for li in range(2):
        for b, q in enumerate(ids):
            n = len(q) - 1
            for i, name in enumerate(("k", "v")):
                same = np.mean(cpu.codes[li, b, :n, :, i].numpy() == orc.codes[b][name][li, :n])
                assert same >= 0.995, (li, b, name, same)
    inputs, pos, slots = [q[-1] for q in ids], [len(q) - 1 for q in ids], [0, 1, 2]
    for step in range(4):
        want = orc.head(orc.body(inputs, pos, slots))
        got = cpu.head(cpu.body(inputs, pos, slots)).double().numpy()
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, step          # float32 GEMMs against float64
        assert np.array_equal(got.argmax(1), want.argmax(1)), step
        inputs, pos = [int(t) for t in want.argmax(1)], [p + 1 for p in pos]


def test_prompt_in_one_call_equals_rows_one_at_a_time():
    m = small_model()
    q = prompts()[1]
    a, b = CpuDecoder(m, 2, 64), CpuDecoder(m, 2, 64)
    n = len(q) - 1
    a.body(q[:-1], list(range(n)), [0] * n, cache_only_last=True)
    for p in range(n):
        b.body([q[p]], [p], [1], cache_only_last=True)
    assert torch.equal(a.codes[:, 0, :n], b.codes[:, 1, :n])
    la = a.head(a.body([q[-1]], [n], [0]))
    lb = b.head(b.body([q[-1]], [n], [1]))
    assert torch.allclose(la, lb, rtol=0, atol=1e-5 * la.abs().max().item())
