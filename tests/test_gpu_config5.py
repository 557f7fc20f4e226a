"""Config 5 (BASELINE: 26 layers, d1664, 13 heads, vocab 65,536, random init N(0, 0.02), RoPE theta 1e6) through the
decoder runtime.

At full size (128 slots, 2,048-token prompts prefilled into the fp8 cache): every step's logits are finite, every
greedy token is the first largest logit of the logits the device computed (oracle.sampling.choose, ties to the
lowest id), and a second decoder fed the same prompts gives bit-identical logits and tokens.

Against the float64 CPU oracle (oracle/model.py) at the same width and depth, on two slots with shorter prompts (the
oracle's 26-layer float64 forward is what bounds the size): teacher-forced steps (each step's input is the device's
own choice) meet the logit bound, and the greedy tokens agree with the oracle's except at near-ties; the first step
where the oracle would choose differently is printed."""
import numpy as np
import pytest
import torch

from nanochat_amd.decoder import DecoderRuntime
from nanochat_amd.workloads import MODELS, model_tensors, prompt_tokens
from oracle import model as om
from oracle import sampling

pytestmark = pytest.mark.gpu

W = MODELS["c5"]
# 26 layers accumulate the fp32-versus-float64 rounding differences of each GEMM and the fp8 codes they flip; relative
# to the largest |logit| (the 2-3 layer tests hold 2e-2 / 3e-3)
LOGIT_MAX_REL = 5e-2
LOGIT_MEAN_REL = 8e-3


@pytest.fixture(scope="module")
def model(device):
    m = model_tensors(W.layers, W.hidden, W.ffn, W.vocab, W.max_length, seed=0, std=W.std, theta=W.theta,
                      softcap=W.softcap, device=device, generator_device="cuda")
    torch.cuda.synchronize()
    yield m
    del m
    torch.cuda.empty_cache()


def full_size_run(model, ids, steps):
    rt = DecoderRuntime(model, bos_token_id=0, max_length=W.max_length, prompt_store=0, max_slots=W.batch)
    try:
        assert rt.batch == W.batch, rt.batch
        for b in range(W.batch):
            rt.place(b, ids[b])
        assert rt.prefill() == W.batch * (W.prompt - 1)
        rt.activate(range(W.batch))
        out = []
        for _ in range(steps):
            tokens = rt.step().copy()
            logits = rt.logits(W.batch)
            out.append((logits, tokens))
        return out
    finally:
        rt.close()


def test_config5_full_size(model):
    ids = prompt_tokens(W.batch, W.prompt, W.vocab, seed=0).tolist()
    first = full_size_run(model, ids, 3)
    for step, (logits, tokens) in enumerate(first):
        assert np.isfinite(logits).all(), step
        for b in range(W.batch):
            assert tokens[b] == sampling.choose(logits[b], lazy=0)[0], (step, b)
        print(f"step {step}: |logit| max {np.abs(logits).max():.3f}, distinct tokens {len(set(tokens.tolist()))}",
              flush=True)
    second = full_size_run(model, ids, 3)
    for step, ((la, ta), (lb, tb)) in enumerate(zip(first, second)):
        assert np.array_equal(la, lb) and np.array_equal(ta, tb), step


def test_config5_teacher_forced_against_oracle(model):
    lengths = [41, 66]
    ids = [row[:n] for row, n in zip(prompt_tokens(2, max(lengths), W.vocab, seed=5).tolist(), lengths)]
    max_length = 96
    rt = DecoderRuntime(model, bos_token_id=0, max_length=max_length, prompt_store=0, max_slots=2)
    orc = om.DecoderOracle(om.weights_from_tensors(model), max_length)
    try:
        for b in range(2):
            rt.place(b, ids[b])
        rt.prefill()
        rows = [(t, p, b) for b in range(2) for p, t in enumerate(ids[b][:-1])]
        orc.body(*map(list, zip(*rows)), cache_only_last=True)
        rt.activate(range(2))
        inputs, positions = [i[-1] for i in ids], [n - 1 for n in lengths]
        diverged = None
        for step in range(4):
            tokens = rt.step().copy()
            got = rt.logits(2).astype(np.float64)
            want = orc.head(orc.body(inputs, positions, [0, 1]))
            err = np.abs(got - want)
            scale = np.abs(want).max()
            print(f"step {step}: logits max abs {err.max():.3e} mean abs {err.mean():.3e} (scale {scale:.3f})",
                  flush=True)
            assert err.max() <= LOGIT_MAX_REL * scale and err.mean() <= LOGIT_MEAN_REL * scale, step
            for b in range(2):
                best = int(np.argmax(want[b]))
                if tokens[b] != best:
                    diverged = diverged if diverged is not None else (step, b)
                    # only a near-tie of the oracle's own scores may be chosen differently
                    assert want[b][tokens[b]] >= want[b][best] - 2 * err.max(), (step, b)
            inputs, positions = [int(t) for t in tokens[:2]], [p + 1 for p in positions]
        print(f"first step where the oracle's greedy choice differs: {diverged}", flush=True)
    finally:
        rt.close()
