"""Pins of oracle/model.py against closed forms and torch (float64), on tiny random models."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import model as om
from oracle.numerics import bf16_round
from oracle.rope import rotary_tables

EPS = float(np.finfo(np.float32).eps)


def tiny(L=2, C=256, Fw=512, vocab=512, T=64, seed=0, std=0.05, ve=(), window=None):
    rng = np.random.default_rng(seed)

    def mat(*shape):
        return bf16_round((rng.standard_normal(shape) * std).astype(np.float32))

    cos, sin = rotary_tables(T, 10000.0)
    layers = []
    for i in range(L):
        ly = om.LayerWeights(qkv=mat(3 * C, C), o=mat(C, C), fc=mat(Fw, C), proj=mat(C, Fw),
                             q_gain=(1 + 0.1 * rng.standard_normal(128)).astype(np.float32),
                             k_gain=(1 + 0.1 * rng.standard_normal(128)).astype(np.float32),
                             resid=1.0, x0=0.25, window=T if window is None else window)
        if i in ve:
            ly.ve = mat(vocab, C)
            ly.ve_gate = (rng.standard_normal((C // 128, C)) * std).astype(np.float32)
        layers.append(ly)
    return om.ModelWeights(wte=(rng.standard_normal((vocab, C)) * std).astype(np.float32), cos=cos, sin=sin,
                           lm_head=mat(vocab, C), layers=layers)


def rms64(x):
    return F.rms_norm(torch.tensor(x, dtype=torch.float64), (x.shape[-1],), eps=EPS).numpy()


def test_zero_mixing_layers_pass_the_embedding_through():
    """o = proj = 0: each layer's x = bf16(l1 h + l2 x0); the head is lm_head . rms_norm(x)."""
    w = tiny(L=3)
    for ly in w.layers:
        ly.o[:] = 0
        ly.proj[:] = 0
    orc = om.DecoderOracle(w, 64)
    tokens = np.array([3, 17, 200, 511])
    x = orc.body(tokens, [0, 1, 2, 3], [0, 0, 0, 0])
    x0 = rms64(w.wte[tokens].astype(np.float64))
    h = x0
    for ly in w.layers:
        h = bf16_round((ly.resid * h + ly.x0 * x0).astype(np.float32)).astype(np.float64)
    assert np.abs(x - h).max() <= 2 ** -7 * np.abs(h).max()
    logits = orc.head(x)
    expect = bf16_round(rms64(x).astype(np.float32)).astype(np.float64) @ w.lm_head.astype(np.float64).T
    assert np.abs(logits - expect).max() <= 1e-3 * np.abs(expect).max()


def test_mlp_is_relu2_of_the_normed_stream():
    """u W_proj^T with u = relu(p)^2, p = (xo W_fc^T) rstd equals torch relu(rms_norm(xo) W_fc^T)^2 W_proj^T."""
    w = tiny(L=1)
    ly = w.layers[0]
    orc = om.DecoderOracle(w, 64)
    tokens, pos = np.array([5, 6, 7]), np.array([0, 1, 2])
    x = orc.body(tokens, pos, [1, 1, 1])
    # rebuild xo from the same layer: attention output through o_proj on the oracle's own path
    x0 = (w.wte[tokens] * om.rms_scale(w.wte[tokens].astype(np.float32))).astype(np.float32)
    v = (ly.resid * x0.astype(np.float64) + (x0 * np.float32(ly.x0)).astype(np.float64)).astype(np.float32)
    xm = bf16_round(v)
    # with o = 0 the attention does not matter: xo = bf16(xm)
    ly.o[:] = 0
    orc2 = om.DecoderOracle(w, 64)
    x2 = orc2.body(tokens, pos, [1, 1, 1])
    xo = bf16_round(xm)
    t = torch.tensor(xo, dtype=torch.float64)
    p = F.linear(F.rms_norm(t, (t.shape[-1],), eps=EPS), torch.tensor(ly.fc, dtype=torch.float64))
    mlp = F.linear(torch.relu(p) ** 2, torch.tensor(ly.proj, dtype=torch.float64)).numpy() + xo
    assert np.abs(x2 - mlp).max() <= 2 ** -7 * np.abs(mlp).max() + 1e-6
    assert np.isfinite(x).all()


def test_first_position_attention_returns_its_value():
    """At position 0 the only key is the row's own: att = its value (fp8 round trip), so o_proj sees V."""
    w = tiny(L=1)
    orc = om.DecoderOracle(w, 64)
    orc.body([9], [0], [0])
    v_cached = orc.v[0][0, 0]                                  # (H, 128) dequantized
    # the same value computed directly
    x0 = (w.wte[[9]] * om.rms_scale(w.wte[[9]].astype(np.float32))).astype(np.float32)
    ly = w.layers[0]
    v = (ly.resid * x0.astype(np.float64) + (x0 * np.float32(ly.x0)).astype(np.float64)).astype(np.float32)
    hn = bf16_round((v * om.rms_scale(v)).astype(np.float32))
    val = bf16_round((hn.astype(np.float64) @ ly.qkv.astype(np.float64).T).astype(np.float32))[0, 2 * w.C:]
    val = val.reshape(w.H, 128)
    assert np.abs(v_cached - val).max() <= 2 ** -4 * np.abs(val).max()


def test_batched_prefill_equals_rows_one_at_a_time():
    w = tiny(L=3, window=5, ve=(0, 2))
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, 512, 12)
    a, b = om.DecoderOracle(w, 64), om.DecoderOracle(w, 64)
    xa = a.body(tokens, np.arange(12), np.zeros(12, int))
    xb = np.concatenate([b.body(tokens[i:i + 1], [i], [0]) for i in range(12)])
    assert np.array_equal(xa, xb)
    assert np.array_equal(a.codes[0]["k"], b.codes[0]["k"]) and np.array_equal(a.codes[0]["v"], b.codes[0]["v"])


def test_zero_gate_adds_the_value_embedding():
    """ve_gate = 0: g = 2 sigmoid(0) = 1, so v = bf16(v + ve[token])."""
    w = tiny(L=1, ve=(0,))
    ly = w.layers[0]
    ly.ve_gate[:] = 0
    plain = om.ModelWeights(wte=w.wte, cos=w.cos, sin=w.sin, lm_head=w.lm_head,
                            layers=[om.LayerWeights(**{**ly.__dict__, "ve": None, "ve_gate": None})])
    a, b = om.DecoderOracle(w, 64), om.DecoderOracle(plain, 64)
    a.body([4], [0], [0])
    b.body([4], [0], [0])
    # recover the pre-quantization v of both from a fresh computation: v_ve = bf16(v_plain + ve[4])
    v_plain = b.v[0][0, 0]
    v_ve = a.v[0][0, 0]
    e = ly.ve[4].reshape(w.H, 128)
    assert np.abs(v_ve - (v_plain + e)).max() <= 2 ** -3 * np.abs(v_plain + e).max()
    assert not np.allclose(v_ve, v_plain)


def sdpa_band(q, K, V, p, window):
    """torch scaled_dot_product_attention (float64) of one query row at position p over keys 0..p with an explicit
    boolean mask: key j is visible iff p - window <= j (window < 0: every key)."""
    qt = torch.tensor(q, dtype=torch.float64).unsqueeze(1)                       # (H, 1, 128)
    kt = torch.tensor(K[:p + 1], dtype=torch.float64).permute(1, 0, 2).contiguous()   # (H, p + 1, 128)
    vt = torch.tensor(V[:p + 1], dtype=torch.float64).permute(1, 0, 2).contiguous()
    j = torch.arange(p + 1)
    mask = (j >= p - window) if window >= 0 else torch.ones(p + 1, dtype=torch.bool)
    return F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask.view(1, 1, -1)).squeeze(1).numpy()


def test_attend_is_sdpa_with_a_band_mask():
    rng = np.random.default_rng(7)
    T, H = 90, 3
    K = rng.standard_normal((T, H, 128)).astype(np.float32)
    V = rng.standard_normal((T, H, 128)).astype(np.float32)
    for p in (0, 1, 17, 63, 89):
        q = (rng.standard_normal((H, 128)) * 2).astype(np.float32)
        for window in (-1, 0, 1, 5, 16, p, p + 40):
            got = om.attend(q, K, V, p, window)
            want = sdpa_band(q, K, V, p, window)
            assert np.abs(got - want).max() <= 1e-12, (p, window)
    # window 0: only the row's own key, so the output is its value
    assert np.abs(om.attend(q, K, V, 40, 0) - V[40]).max() <= 1e-12


@pytest.mark.parametrize("window", [0, 3, 10])
def test_window_edge_through_the_model(window):
    """One layer, window w: row p's output does not change (bitwise) when the token at p - w - 1 changes, and does when
    the token at p - w changes (K, V of a position depend only on its own token in layer 0)."""
    w = tiny(L=1, window=window, T=64)
    rng = np.random.default_rng(window)
    p = 20
    base = rng.integers(1, 512, p + 1)

    def row_p(tokens):
        orc = om.DecoderOracle(w, 64)
        return orc.body(tokens, np.arange(p + 1), np.zeros(p + 1, int))[p]

    ref = row_p(base)
    outside = base.copy()
    outside[p - window - 1] = (base[p - window - 1] + 101) % 511 + 1
    assert np.array_equal(row_p(outside), ref)
    edge = base.copy()
    edge[p - window] = (base[p - window] + 101) % 511 + 1
    assert not np.array_equal(row_p(edge), ref)
