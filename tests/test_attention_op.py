"""The registered training attention ops without a GPU: both ops exist under torch.ops.nanochat_amd, and their fake
(meta) implementations give the shapes and dtypes of the reference's nanochat::attention / attention_bwd
(model/ops/flash_attn.py:349-361, 394-403), with and without value embeddings, so torch.compile can trace a model
that calls them; and the autograd wiring, run on meta tensors: which inputs receive a gradient and of which shape
(model/ops/flash_attn.py:416-425). That the residual's gradient equals dh is checked on the GPU."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import nanochat_amd.attention_op  # noqa: F401  (registers the ops)


def fake_inputs(B, T, H, vocab, with_table, d="cuda"):
    C = H * 128
    bf = dict(dtype=torch.bfloat16, device=d)
    args = dict(qkv=torch.empty(B, T, 3 * C, **bf), q_norm_weight=torch.empty(128, device=d),
                k_norm_weight=torch.empty(128, device=d), cos=torch.empty(T, 64, device=d),
                sin=torch.empty(T, 64, device=d), window_left=T, cu_seqlens=torch.empty(9, dtype=torch.int32, device=d),
                segments=torch.empty((), dtype=torch.int64, device=d), o_weight=torch.empty(C, C, **bf),
                o_grad=torch.empty(C, C, device=d), residual=torch.empty(B, T, C, **bf))
    ve = dict(n=None, input_ids=None, table=None, w_gate=None, ids=None, order=None)
    if with_table:
        ve = dict(n=torch.empty(B, T, C, **bf), input_ids=torch.empty(B, T, dtype=torch.int32, device=d),
                  table=torch.empty(vocab, C, device=d), w_gate=torch.empty(H, C, device=d),
                  ids=torch.empty(B * T, dtype=torch.int32, device=d),
                  order=torch.empty(B * T, dtype=torch.int64, device=d))
    return args, ve


def test_ops_are_registered():
    assert hasattr(torch.ops.nanochat_amd, "attention")
    assert hasattr(torch.ops.nanochat_amd, "attention_bwd")


def test_fake_shapes_match_the_reference_ops():
    B, T, H, vocab = 2, 96, 3, 50
    C, rows = H * 128, B * T
    for with_table in (False, True):
        with FakeTensorMode():
            a, ve = fake_inputs(B, T, H, vocab, with_table)
            outs = torch.ops.nanochat_amd.attention(*a.values(), *ve.values())
            shapes = [(tuple(o.shape), o.dtype) for o in outs]
            head = (B, T, H, 128)
            assert shapes[:6] == [((B, T, C), torch.bfloat16), ((rows,), torch.float32), (head, torch.bfloat16),
                                  ((H, rows), torch.float32), (head, torch.bfloat16), (head, torch.bfloat16)]
            if with_table:
                assert shapes[6:] == [(head, torch.bfloat16), ((rows, H), torch.float32)]
            else:
                assert [s for s, _ in shapes[6:]] == [(0,), (0,)]
            grads = torch.ops.nanochat_amd.attention_bwd(a["residual"], a["qkv"], a["q_norm_weight"],
                                                         a["k_norm_weight"], a["cos"], a["sin"], *outs[2:],
                                                         a["window_left"], a["cu_seqlens"], a["segments"],
                                                         a["o_weight"], a["o_grad"], ve["n"], ve["table"],
                                                         ve["w_gate"], ve["ids"], ve["order"])
            gshapes = [tuple(g.shape) for g in grads]
            assert gshapes[:3] == [(B, T, 3 * C), (128,), (128,)]
            assert gshapes[3:] == ([(B, T, C), (H, C)] if with_table else [(0,), (0,)])


def test_gradients_reach_the_reference_positions():
    B, T, H, vocab = 2, 48, 2, 40
    C = H * 128
    for with_table in (False, True):
        a, ve = fake_inputs(B, T, H, vocab, with_table, d="meta")
        wanted = {"qkv": (B, T, 3 * C), "q_norm_weight": (128,), "k_norm_weight": (128,), "residual": (B, T, C)}
        if with_table:
            wanted.update(n=(B, T, C), w_gate=(H, C))
        inputs = {**a, **ve}
        for name in wanted:
            inputs[name].requires_grad_()
        if with_table:
            inputs["table"].requires_grad_()        # the table's gradient goes to table.grad inside the op, not here
        outs = torch.ops.nanochat_amd.attention(*inputs.values())
        assert [o.requires_grad for o in outs] == [True] + [False] * 7
        outs[0].backward(torch.empty_like(outs[0]))
        got = {k: tuple(v.grad.shape) for k, v in inputs.items() if isinstance(v, torch.Tensor) and v.grad is not None}
        assert got == wanted, (with_table, got)
