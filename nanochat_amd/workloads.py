"""Synthetic, seeded inputs of the BASELINE configurations (host tensors; the caller moves them to HBM).

Every draw comes from one `torch.Generator().manual_seed(seed)` on the CPU in a documented order, fp32
normal draws rounded to bf16, so a GPU run and the CPU oracle see identical bytes.

Decode (configs 1-3 and the derived headline 3u), order of draws:
  1. ragged only: context lengths  randint(ctx_min, ctx + 1, (B,))
  2. q [B, Hq, 128], k_cache [B, ctx, Hkv, 128], v_cache (same), k_new [B, 1, Hkv, 128], v_new (same)
  3. outliers only, per tensor in the order k_cache, v_cache, k_new, v_new: mask = rand < fraction,
     x[mask] = 8 * sign(x[mask])
  4. paged only: randperm of B * max_pages pages, assigned in order (max_pages = pages of ctx + 1)
Chunked prefill (config 4), order of draws: qkv [B, T, (Hq + 2 Hkv) * 128], k_cache, v_cache
[B, ctx, Hkv, 128], q_gain and k_gain = 1 + 0.1 * randn(128), then the block-table permutation.
End-to-end decoding (config 5), random-init weights (model_tensors), order of draws: wte [vocab, C] (fp32),
lm_head [vocab, C]; per layer qkv [3C, C], o [C, C], fc [F, C], proj [C, F], q_norm and k_norm = 1 + 0.1 randn(128),
then on value-embedding layers ve [vocab, C] and ve_gate [H, C]; every matrix std * randn (bf16 but wte and ve_gate);
then the prompts (prompt_tokens): randint(1, vocab, (B, prompt)) with BOS (0) first.
"""
from dataclasses import dataclass

import torch

from .config import HEAD_DIM, ROPE_THETA
from .kv_cache import pages_for


@dataclass(frozen=True)
class DecodeWorkload:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    ctx: int               # cached tokens before the step (the maximum when ragged)
    ctx_min: int = 0       # ragged lower bound; 0 = uniform context
    paged: bool = False    # random-permutation block table; False = identity (contiguous)
    outliers: float = 0.0  # fraction of cache values replaced by +-8 sigma
    description: str = ""


@dataclass(frozen=True)
class PrefillWorkload:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    ctx: int               # cached tokens before the chunk
    chunk: int             # tokens appended and attended per sequence
    theta: float = 10000.0
    paged: bool = True
    description: str = ""


DECODE = {
    "c1": DecodeWorkload("c1", 1, 6, 6, 1024, description="CPU plumbing: B=1, 6/6 heads, 1024 cached + 1"),
    "c2": DecodeWorkload("c2", 32, 10, 10, 4096, description="d20 shape: B=32, 10/10 heads, 4096 cached + 1"),
    "c3": DecodeWorkload("c3", 64, 16, 4, 8192, ctx_min=512, paged=True, outliers=0.01,
                         description="ragged GQA: B=64, 16/4 heads, ctx U[512, 8192] + 1, 16-token pages"),
    "c3u": DecodeWorkload("c3u", 64, 16, 4, 8192, paged=True, outliers=0.01,
                          description="headline bs64 ctx8K: B=64, 16/4 heads, 8192 cached + 1, 16-token pages"),
}

PREFILL = {
    "c4": PrefillWorkload("c4", 8, 16, 4, 3584, 512,
                          description="chunked prefill: B=8, 512-token chunk onto 3584 cached, 16/4 heads"),
}


def _bf16_randn(gen: torch.Generator, *shape: int) -> torch.Tensor:
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)


def _outliers(gen: torch.Generator, x: torch.Tensor, fraction: float) -> torch.Tensor:
    mask = torch.rand(x.shape, generator=gen) < fraction
    return torch.where(mask, 8.0 * torch.sign(x.float()), x.float()).to(torch.bfloat16)


def decode_ctx_lens(w: DecodeWorkload, gen: torch.Generator) -> torch.Tensor:
    """The sequences' cached lengths: U[ctx_min, ctx] from gen's next draw, or ctx for every sequence."""
    if w.ctx_min:
        return torch.randint(w.ctx_min, w.ctx + 1, (w.batch,), generator=gen, dtype=torch.int64).to(torch.int32)
    return torch.full((w.batch,), w.ctx, dtype=torch.int32)


def decode_inputs(w: DecodeWorkload, seed: int = 0) -> dict:
    """Host tensors of one decode step: the cache contents before it, the new token, the block table."""
    gen = torch.Generator().manual_seed(seed)
    B, D = w.batch, HEAD_DIM
    ctx_lens = decode_ctx_lens(w, gen)
    q = _bf16_randn(gen, B, w.q_heads, D)
    k_cache = _bf16_randn(gen, B, w.ctx, w.kv_heads, D)
    v_cache = _bf16_randn(gen, B, w.ctx, w.kv_heads, D)
    k_new = _bf16_randn(gen, B, 1, w.kv_heads, D)
    v_new = _bf16_randn(gen, B, 1, w.kv_heads, D)
    if w.outliers:
        k_cache, v_cache, k_new, v_new = (_outliers(gen, x, w.outliers) for x in (k_cache, v_cache, k_new, v_new))
    max_pages = pages_for(w.ctx + 1)
    if w.paged:
        table = torch.randperm(B * max_pages, generator=gen).to(torch.int32).view(B, max_pages)
    else:
        table = torch.arange(B * max_pages, dtype=torch.int32).view(B, max_pages)
    return dict(ctx_lens=ctx_lens, q=q, k_cache=k_cache, v_cache=v_cache, k_new=k_new, v_new=v_new,
                block_table=table, num_pages=B * max_pages, max_seq_len=w.ctx + 1)


def prefill_inputs(w: PrefillWorkload, seed: int = 0) -> dict:
    """Host tensors of one chunked-prefill step."""
    gen = torch.Generator().manual_seed(seed)
    B, D = w.batch, HEAD_DIM
    qkv = _bf16_randn(gen, B, w.chunk, (w.q_heads + 2 * w.kv_heads) * D)
    k_cache = _bf16_randn(gen, B, w.ctx, w.kv_heads, D)
    v_cache = _bf16_randn(gen, B, w.ctx, w.kv_heads, D)
    q_gain = 1.0 + 0.1 * torch.randn(D, generator=gen, dtype=torch.float32)
    k_gain = 1.0 + 0.1 * torch.randn(D, generator=gen, dtype=torch.float32)
    max_pages = pages_for(w.ctx + w.chunk)
    if w.paged:
        table = torch.randperm(B * max_pages, generator=gen).to(torch.int32).view(B, max_pages)
    else:
        table = torch.arange(B * max_pages, dtype=torch.int32).view(B, max_pages)
    return dict(qkv=qkv, k_cache=k_cache, v_cache=v_cache, q_gain=q_gain, k_gain=k_gain, block_table=table,
                num_pages=B * max_pages, start_pos=torch.full((B,), w.ctx, dtype=torch.int32))


@dataclass(frozen=True)
class ModelWorkload:
    name: str
    layers: int
    hidden: int
    ffn: int
    vocab: int
    batch: int             # slots decoding together
    prompt: int            # tokens of each prompt, BOS included (all but the last are prefilled)
    steps: int             # greedy decode steps (tokens generated per slot)
    std: float = 0.02      # weight init N(0, std)
    theta: float = ROPE_THETA
    softcap: float = 15.0
    description: str = ""

    @property
    def max_length(self) -> int:
        """Cache positions a slot needs: the prompt but its last token, then one per step."""
        return self.prompt - 1 + self.steps


MODELS = {
    "c5": ModelWorkload("c5", 26, 1664, 4 * 1664, 65536, 128, 2048, 512,
                        description="end-to-end greedy decode: 26 layers, d1664, 13 heads, vocab 65536, B=128, "
                                    "2048-token prompts, 512 steps"),
}


def model_tensors(layers: int, hidden: int, ffn: int, vocab: int, max_length: int, *, seed: int = 0,
                  std: float = 0.02, theta: float = ROPE_THETA, softcap: float = 15.0, ve_layers=(), windows=None,
                  resid_lambda: float = 1.0, x0_lambda: float = 0.1, device=None, generator_device="cpu"):
    """Random-init decoder inputs (a decoder.ModelTensors on `device`), drawn in the order the module docstring
    lists from a generator on generator_device ("cpu": the bytes a CPU oracle can redraw; a GPU generator draws
    the large models fast). windows: keys before a query per layer (None: max_length, full attention)."""
    from .decoder import LayerTensors, ModelTensors
    from .rotary import rotary_tables

    gen = torch.Generator(device=generator_device).manual_seed(seed)

    def draw(*shape, dtype=torch.bfloat16, scale=std):
        x = torch.randn(*shape, generator=gen, device=generator_device, dtype=torch.float32) * scale
        return x.to(dtype).to(device).contiguous()

    C, H = hidden, hidden // HEAD_DIM
    wte = draw(vocab, C, dtype=torch.float32)
    lm_head = draw(vocab, C)
    lys = []
    for i in range(layers):
        ly = LayerTensors(qkv=draw(3 * C, C), o=draw(C, C), fc=draw(ffn, C), proj=draw(C, ffn),
                          q_norm=(1.0 + draw(HEAD_DIM, dtype=torch.float32, scale=0.1)),
                          k_norm=(1.0 + draw(HEAD_DIM, dtype=torch.float32, scale=0.1)))
        if i in ve_layers:
            ly.ve = draw(vocab, C)
            ly.ve_gate = draw(H, C, dtype=torch.float32)
        lys.append(ly)
    cos, sin = rotary_tables(max_length, theta, device)
    return ModelTensors(wte=wte, cos=cos, sin=sin, lm_head=lm_head, layers=lys,
                        resid_lambdas=[resid_lambda] * layers, x0_lambdas=[x0_lambda] * layers,
                        windows=list(windows) if windows is not None else [max_length] * layers, softcap=softcap)


def prompt_tokens(batch: int, prompt: int, vocab: int, seed: int = 0, bos: int = 0) -> torch.Tensor:
    """Random prompts [batch, prompt] int64: BOS, then tokens in [1, vocab)."""
    gen = torch.Generator().manual_seed(seed)
    ids = torch.randint(1, vocab, (batch, prompt), generator=gen)
    ids[:, 0] = bos
    return ids
