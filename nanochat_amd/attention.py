"""Host wrappers of the fp8 KV path's HIP entry points (include/nanochat_amd.h).

- qk_norm_rope_append: the fused append of a decode or prefill step — the reference's attn_prologue
  q/k math (model/kernels/decode.cu:478-507, qk_row.cuh:26-51) plus the fp8 store that replaces
  k_prologue's bf16 store (decode.cu:551-565).
- decode_attention: split-K flash-decode over the paged cache, replacing k_attn (decode.cu:567-675).
- decode_step: the two in one launch (k_prologue + k_attn of a decode step, decode.cu:551-675, 861-863), with the
  same bits as qk_norm_rope_append followed by decode_attention.
- prefill_attention: MFMA chunked prefill, replacing the prefill rows of dec_prefill
  (decode.cu:1041-1051, append-then-attend order 859-863).

Every function launches on the current torch stream and requires device tensors: there is no CPU path.
"""
import functools
from collections import OrderedDict

import torch

from .config import HEAD_DIM
from .kv_cache import PagedKVCache, _require
from .native import check, hip_library, pointer, stream


def qk_norm_rope_append(qkv: torch.Tensor, num_q_heads: int, cache: PagedKVCache, block_table: torch.Tensor,
                        start_pos: torch.Tensor, q_gain: torch.Tensor, k_gain: torch.Tensor, cos: torch.Tensor,
                        sin: torch.Tensor, num_new: torch.Tensor | None = None,
                        q_out: torch.Tensor | None = None) -> torch.Tensor:
    """qkv bf16 [B, T, (Hq + 2 Hkv) * 128] (rows contiguous; token stride = qkv.stride(1)) -> q bf16
    [B, T, Hq, 128] normed and rotated; k (normed, rotated) and v are quantized into `cache` at positions
    start_pos[b] + t."""
    B, T, W = qkv.shape
    Hkv = cache.num_kv_heads
    if W != (num_q_heads + 2 * Hkv) * HEAD_DIM:
        raise ValueError(f"qkv width {W} != (Hq + 2 Hkv) * {HEAD_DIM} = {(num_q_heads + 2 * Hkv) * HEAD_DIM}")
    if qkv.dtype != torch.bfloat16 or not qkv.is_cuda or qkv.stride(2) != 1 or qkv.stride(0) != T * qkv.stride(1):
        raise ValueError("qkv must be a bf16 device tensor with contiguous rows and a uniform token stride")
    for name, t in (("q_gain", q_gain), ("k_gain", k_gain), ("cos", cos), ("sin", sin)):
        _require(t, name, torch.float32)
    if cos.shape != sin.shape or cos.dim() != 2 or cos.size(1) != HEAD_DIM // 2:
        raise ValueError("cos, sin must be [positions, 64]")
    _require(start_pos, "start_pos", torch.int32)
    if num_new is not None:
        _require(num_new, "num_new", torch.int32)
    cache.check_table(block_table)
    if q_out is None:
        q_out = torch.empty(B, T, num_q_heads, HEAD_DIM, dtype=torch.bfloat16, device=qkv.device)
    _require(q_out, "q_out", torch.bfloat16)
    if q_out.shape != (B, T, num_q_heads, HEAD_DIM):
        raise ValueError(f"q_out must be [{B}, {T}, {num_q_heads}, {HEAD_DIM}]")
    check(hip_library().nc_qk_norm_rope_append_fp8(
        pointer(qkv), qkv.stride(1), B, T, num_q_heads, Hkv, pointer(start_pos),
        pointer(num_new) if num_new is not None else None, pointer(q_gain), pointer(k_gain), pointer(cos),
        pointer(sin), cos.size(0), pointer(q_out), pointer(block_table), block_table.size(1),
        pointer(cache.k_pages), pointer(cache.v_pages), pointer(cache.kv_scale), cache.num_pages, stream()))
    return q_out


_WORKSPACES: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
_WORKSPACE_STREAMS = 8


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A decode workspace of at least nbytes for this device and its current stream, kept for reuse. It starts
    zero-filled (its arrival counts must be zero before the first call; every call leaves them zero). Keyed by
    stream, so calls on two streams never share partials or counts. At most _WORKSPACE_STREAMS (device, stream)
    entries are kept, the least recently used dropped first; a caller that cycles through more streams than that, or
    creates streams per request, should pass a workspace of its own. A dropped or outgrown workspace goes back to the
    caching allocator's pool of the stream it was allocated on, and that pool keeps the block until the cache is
    emptied (torch.cuda.empty_cache). A stream whose handle is reused after the stream is destroyed picks up the old
    entry, which is safe: its counts are zero whenever no call is in flight."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.pop(key, None)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    _WORKSPACES[key] = ws
    while len(_WORKSPACES) > _WORKSPACE_STREAMS:
        _WORKSPACES.popitem(last=False)
    return ws


@functools.lru_cache(maxsize=256)
def decode_workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, max_seq_len: int,
                           window: int = -1) -> int:
    """nc_decode_workspace_bytes (0: an unsupported shape), kept per shape: a decode step asks for it every call."""
    return hip_library().nc_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, max_seq_len, window)


def decode_attention(q: torch.Tensor, cache: PagedKVCache, block_table: torch.Tensor, seq_lens: torch.Tensor,
                     max_seq_len: int, window: int = -1, sm_scale: float | None = None, workers: int = 0,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """q bf16 [B, Hq, 128] (the current token's, already appended) -> out bf16 [B, Hq, 128].

    Sequence b attends its keys [max(p - window, 0), p], p = seq_lens[b] - 1; max_seq_len bounds seq_lens (a longer
    sequence's output is NaN). workers caps the waves taking the work items (0: every wave slot of the device); it
    changes no output bit, and neither does anything about the other sequences of the call. A workspace passed in
    must have been zero-filled before its first use (torch.zeros) and only used by these calls since."""
    _require(q, "q", torch.bfloat16)
    B, Hq, D = q.shape
    if D != HEAD_DIM:
        raise ValueError(f"q must be [B, Hq, {HEAD_DIM}]")
    _require(seq_lens, "seq_lens", torch.int32)
    if seq_lens.numel() < B:
        raise ValueError(f"seq_lens holds {seq_lens.numel()} entries for {B} sequences")
    cache.check_table(block_table)
    if block_table.size(0) < B:
        raise ValueError(f"block_table has {block_table.size(0)} rows for {B} sequences")
    if sm_scale is None:
        sm_scale = HEAD_DIM ** -0.5
    if out is None:
        out = torch.empty_like(q)
    _require(out, "out", torch.bfloat16)
    if out.numel() != q.numel():
        raise ValueError(f"out must hold [{B}, {Hq}, {HEAD_DIM}]")
    lib = hip_library()
    need = decode_workspace_bytes(B, Hq, cache.num_kv_heads, max_seq_len, window)
    if need == 0:
        raise ValueError(f"unsupported decode shape: B={B}, Hq={Hq}, Hkv={cache.num_kv_heads}")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = _workspace(q.device, need)
    check(lib.nc_decode_attn_fp8(
        pointer(q), pointer(cache.k_pages), pointer(cache.v_pages), pointer(cache.kv_scale),
        pointer(block_table), block_table.size(1), cache.num_pages, pointer(seq_lens), max_seq_len, B, Hq,
        cache.num_kv_heads, window, sm_scale, workers, pointer(out),
        pointer(workspace), workspace.numel() * workspace.element_size(), stream()))
    return out


def decode_step(qkv: torch.Tensor, num_q_heads: int, cache: PagedKVCache, block_table: torch.Tensor,
                seq_lens: torch.Tensor, q_gain: torch.Tensor, k_gain: torch.Tensor, cos: torch.Tensor,
                sin: torch.Tensor, max_seq_len: int, window: int = -1, sm_scale: float | None = None,
                workers: int = 0, q_out: torch.Tensor | None = None, ve: tuple | None = None,
                out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One decode step in one launch: qkv bf16 [B, (Hq + 2 Hkv) * 128] (or [B, 1, ...]) holds each sequence's token
    at position seq_lens[b] - 1; its q, k are normed and rotated, k and v quantized into `cache`, and q attends as in
    decode_attention -> out bf16 [B, Hq, 128]. The same bits as qk_norm_rope_append (start_pos = seq_lens - 1)
    followed by decode_attention. q_out (bf16 [B, Hq, 128]) receives the rotated queries when given. ve: None or
    (h bf16 [B, C], table bf16 [vocab, C], gate fp32 [Hkv, C], tokens int32 [B]) for value embeddings; a token
    outside [0, vocab) mixes nothing. The page receiving a sequence's token must not be in another sequence's row of
    block_table."""
    if qkv.dim() == 3:
        qkv = qkv.view(qkv.size(0), qkv.size(2)) if qkv.size(1) == 1 else qkv
    if qkv.dim() != 2:
        raise ValueError("qkv must be [B, (Hq + 2 Hkv) * 128] or [B, 1, (Hq + 2 Hkv) * 128]")
    B, W = qkv.shape
    Hkv = cache.num_kv_heads
    if W != (num_q_heads + 2 * Hkv) * HEAD_DIM:
        raise ValueError(f"qkv width {W} != (Hq + 2 Hkv) * {HEAD_DIM} = {(num_q_heads + 2 * Hkv) * HEAD_DIM}")
    if qkv.dtype != torch.bfloat16 or not qkv.is_cuda or qkv.stride(1) != 1:
        raise ValueError("qkv must be a bf16 device tensor with contiguous rows")
    for name, t in (("q_gain", q_gain), ("k_gain", k_gain), ("cos", cos), ("sin", sin)):
        _require(t, name, torch.float32)
    if cos.shape != sin.shape or cos.dim() != 2 or cos.size(1) != HEAD_DIM // 2:
        raise ValueError("cos, sin must be [positions, 64]")
    _require(seq_lens, "seq_lens", torch.int32)
    if seq_lens.numel() < B:
        raise ValueError(f"seq_lens holds {seq_lens.numel()} entries for {B} sequences")
    cache.check_table(block_table)
    if block_table.size(0) < B:
        raise ValueError(f"block_table has {block_table.size(0)} rows for {B} sequences")
    if sm_scale is None:
        sm_scale = HEAD_DIM ** -0.5
    if out is None:
        out = torch.empty(B, num_q_heads, HEAD_DIM, dtype=torch.bfloat16, device=qkv.device)
    _require(out, "out", torch.bfloat16)
    if out.numel() != B * num_q_heads * HEAD_DIM:
        raise ValueError(f"out must hold [{B}, {num_q_heads}, {HEAD_DIM}]")
    if q_out is not None:
        _require(q_out, "q_out", torch.bfloat16)
        if q_out.numel() != B * num_q_heads * HEAD_DIM:
            raise ValueError(f"q_out must hold [{B}, {num_q_heads}, {HEAD_DIM}]")
    ve_h = ve_table = ve_gate = ve_tokens = None
    C = rows = 0
    if ve is not None:
        ve_h, ve_table, ve_gate, ve_tokens = ve
        _require(ve_h, "ve h", torch.bfloat16)
        _require(ve_table, "ve table", torch.bfloat16)
        _require(ve_gate, "ve gate", torch.float32)
        _require(ve_tokens, "ve tokens", torch.int32)
        C = ve_h.size(-1)
        rows = ve_table.size(0)
        if ve_h.dim() != 2 or ve_h.size(0) < B:
            raise ValueError(f"ve h must be [>= {B}, C]")
        if ve_table.dim() != 2 or ve_table.size(1) != C:
            raise ValueError(f"ve table must be [vocab, {C}]")
        if tuple(ve_gate.shape) != (Hkv, C):
            raise ValueError(f"ve gate must be [{Hkv}, {C}]")
        if ve_tokens.numel() < B:
            raise ValueError(f"ve tokens holds {ve_tokens.numel()} entries for {B} sequences")
    lib = hip_library()
    need = decode_workspace_bytes(B, num_q_heads, Hkv, max_seq_len, window)
    if need == 0:
        raise ValueError(f"unsupported decode shape: B={B}, Hq={num_q_heads}, Hkv={Hkv}")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = _workspace(qkv.device, need)
    check(lib.nc_decode_step_fp8(
        pointer(qkv), qkv.stride(0), B, num_q_heads, Hkv, pointer(seq_lens), pointer(q_gain), pointer(k_gain),
        pointer(cos), pointer(sin), cos.size(0), pointer(q_out) if q_out is not None else None,
        pointer(ve_h) if ve is not None else None, pointer(ve_table) if ve is not None else None,
        pointer(ve_gate) if ve is not None else None, pointer(ve_tokens) if ve is not None else None, C, rows,
        pointer(block_table), block_table.size(1), pointer(cache.k_pages), pointer(cache.v_pages),
        pointer(cache.kv_scale), cache.num_pages, max_seq_len, window, sm_scale, workers, pointer(out),
        pointer(workspace), workspace.numel() * workspace.element_size(), stream()))
    return out


def prefill_attention(q: torch.Tensor, cache: PagedKVCache, block_table: torch.Tensor, start_pos: torch.Tensor,
                      window: int = -1, sm_scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """q bf16 [B, T, Hq, 128] of a chunk already appended at positions start_pos[b] + t -> out bf16 like q."""
    _require(q, "q", torch.bfloat16)
    B, T, Hq, D = q.shape
    if D != HEAD_DIM:
        raise ValueError(f"q must be [B, T, Hq, {HEAD_DIM}]")
    _require(start_pos, "start_pos", torch.int32)
    cache.check_table(block_table)
    if sm_scale is None:
        sm_scale = HEAD_DIM ** -0.5
    if out is None:
        out = torch.empty_like(q)
    _require(out, "out", torch.bfloat16)
    check(hip_library().nc_prefill_attn_fp8(
        pointer(q), pointer(cache.k_pages), pointer(cache.v_pages), pointer(cache.kv_scale),
        pointer(block_table), block_table.size(1), cache.num_pages, pointer(start_pos), B, T, Hq, cache.num_kv_heads,
        window, sm_scale, pointer(out), stream()))
    return out
