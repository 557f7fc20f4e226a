"""Host driver of libnanochat_decode.so (include/nanochat_decode.h) for this repository's tests, smoke check and
benchmark: the fp8 paged-cache decoder behind the reference's dec_* ABI (model/kernels/decode.cu:904-1131).

The reference's own host class, NativeDecoder (inference/decoder.py:123-324), binds the same library unchanged through
`hip_library("decode")` with the argtypes of `nanochat_amd/native.py`; this module is not a copy of it. It has two
layers:

- `DecoderRuntime` holds one decoder handle and exposes the ABI with no scheduling policy: put a prompt in a slot
  (shared from the prompt store when stored, else queued), run the queued prefill, choose the active and masked slots,
  run a step, read the choices; plus the test hooks (logits, cache rows, block tables).
- `serve` is a minimal scheduler over it: requests fill free slots in order, every step decodes all live slots, and a
  request ends on its token budget, its stopping test or BOS.

The model is a `ModelTensors` (the decoder's inputs themselves). A constraint is any object with `mask()` (None, or the
allowed tokens as uint32 words, bit t % 32 of word t // 32) and `push(token)`, optionally `ends()` deciding whether a
chosen BOS may end the request (if not, the step's best other token is taken instead).
"""
import time
import weakref
from collections import deque
from collections.abc import Callable, Iterable, Iterator, Sequence
from dataclasses import dataclass, field

import numpy as np
import torch

from .config import HEAD_DIM, PAGE_SIZE
from .native import hip_library

GLOBAL_PTRS, LAYER_PTRS = 4, 8   # dec_create's pointer layout (decode.cu:950-953)
SLOTS_PER_WORD = 64              # dec_set_active's slot masks are uint64 words


@dataclass
class LayerTensors:
    """One layer's decoder inputs (device): bf16 GEMM weights [out][in], fp32 q/k norm gains [128], and, on value-
    embedding layers, the bf16 table [vocab][C] and its fp32 gate [H][C]."""
    qkv: torch.Tensor
    o: torch.Tensor
    fc: torch.Tensor
    proj: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    ve: torch.Tensor | None = None
    ve_gate: torch.Tensor | None = None


@dataclass
class ModelTensors:
    """A model as dec_create reads it (decode.cu:950-953; decoder.py:155-171): fp32 embedding [vocab][C], fp32
    rotary tables [>= max_length][64], bf16 lm_head [vocab][C], the layers, per-layer (resid, x0) lambdas and
    windows (keys before a query), and the logit cap."""
    wte: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor
    lm_head: torch.Tensor
    layers: list[LayerTensors]
    resid_lambdas: list[float]
    x0_lambdas: list[float]
    windows: list[int]
    softcap: float = 15.0

    @property
    def hidden(self) -> int:
        return self.wte.size(1)

    @property
    def vocab(self) -> int:
        return self.wte.size(0)

    @property
    def ffn(self) -> int:
        return self.layers[0].fc.size(0)

    def check(self) -> None:
        C, V, L = self.hidden, self.vocab, len(self.layers)
        if C % HEAD_DIM or V % 32:
            raise ValueError(f"hidden {C} must be a multiple of {HEAD_DIM} and vocab {V} of 32")
        if not (len(self.resid_lambdas) == len(self.x0_lambdas) == len(self.windows) == L):
            raise ValueError("one resid lambda, x0 lambda and window per layer")
        F = self.ffn
        expect = [(self.wte, (V, C), torch.float32), (self.lm_head, (V, C), torch.bfloat16),
                  (self.cos, None, torch.float32), (self.sin, None, torch.float32)]
        for ly in self.layers:
            expect += [(ly.qkv, (3 * C, C), torch.bfloat16), (ly.o, (C, C), torch.bfloat16),
                       (ly.fc, (F, C), torch.bfloat16), (ly.proj, (C, F), torch.bfloat16),
                       (ly.q_norm, (HEAD_DIM,), torch.float32), (ly.k_norm, (HEAD_DIM,), torch.float32)]
            if (ly.ve is None) != (ly.ve_gate is None):
                raise ValueError("a value-embedding table needs its gate")
            if ly.ve is not None:
                expect += [(ly.ve, (V, C), torch.bfloat16), (ly.ve_gate, (C // HEAD_DIM, C), torch.float32)]
        for t, shape, dtype in expect:
            if not t.is_cuda or t.dtype != dtype or not t.is_contiguous() or (shape and tuple(t.shape) != shape):
                raise ValueError(f"expected a contiguous {dtype} device tensor of shape {shape}, got "
                                 f"{t.dtype} {tuple(t.shape)} on {t.device}")


@dataclass(frozen=True, kw_only=True)
class Request:
    """What to decode (the fields of the reference's Request, inference/decoder.py:28-40). input_ids starts with BOS
    and holds at least one more token; at most max_new_tokens (>= 1) tokens follow. temperature 0 picks the largest
    logit (lowest id on ties); T > 0 samples softmax(capped logits / T) with noise drawn from (seed, generated
    position), within the top_p nucleus when top_p < 1. stopping_criteria sees the tokens generated so far."""
    input_ids: list[int]
    max_new_tokens: int
    stopping_criteria: Callable[[list[int]], bool] = lambda out: False
    constraint: object | None = None
    temperature: float = 0.0
    top_p: float = 1.0
    seed: int = 0


class DecoderRuntime:
    """One libnanochat_decode.so decoder with up to `max_slots` slots (fewer when device memory runs short).

    max_length: cache positions per slot; prompt_store: positions of the device prompt store, where every prefilled
    prompt is kept (page-aligned, never evicted) so that a later slot given the same prompt shares its pages.
    pool_pages: the KV page pool the slots draw from (16 positions a page); by default every slot can reach
    max_length, a smaller pool lets more slots run sequences shorter than that (serve admits requests by it)."""

    @torch.no_grad()
    def __init__(self, model: ModelTensors, *, bos_token_id: int, max_length: int, prompt_store: int = 0,
                 max_slots: int | None = None, pool_pages: int | None = None):
        model.check()
        if max_length > model.cos.size(0):
            raise ValueError(f"max_length {max_length} exceeds the rotary table's {model.cos.size(0)} positions")
        self.lib = hip_library("decode")
        self.model = model   # the handle reads these tensors in place until it is destroyed
        self.vocab, self.max_length, self.bos, self.store_size = model.vocab, max_length, bos_token_id, prompt_store
        ptrs = [model.wte, model.cos, model.sin, model.lm_head]
        for ly in model.layers:
            ptrs += [ly.qkv, ly.o, ly.fc, ly.proj, ly.ve, ly.ve_gate, ly.q_norm, ly.k_norm]
        self._ptrs = np.array([0 if t is None else t.data_ptr() for t in ptrs], dtype=np.uint64)
        lambdas = [x for pair in zip(model.resid_lambdas, model.x0_lambdas) for x in pair]
        self._scal = np.array(lambdas + [model.softcap], dtype=np.float32)
        self._cfg = np.array([len(model.layers), model.hidden, model.ffn, model.vocab, max_length, prompt_store,
                              bos_token_id], dtype=np.int32)
        self._window = np.array(model.windows, dtype=np.int32)
        torch.cuda.empty_cache()
        self.stream = torch.cuda.Stream(model.wte.device)
        torch.cuda.synchronize()   # the weights were written on another stream
        args = (self._cfg.ctypes.data, self._ptrs.ctypes.data, self._scal.ctypes.data, self._window.ctypes.data,
                self.stream.cuda_stream)
        if pool_pages is not None:
            self.handle = self.lib.dec_create_pool(*args, 1024 if max_slots is None else max_slots, pool_pages)
        elif max_slots is not None:
            self.handle = self.lib.dec_create_slots(*args, max_slots)
        else:
            self.handle = self.lib.dec_create(*args)
        self._release = weakref.finalize(self, self.lib.dec_destroy, self.handle)
        self.batch = self.lib.dec_batch(self.handle)
        self.rows_per_prefill = self.lib.dec_prefill_rows(self.handle)
        self.masks = np.ctypeslib.as_array(self.lib.dec_masks(self.handle), shape=(self.batch, self.vocab // 32))
        self._out = np.zeros(2 * self.batch, dtype=np.int32)    # dec_tokens: choices, then alternatives
        self.choices, self.alternatives = self._out[:self.batch], self._out[self.batch:]
        self.stored: dict[tuple[int, ...], int] = {}            # prompt -> its first store position
        self.store_used = 0
        self.queued: list[tuple[int, list[int]]] = []           # (slot, prompt) awaiting prefill

    def close(self) -> None:
        """Destroy the decoder now (otherwise when the object is collected)."""
        self._release()

    # --- prompts
    def place(self, slot: int, prompt: Sequence[int], *, temperature: float = 0.0, top_p: float = 1.0,
              seed: int = 0) -> bool:
        """Slot `slot` continues `prompt` (BOS first), decoding from its last token. The positions before that come
        from the prompt store when the same prompt is stored (returns True), else they are queued for `prefill`."""
        prompt = [int(t) for t in prompt]
        n = len(prompt) - 1
        if not 0 <= slot < self.batch:
            raise ValueError(f"slot {slot} outside [0, {self.batch})")
        if n < 1 or n >= self.max_length:
            raise ValueError(f"a prompt of {n + 1} tokens does not fit: BOS, at least one more, under max_length "
                             f"{self.max_length}")
        if min(prompt) < 0 or max(prompt) >= self.vocab:
            raise ValueError(f"prompt token outside [0, {self.vocab})")
        at = self.stored.get(tuple(prompt))
        if at is not None:
            self.lib.dec_load_prompt(self.handle, slot, 0, at, n)
        else:
            self.queued.append((slot, prompt))
        self.lib.dec_set_prompt(self.handle, slot, prompt[-1], n, temperature, top_p, seed)
        return at is not None

    def prefill(self) -> int:
        """Run every queued prompt (all but its last token) through the decoder, rows_per_prefill rows a call, then
        keep each in the store; returns the rows run."""
        if not self.queued:
            return 0
        table = np.concatenate([np.stack([np.array(p[:-1]), np.arange(len(p) - 1), np.full(len(p) - 1, slot)])
                                for slot, p in self.queued], axis=1).astype(np.int32)
        for lo in range(0, table.shape[1], self.rows_per_prefill):
            part = np.ascontiguousarray(table[:, lo:lo + self.rows_per_prefill])
            self.lib.dec_prefill(self.handle, part.shape[1], part.ctypes.data)
        for slot, p in self.queued:
            self._keep(slot, p)
        self.queued = []
        return table.shape[1]

    def _keep(self, slot: int, prompt: list[int]) -> None:
        """Copy the slot's prompt rows into the store at the next page boundary, if new and room is left."""
        key, n = tuple(prompt), len(prompt) - 1
        if key in self.stored or self.store_used + n > self.store_size:
            return
        self.lib.dec_save_prompt(self.handle, slot, 0, self.store_used, n)
        self.stored[key] = self.store_used
        self.store_used += -(-n // PAGE_SIZE) * PAGE_SIZE

    # --- steps
    def activate(self, slots: Iterable[int], masked: Iterable[int] = ()) -> None:
        """The slots the next steps decode, and those whose choice is limited to their row of `masks`."""
        words = -(-self.batch // SLOTS_PER_WORD)
        bits = np.zeros((2, words * SLOTS_PER_WORD), dtype=bool)
        for row, chosen in enumerate((slots, masked)):
            for b in chosen:
                if not 0 <= b < self.batch:
                    raise ValueError(f"slot {b} outside [0, {self.batch})")
                bits[row, b] = True
        packed = np.ascontiguousarray(np.packbits(bits, axis=1, bitorder="little").view("<u8"))
        self.lib.dec_set_active(self.handle, packed.ctypes.data)

    def step(self) -> np.ndarray:
        """One decode step of the active slots; returns the choices [batch] (alternatives in `alternatives`)."""
        self.lib.dec_launch_body(self.handle)
        self.lib.dec_launch_head(self.handle)
        self.lib.dec_tokens(self.handle, self._out.ctypes.data)
        return self.choices

    def release(self, slot: int) -> None:
        """The slot's KV pages return to the pool (its next prompt starts a new sequence anyway)."""
        self.lib.dec_release(self.handle, slot)

    def pages(self) -> tuple[int, int]:
        """(free pages, pool size) of the KV page pool."""
        out = np.zeros(2, dtype=np.int64)
        self.lib.dec_debug_pages(self.handle, out.ctypes.data)
        return int(out[0]), int(out[1])

    def take_alternative(self, slot: int) -> None:
        """Slot's next input becomes its alternative (its best choice other than BOS) instead of its choice."""
        self.lib.dec_take_alt(self.handle, slot)

    # --- test hooks
    def logits(self, rows: int) -> np.ndarray:
        """The last step's fp32 logits of slots [0, rows)."""
        out = np.empty((rows, self.vocab), dtype=np.float32)
        self.lib.dec_debug_logits(self.handle, out.ctypes.data, rows)
        return out

    def cache_rows(self, layer: int, slot: int, at: int, n: int):
        """K codes, V codes [n][H][128] uint8 and scales [n][H][2] fp32 of positions [at, at + n) of a slot (-1: the
        prompt store) in one layer."""
        H = self.model.hidden // HEAD_DIM
        k = np.empty((n, H, HEAD_DIM), np.uint8)
        v = np.empty_like(k)
        s = np.empty((n, H, 2), np.float32)
        self.lib.dec_debug_cache(self.handle, layer, slot, at, n, k.ctypes.data, v.ctypes.data, s.ctypes.data)
        return k, v, s

    def table(self, slot: int) -> np.ndarray:
        """The slot's block-table row: entry e is -1 (no page yet), a pool page of the slot's own (below the pool
        size), or pool size + i for page i of the prompt store (shared)."""
        out = np.empty(-(-self.max_length // PAGE_SIZE), np.int32)
        self.lib.dec_debug_table(self.handle, slot, out.ctypes.data)
        return out


@dataclass
class _Live:
    index: int
    request: Request
    started: float
    first: float | None = None
    out: list[int] = field(default_factory=list)


@torch.no_grad()
def serve(rt: DecoderRuntime, requests: Iterable[Request],
          timings: dict | None = None) -> Iterator[tuple[int, list[int]]]:
    """Decode `requests` on rt's slots; yields (request index, generated tokens) as requests end.

    Requests take free slots in order, while the KV page pool can hold every admitted request at its longest (prompt
    plus max_new_tokens positions); a slot's pages return to the pool when its request ends. Each step: the new
    prompts are prefilled, the constrained slots' masks are written, every live slot decodes one token. A request ends after max_new_tokens tokens, when its stopping test
    holds, or on BOS (not included). A BOS its constraint does not accept (`ends()` false) is replaced by the step's
    alternative. Raises ValueError when a constraint leaves no token. timings, when given, receives
    {index: (start, first token, end)} in time.perf_counter() seconds."""
    todo = deque(enumerate(requests))
    live: dict[int, _Live] = {}
    pool = rt.pages()[1]
    reserved: dict[int, int] = {}   # slot -> pages its request may take at its longest

    def pages_for(req: Request) -> int:
        return -(-(len(req.input_ids) - 1 + req.max_new_tokens) // PAGE_SIZE)

    while todo or live:
        for slot in range(rt.batch):
            if slot not in live and todo:
                index, req = todo[0]
                if req.max_new_tokens < 1 or len(req.input_ids) - 1 + req.max_new_tokens > rt.max_length:
                    raise ValueError(f"request {index}: {len(req.input_ids)} prompt tokens and {req.max_new_tokens} "
                                     f"new ones do not fit max_length {rt.max_length}")
                need = pages_for(req)
                if sum(reserved.values()) + need > pool:
                    if not live:
                        raise ValueError(f"request {index} needs {need} KV pages, the pool holds {pool}")
                    break
                todo.popleft()
                rt.place(slot, req.input_ids, temperature=req.temperature, top_p=req.top_p, seed=req.seed)
                live[slot] = _Live(index, req, time.perf_counter())
                reserved[slot] = need
        rt.prefill()
        masked = []
        for slot, run in live.items():
            mask = run.request.constraint.mask() if run.request.constraint is not None else None
            if mask is None:
                continue
            if not np.any(mask):
                raise ValueError(f"request {run.index}: no token allowed after {len(run.out)} tokens")
            rt.masks[slot] = mask
            masked.append(slot)
        rt.activate(live, masked)
        choices = rt.step()
        now = time.perf_counter()
        ended = []
        for slot, run in live.items():
            token = int(choices[slot])
            c = run.request.constraint
            if token == rt.bos and c is not None and hasattr(c, "ends") and not c.ends():
                token = int(rt.alternatives[slot])
                if token < 0:
                    raise ValueError(f"request {run.index}: no token allowed after {len(run.out)} tokens")
                rt.take_alternative(slot)
            if token == rt.bos:
                ended.append(slot)
                continue
            if run.first is None:
                run.first = now
            run.out.append(token)
            if c is not None:
                c.push(token)
            if len(run.out) >= run.request.max_new_tokens or run.request.stopping_criteria(run.out):
                ended.append(slot)
        for slot in ended:
            run = live.pop(slot)
            del reserved[slot]
            rt.release(slot)
            if timings is not None:
                timings[run.index] = (run.started, now if run.first is None else run.first, now)
            yield run.index, run.out
