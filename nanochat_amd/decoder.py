"""Batched decoding by libnanochat_decode.so: the host side of the reference's NativeDecoder
(inference/decoder.py:122-324) over the dec_* ABI (include/nanochat_decode.h), with the fp8 paged KV cache.

The call sequence is the reference's: dec_create from the weights' device addresses; per request dec_load_prompt
(a stored prompt) or a queued prefill, then dec_set_prompt; per step dec_launch_body, the masks of the constrained
slots (dec_masks, dec_set_active), dec_launch_head, dec_tokens; a lazy BOS that the constraint rejects gives way to
the step's alternative (dec_take_alt).

What differs from the reference's host side: the model is a `ModelTensors` (the decoder's inputs themselves, where
the reference takes a CausalLM and copies its tensors), and a constraint is any object with `mask()` (None, or the
allowed tokens as uint32 words, bit t % 32 of word t // 32) and `push(token)`, optionally `ends()` deciding a lazy
BOS; the tokenizer-bound Reemit and syntax constraints of the reference stay with their tokenizer.
"""
import ctypes
import time
import weakref
from collections.abc import Callable, Iterable, Iterator
from dataclasses import dataclass, field

import numpy as np
import torch

from .config import HEAD_DIM, PAGE_SIZE
from .native import hip_library

GLOBAL_PTRS, LAYER_PTRS = 4, 8   # dec_create's pointer layout (decode.cu:950-953)
MASK_BITS = 64                   # slots per word of dec_set_active's masks


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
    """A continuation of input_ids (BOS and at least one more token) by at most max_new_tokens (>= 1) tokens, within
    the constraint's masks, until stopping_criteria holds (reference decoder.py:28-40). temperature 0: argmax (ties
    to the lowest id); > 0: a softmax(logits / temperature) sample drawn from (seed, generated position) alone;
    top_p < 1: nucleus sampling."""
    input_ids: list[int]
    max_new_tokens: int
    stopping_criteria: Callable[[list[int]], bool] = lambda out: False
    constraint: object | None = None
    temperature: float = 0.0
    top_p: float = 1.0
    seed: int = 0


@dataclass
class Slot:
    """A request in a slot: index, request, start and first-token host times, generated tokens."""
    index: int
    request: Request
    start: float
    first: float | None = None
    out: list[int] = field(default_factory=list)


class PagedDecoder:
    """Decoding of up to `batch` slots by libnanochat_decode.so, slots sized by free device memory (at most
    max_slots). max_length: a slot's cache positions; prompt_store: positions of the device prompt store."""

    @torch.no_grad()
    def __init__(self, model: ModelTensors, *, bos_token_id: int, max_length: int, prompt_store: int,
                 max_slots: int | None = None):
        model.check()
        if max_length > model.cos.size(0):
            raise ValueError(f"max_length {max_length} exceeds the rotary table's {model.cos.size(0)} positions")
        torch.cuda.empty_cache()
        self.lib = lib = hip_library("decode")
        self.model = model  # the decoder reads these tensors in place for its whole life
        L, C = len(model.layers), model.hidden
        self.vocab, self.max_length, self.bos = model.vocab, max_length, bos_token_id
        ptrs = [model.wte.data_ptr(), model.cos.data_ptr(), model.sin.data_ptr(), model.lm_head.data_ptr()]
        for ly in model.layers:
            ptrs += [ly.qkv.data_ptr(), ly.o.data_ptr(), ly.fc.data_ptr(), ly.proj.data_ptr(),
                     0 if ly.ve is None else ly.ve.data_ptr(), 0 if ly.ve_gate is None else ly.ve_gate.data_ptr(),
                     ly.q_norm.data_ptr(), ly.k_norm.data_ptr()]
        ptrs = np.array(ptrs, dtype=np.uint64)
        scal = np.array([v for pair in zip(model.resid_lambdas, model.x0_lambdas) for v in pair] + [model.softcap],
                        dtype=np.float32)
        cfg = np.array([L, C, model.ffn, model.vocab, max_length, prompt_store, bos_token_id], dtype=np.int32)
        window = np.array(model.windows, dtype=np.int32)
        self.stream = torch.cuda.Stream(model.wte.device)
        torch.cuda.synchronize()  # the weights were written on the current stream; the decoder runs on its own
        if max_slots is None:
            self.handle = lib.dec_create(cfg.ctypes.data, ptrs.ctypes.data, scal.ctypes.data, window.ctypes.data,
                                         self.stream.cuda_stream)
        else:
            self.handle = lib.dec_create_slots(cfg.ctypes.data, ptrs.ctypes.data, scal.ctypes.data,
                                               window.ctypes.data, self.stream.cuda_stream, max_slots)
        self._finalizer = weakref.finalize(self, lib.dec_destroy, self.handle)
        self.batch = lib.dec_batch(self.handle)
        self.tokens = np.zeros(2 * self.batch, dtype=np.int32)
        self.masks = np.ctypeslib.as_array(lib.dec_masks(self.handle), shape=(self.batch, self.vocab // 32))
        self.prefill_rows = lib.dec_prefill_rows(self.handle)
        self.store = prompt_store
        self.stored: dict[tuple[int, ...], int] = {}
        self.used = 0
        self.pending: list[tuple[int, list[int]]] = []
        self.timings: dict[int, tuple[float, float, float]] = {}
        word_slots = -(-self.batch // MASK_BITS) * MASK_BITS
        self.flags = np.zeros((2, word_slots), dtype=bool)   # row 0: active slots, row 1: masked slots

    def close(self) -> None:
        """Free the decoder's device and pinned memory now (otherwise when it is collected)."""
        self._finalizer()

    # ---- the ABI, one call each
    def set_active(self) -> None:
        words = np.packbits(self.flags, axis=1, bitorder="little").view("<u8")
        self.lib.dec_set_active(self.handle, np.ascontiguousarray(words).ctypes.data)

    def step(self) -> np.ndarray:
        """One step over the active slots (no constraints): the chosen tokens [B]."""
        self.lib.dec_launch_body(self.handle)
        self.lib.dec_launch_head(self.handle)
        self.lib.dec_tokens(self.handle, self.tokens.ctypes.data)
        return self.tokens[:self.batch]

    def logits(self, rows: int) -> np.ndarray:
        """Test hook: the last head's fp32 logits of slots [0, rows)."""
        out = np.empty((rows, self.vocab), dtype=np.float32)
        self.lib.dec_debug_logits(self.handle, out.ctypes.data, rows)
        return out

    def cache_rows(self, layer: int, b: int, at: int, n: int):
        """Test hook: slot b's (b = -1: the store's) cached rows at [at, at + n) of a layer: K codes, V codes
        [n][H][128] uint8 and scales [n][H][2] fp32."""
        H = self.model.hidden // HEAD_DIM
        k = np.empty((n, H, HEAD_DIM), np.uint8)
        v = np.empty_like(k)
        s = np.empty((n, H, 2), np.float32)
        self.lib.dec_debug_cache(self.handle, layer, b, at, n, k.ctypes.data, v.ctypes.data, s.ctypes.data)
        return k, v, s

    def table(self, b: int) -> np.ndarray:
        """Test hook: slot b's block-table row (own page b * pages + e, or batch * pages + i: store page i)."""
        out = np.empty(-(-self.max_length // PAGE_SIZE), np.int32)
        self.lib.dec_debug_table(self.handle, b, out.ctypes.data)
        return out

    # ---- requests (the reference's NativeDecoder.start / prefill / save / generate)
    def start(self, b: int, index: int, request: Request) -> Slot:
        n = len(request.input_ids) - 1
        if n < 1:
            raise ValueError(f"request {index}: input_ids needs BOS and at least one more token")
        if request.max_new_tokens < 1:
            raise ValueError(f"request {index}: max_new_tokens {request.max_new_tokens} < 1")
        if n + request.max_new_tokens > self.max_length:
            raise ValueError(f"request {index}: {n + 1} prompt and {request.max_new_tokens} new tokens need "
                             f"{n + request.max_new_tokens} positions, max_length {self.max_length}")
        if any(not 0 <= t < self.vocab for t in request.input_ids):
            raise ValueError(f"request {index}: token outside [0, {self.vocab})")
        at = self.stored.get(tuple(request.input_ids))
        if at is None:
            self.pending.append((b, request.input_ids))
        else:
            self.lib.dec_load_prompt(self.handle, b, 0, at, n)
        self.lib.dec_set_prompt(self.handle, b, request.input_ids[-1], n, request.temperature, request.top_p,
                                request.seed)
        return Slot(index, request, start=time.perf_counter())

    def prefill(self) -> None:
        """The pending prompts but their last tokens, prefill_rows rows a call, then each kept in the store."""
        if not self.pending:
            return
        rows = np.concatenate([np.array([ids[:-1], range(len(ids) - 1), [b] * (len(ids) - 1)], dtype=np.int32)
                               for b, ids in self.pending], axis=1)
        for i in range(0, rows.shape[1], self.prefill_rows):
            chunk = np.ascontiguousarray(rows[:, i:i + self.prefill_rows])
            self.lib.dec_prefill(self.handle, chunk.shape[1], chunk.ctypes.data)
        for b, ids in self.pending:
            self.save(b, ids)
        self.pending = []

    def save(self, b: int, input_ids: list[int]) -> None:
        """Keep slot b's prompt K and V in the store's next free positions, unless stored or full (never evicted).
        Each prompt starts on a page boundary of the store, so dec_load_prompt shares its whole pages with the slots
        that load it instead of copying them (the reference packs prompts back to back, decoder.py:226-232)."""
        key, n = tuple(input_ids), len(input_ids) - 1
        if key in self.stored or self.used + n > self.store:
            return
        self.lib.dec_save_prompt(self.handle, b, 0, self.used, n)
        self.stored[key] = self.used
        self.used = -(-(self.used + n) // PAGE_SIZE) * PAGE_SIZE

    @torch.no_grad()
    def generate(self, requests: Iterable[Request]) -> Iterator[tuple[int, list[int]]]:
        """Continuations of requests, consumed lazily; yields (request index, generated ids) in completion order.
        Raises ValueError when a constraint allows no token. Sets timings {index: (start, first, end)}."""
        lib, B = self.lib, self.batch
        self.timings = {}
        queue, slots = enumerate(requests), [None] * B
        self.flags[:] = False
        stopping: list[int] = []

        def fill(b: int) -> None:
            for i, request in queue:
                slots[b] = self.start(b, i, request)
                self.flags[0, b] = True
                return
            slots[b] = None
            self.flags[0, b] = False

        for b in range(B):
            fill(b)
        self.set_active()
        while self.flags[0].any():
            self.prefill()
            active = [b for b, s in enumerate(slots) if s is not None]
            lib.dec_launch_body(self.handle)
            finished = sorted(b for b in stopping if slots[b].request.stopping_criteria(slots[b].out))
            stopping = []
            for b in active:
                if b in finished or slots[b].request.constraint is None:
                    continue
                mask = slots[b].request.constraint.mask()
                if mask is None:
                    continue
                self.masks[b] = mask
                self.flags[1, b] = True
                if not self.masks[b].any():
                    raise ValueError(f"request {slots[b].index}: its constraint allows no token at position "
                                     f"{len(slots[b].out)}")
            self.set_active()
            self.flags[1] = False
            lib.dec_launch_head(self.handle)
            lib.dec_tokens(self.handle, self.tokens.ctypes.data)
            for b in active:  # a lazy BOS the constraint rejects gives way to the alternative (decoder.py:234-248)
                c = slots[b].request.constraint
                if b in finished or self.tokens[b] != self.bos or c is None or not hasattr(c, "ends") or c.ends():
                    continue
                if self.tokens[B + b] < 0:
                    raise ValueError(f"request {slots[b].index}: its constraint allows no token at position "
                                     f"{len(slots[b].out)}")
                self.tokens[b] = self.tokens[B + b]
                lib.dec_take_alt(self.handle, b)
            now = time.perf_counter()
            for b, s in enumerate(slots):
                if s is None or b in finished:
                    continue
                token = int(self.tokens[b])
                if token == self.bos:
                    finished.append(b)
                    continue
                if not s.out:
                    s.first = now
                s.out.append(token)
                if s.request.constraint is not None:
                    s.request.constraint.push(token)
                if len(s.out) == s.request.max_new_tokens:
                    finished.append(b)
                else:
                    stopping.append(b)
            if finished:
                for b in finished:
                    done = slots[b]
                    fill(b)
                    self.timings[done.index] = (done.start, now if done.first is None else done.first, now)
                    yield done.index, done.out
                self.set_active()
