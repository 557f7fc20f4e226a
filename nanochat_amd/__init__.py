"""nanochat_amd: the MI355X (gfx950) fp8 KV-cache decode path of nanochat, as hand-written HIP kernels
behind a C ABI (include/nanochat_amd.h), with the reference's Python operator surface on top.

- `qk_prologue.qk_forward`  drop-in for the reference's model/ops/qk_prologue.py:13-21
- `kv_cache.PagedKVCache`   the paged fp8 cache (pages, scales) and its block tables
- `attention`               fused QK-norm/RoPE + fp8 append, split-K decode, MFMA chunked prefill
- `rotary`                  the fp64 -> fp32 rotary tables (reference model/modeling.py:169-176)
- `native`                  the hipcc build and ctypes binding
"""
from .config import HEAD_DIM, PAGE_SIZE

__all__ = ["HEAD_DIM", "PAGE_SIZE"]
