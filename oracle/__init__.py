"""CPU oracle for the fp8 KV-cache decode path — TEST INFRASTRUCTURE ONLY.

A plain-numpy restatement of the reference's math for this path, used as the checker by
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`, and by nothing
else. The product path (`nanochat_amd`) never imports it and has no CPU fallback.

Modules and the reference text each follows:

- `numerics`  bf16 round-to-nearest-even and the OCP e4m3fn encoder/decoder (integer arithmetic).
- `rope`      rotary tables (model/modeling.py:169-176; inference/modeling_nanochat.py:29-34) and the
              fused QK-norm + -theta rotation (model/kernels/qk_row.cuh:19-51;
              inference/modeling_nanochat.py:37-45) with an explicit fp32 operation order.
- `quant`     per-token, per-KV-head absmax fp8 quantization (the build's spec; the reference caches
              bf16 at model/kernels/decode.cu:562-564 and has no quantizer).
- `layout`    the paged cache's physical byte layout, the block-table scatter and the gather.
- `attention` decode attention (model/kernels/decode.cu:567-675 semantics: keys [max(p-window,0), p])
              and chunked prefill (decode.cu:859-863: every chunk row appended first, then causal
              attention), both in float64 over the dequantized cache.

Pinning (what checks each function beyond restating it) is listed in each module's docstring.
"""
