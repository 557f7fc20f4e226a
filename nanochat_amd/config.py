"""Fixed dimensions of the path (reference model/config.py:1-9; the page geometry is the build's)."""

# Attention head width; a compile-time constant of the kernels (reference model/config.py:7)
HEAD_DIM = 128
# Tokens per cache page
PAGE_SIZE = 16
# Bytes of one page of one KV head (fp8 codes)
PAGE_BYTES = PAGE_SIZE * HEAD_DIM
# Largest finite e4m3fn magnitude: the absmax element of a (token, KV head) row maps to it
FP8_MAX = 448.0
# RoPE base of the reference model (model/config.py:9); the BASELINE prefill config uses 1e4
ROPE_THETA = 1_000_000
