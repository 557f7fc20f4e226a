"""Per-token, per-KV-head absmax fp8 (e4m3fn) quantization — test infrastructure only.

The reference caches K and V as bf16 (model/kernels/decode.cu:562-564) and has no quantizer, so this
module is the build's specification of the fp8 cache contents:

    amax  = max_d |x_d|                          (x: one token's 128 bf16 values of one KV head)
    scale = amax / 448  (fp32 IEEE division);    scale = 1 when amax == 0
    code  = e4m3fn_rne(clamp(x / scale, -448, 448))   (fp32 IEEE division per element)
    value = fp32(code) * scale

Pinned by tests/test_oracle_quant.py: the encoder against torch's cast (see numerics), the amax
element mapping to +-448 (0x7E / 0xFE), the half-ulp error bound |code*scale - x| <= 2^-4 |x| for
normal codes and <= 2^-10 scale for subnormal ones, the all-zero row, and the config-1 golden
fixture's committed codes and scales.
"""
import numpy as np

from .numerics import FP8_MAX, e4m3_decode, e4m3_encode


def quantize_rows(x):
    """x (..., 128) fp32 holding bf16 values -> (codes uint8 (..., 128), scale fp32 (...))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=-1)
    scale = np.where(amax > 0, amax / FP8_MAX, np.float32(1.0)).astype(np.float32)
    y = (x / scale[..., None]).astype(np.float32)
    y = np.clip(y, -FP8_MAX, FP8_MAX)
    return e4m3_encode(y), scale


def dequantize_rows(codes, scale):
    """codes uint8 (..., 128), scale fp32 (...) -> fp32 values fp32(code) * scale."""
    return (e4m3_decode(codes) * np.asarray(scale, dtype=np.float32)[..., None]).astype(np.float32)
