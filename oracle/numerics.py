"""bf16 and fp8 (OCP e4m3fn) scalar formats in integer arithmetic — test infrastructure only.

Pinned by tests/test_oracle_numerics.py:
- `bf16_round` against torch's CPU `.to(torch.bfloat16)` over every fp32 exponent and random bits;
- `e4m3_encode` against torch's CPU `.to(torch.float8_e4m3fn)` (a library RNE routine) over every
  bf16 value in [-448, 448] and 2^20 random fp32 values, and against the committed exhaustive table
  tests/golden/e4m3fn_codes.npy; `e4m3_decode` against the closed form (-1)^s 2^(e-7) (1 + m/8)
  (e > 0) and m 2^-9 (e = 0) for all 256 codes.
"""
import numpy as np

FP8_MAX = np.float32(448.0)


def bf16_bits(x):
    """fp32 array -> uint16 bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(bits):
    """uint16 bf16 bit patterns -> fp32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x):
    """fp32 -> nearest-even bf16 value, returned as fp32."""
    return bf16_to_f32(bf16_bits(x))


def e4m3_encode(x):
    """fp32 array, |x| <= 448 and finite -> uint8 e4m3fn codes, round to nearest even.

    Normal range (|x| >= 2^-6): round the fp32 bit pattern to 3 mantissa bits (a carry moves into the
    exponent) and rebias 127 -> 7. Subnormal range: |x| * 2^9 is exact and rounds to an integer
    0..8 (8 is the smallest normal, code 0x08). The sign bit is copied, so -0 and negative values
    that round to zero give 0x80, as torch's cast does.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = np.abs(x)
    au = a.view(np.uint32).astype(np.int64)
    normal = (au + 0x7FFFF + ((au >> 20) & 1)) >> 20
    normal = normal - ((127 - 7) << 3)
    sub = np.rint(a * np.float32(512.0)).astype(np.int64)
    code = np.where(a >= np.float32(2.0 ** -6), normal, sub)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_decode(codes):
    """uint8 e4m3fn codes -> fp32 values (0x7F/0xFF, the NaN codes, are out of contract)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e > 0, np.ldexp(1.0 + m / 8.0, e - 7), np.ldexp(m.astype(np.float64), -9))
    return (s * mag).astype(np.float32)
