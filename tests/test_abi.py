"""The C ABI without a GPU: the library loads, exports every function include/nanochat_amd.h declares, and
rejects null pointers and bad sizes with status codes before any device call."""
import ctypes
import re
from pathlib import Path

import pytest

from nanochat_amd.native import SIGNATURES

HEADER = Path(__file__).resolve().parent.parent / "include" / "nanochat_amd.h"
DUMMY = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails its host checks first


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*;", text))


def test_header_and_binding_agree():
    assert declared() == set(SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.nc_abi_version() == 2


def test_status_strings(lib):
    assert lib.nc_status_string(0) == b"ok"
    assert b"NULL" in lib.nc_status_string(-1)
    assert b"workspace" in lib.nc_status_string(-3)


def test_null_pointers_rejected(lib):
    assert lib.nc_kv_append_fp8(None, None, 512, 1, 1, 4, None, None, None, 1, None, None, None, 1, None) == -1
    assert lib.nc_decode_attn_fp8(None, *([DUMMY] * 4), 1, 1, DUMMY, 16, 1, 4, 4, -1, 0.1, 0, DUMMY, None, 0,
                                  None) == -1
    assert lib.nc_prefill_attn_fp8(DUMMY, *([DUMMY] * 4), 1, 1, None, 1, 1, 4, 4, -1, 0.1, DUMMY, None) == -1


@pytest.mark.parametrize("B,Hq,Hkv,max_seq,max_pages", [
    (0, 4, 4, 16, 1), (1, 6, 4, 16, 1), (1, 34, 2, 16, 1), (1, 4, 4, 17, 1), (1, 4, 4, 0, 1), (1, 4, 0, 16, 1)])
def test_bad_decode_shapes_rejected(lib, B, Hq, Hkv, max_seq, max_pages):
    assert lib.nc_decode_attn_fp8(*([DUMMY] * 5), max_pages, 4, DUMMY, max_seq, B, Hq, Hkv, -1, 0.1, 0, DUMMY,
                                  DUMMY, 1 << 30, None) == -2


def test_small_workspace_rejected(lib):
    need = lib.nc_decode_workspace_bytes(64, 16, 4, 8193, -1, 0)
    assert need > 0
    assert lib.nc_decode_attn_fp8(*([DUMMY] * 5), 513, 64 * 513, DUMMY, 8193, 64, 16, 4, -1, 0.1, 0, DUMMY, DUMMY,
                                  need - 1, None) == -3


def expected_workspace(B, Hq, Hkv, max_seq, window, pps):
    """The documented layout: fp32 partials (O [128] + max, sum) for B*Hkv + W slots of G heads, then int32
    meta [B*Hkv][2]; W = one wave per 16 pages of the largest possible page list (at most 4096), or per `pps`."""
    unit_pages = -(-max_seq // 16)
    if window >= 0:
        unit_pages = min(unit_pages, window // 16 + 2)
    pages = B * Hkv * unit_pages
    w = -(-pages // 16)
    if pps > 0:
        w = min(w, -(-pages // pps))
    w = max(1, min(w, 4096))
    return (B * Hkv + w) * (Hq // Hkv) * 130 * 4 + B * Hkv * 2 * 4


@pytest.mark.parametrize("args", [(1, 4, 4, 16, -1, 64), (8, 16, 4, 8193, -1, 0), (8, 16, 4, 8193, 512, 0),
                                  (64, 16, 4, 8193, -1, 0), (64, 16, 4, 8193, -1, 258), (32, 10, 10, 4097, -1, 0)])
def test_workspace_sizes(lib, args):
    assert lib.nc_decode_workspace_bytes(*args) == expected_workspace(*args)


def test_workspace_window_and_bad_sizes(lib):
    assert lib.nc_decode_workspace_bytes(8, 16, 4, 8193, 512, 0) < lib.nc_decode_workspace_bytes(8, 16, 4, 8193, -1, 0)
    assert lib.nc_decode_workspace_bytes(0, 16, 4, 8193, -1, 0) == 0
    assert lib.nc_decode_workspace_bytes(8, 6, 4, 8193, -1, 0) == 0


def test_bad_append_shapes_rejected(lib):
    assert lib.nc_kv_append_fp8(*([DUMMY] * 2), 100, 1, 1, 4, *([DUMMY] * 3), 1, *([DUMMY] * 3), 1, None) == -2
    assert lib.nc_qk_norm_rope_append_fp8(DUMMY, 128 * 5, 1, 1, 4, 1, *([DUMMY] * 6), 0, DUMMY, DUMMY, 1,
                                          *([DUMMY] * 3), 1, None) == -2


def test_qkp_forward_reports_errors(lib):
    lib.qkp_forward(None, *([DUMMY] * 7), 6, 6, 1, None)
    assert lib.nc_last_error() == -1
    lib.qkp_forward(*([DUMMY] * 8), 7, 6, 1, None)
    assert lib.nc_last_error() == -2
