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
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)
    return set(re.findall(r"\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*;", text))


def test_header_and_binding_agree():
    assert declared() == set(SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.nc_abi_version() == 4


def test_status_strings(lib):
    assert lib.nc_status_string(0) == b"ok"
    assert b"NULL" in lib.nc_status_string(-1)
    assert b"workspace" in lib.nc_status_string(-3)


def test_read_pages_rejects_bad_arguments(lib):
    assert lib.nc_debug_read_pages(None, 2048, None, 1, 1, DUMMY, None) == -1
    assert lib.nc_debug_read_pages(DUMMY, 2048, None, 1, 1, None, None) == -1
    for size, n, grid in ((2047, 1, 1), (3000, 1, 1), (0, 1, 1), (2048, -1, 1), (2048, 1, 0), (2048, 1, 65536)):
        assert lib.nc_debug_read_pages(DUMMY, size, None, n, grid, DUMMY, None) == -2, (size, n, grid)


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
    need = lib.nc_decode_workspace_bytes(64, 16, 4, 8193, -1)
    assert need > 0
    assert lib.nc_decode_attn_fp8(*([DUMMY] * 5), 513, 64 * 513, DUMMY, 8193, 64, 16, 4, -1, 0.1, 0, DUMMY, DUMMY,
                                  need - 1024, None) == -3


def expected_workspace(B, Hq, Hkv, max_seq, window):
    """The documented layout: fp32 partials (O [128] + max, sum) of G heads for every item a launch can hold below the
    last 1/256 of the workspace, which holds one int32 arrival count per (sequence, KV head); a unit of n pages (n
    capped by the window) touches at most ceil(n / 64) + 1 chunks of 1,024 positions, or, at most 67 pages long and cut
    every 16 pages, ceil(n / 16) + 1 chunks. The smallest such size that is a multiple of 1,024 of the form 256 k, k a
    multiple of 4 with 255 k >= partials and k >= 4 B Hkv."""
    unit_pages = -(-max_seq // 16)
    if window >= 0:
        unit_pages = min(unit_pages, window // 16 + 2)
    items = B * Hkv * max(-(-unit_pages // 64) + 1, -(-min(unit_pages, 67) // 16) + 1)
    partials = items * (Hq // Hkv) * 130 * 4
    k = max(-(-partials // 255), 4 * B * Hkv)
    k = -(-k // 4) * 4
    assert 255 * k >= partials and k >= 4 * B * Hkv
    return 256 * k


@pytest.mark.parametrize("args", [(1, 4, 4, 16, -1), (8, 16, 4, 8193, -1), (8, 16, 4, 8193, 512),
                                  (64, 16, 4, 8193, -1), (64, 16, 4, 8193, 1023), (32, 10, 10, 4097, -1)])
def test_workspace_sizes(lib, args):
    assert lib.nc_decode_workspace_bytes(*args) == expected_workspace(*args)


def test_noalloc_rejects_what_its_scratch_cannot_hold(lib):
    """nc_decode_attn_fp8_noalloc checks its static workspace's size before any device call."""
    scratch = 16 << 20
    assert lib.nc_decode_workspace_bytes(64, 16, 4, 8193, -1) <= scratch
    big = (256, 16, 4, 32768)
    assert lib.nc_decode_workspace_bytes(*big, -1) > scratch
    assert lib.nc_decode_attn_fp8_noalloc(*([DUMMY] * 5), 2048, 4, DUMMY, 32768, *big[:3], -1, 0.1, 0, DUMMY,
                                          None) == -3
    assert lib.nc_decode_attn_fp8_noalloc(None, *([DUMMY] * 4), 1, 1, DUMMY, 16, 1, 4, 4, -1, 0.1, 0, DUMMY,
                                          None) == -1
    assert lib.nc_decode_attn_fp8_noalloc(*([DUMMY] * 5), 1, 4, DUMMY, 17, 1, 4, 4, -1, 0.1, 0, DUMMY, None) == -2


def test_workspace_window_and_bad_sizes(lib):
    assert lib.nc_decode_workspace_bytes(8, 16, 4, 8193, 512) < lib.nc_decode_workspace_bytes(8, 16, 4, 8193, -1)
    assert lib.nc_decode_workspace_bytes(0, 16, 4, 8193, -1) == 0
    assert lib.nc_decode_workspace_bytes(8, 6, 4, 8193, -1) == 0
    assert lib.nc_decode_workspace_bytes(4097, 16, 4, 8193, -1) == 0


def step_args(**over):
    """nc_decode_step_fp8's arguments for B = 2, Hq = 16, Hkv = 4, max_seq_len 100 with dummy pointers; `over`
    replaces any of them by name."""
    args = dict(qkv=DUMMY, token_stride=24 * 128, B=2, Hq=16, Hkv=4, seq_lens=DUMMY, q_gain=DUMMY, k_gain=DUMMY,
                cos=DUMMY, sin=DUMMY, rope_len=100, q_out=None, ve_h=None, ve=None, ve_gate=None, ve_tokens=None, C=0, ve_rows=0,
                block_table=DUMMY, max_pages=7, k_pages=DUMMY, v_pages=DUMMY, kv_scale=DUMMY, num_pages=14,
                max_seq_len=100, window=-1, sm_scale=0.1, workers=0, out=DUMMY, workspace=DUMMY,
                workspace_bytes=1 << 30, stream=None)
    args.update(over)
    return list(args.values())


@pytest.mark.parametrize("over,code", [
    (dict(qkv=None), -1), (dict(cos=None), -1), (dict(workspace=None), -1), (dict(ve=DUMMY), -1),
    (dict(ve=DUMMY, ve_h=DUMMY, ve_gate=DUMMY), -1),
    (dict(rope_len=99), -2), (dict(token_stride=24 * 128 - 1), -2), (dict(Hq=6), -2), (dict(max_pages=6), -2),
    (dict(ve=DUMMY, ve_h=DUMMY, ve_gate=DUMMY, ve_tokens=DUMMY, C=511, ve_rows=10), -2),
    (dict(ve=DUMMY, ve_h=DUMMY, ve_gate=DUMMY, ve_tokens=DUMMY, C=512, ve_rows=0), -2), (dict(workers=-1), -2),
    (dict(workspace_bytes=0), -3)])
def test_decode_step_rejects_bad_arguments(lib, over, code):
    """nc_decode_step_fp8 checks its pointers, shapes (rope tables covering max_seq_len, the qkv row width, the value
    embedding width and table rows) and workspace before any device call."""
    assert lib.nc_decode_step_fp8(*step_args(**over)) == code


def test_bad_append_shapes_rejected(lib):
    assert lib.nc_kv_append_fp8(*([DUMMY] * 2), 100, 1, 1, 4, *([DUMMY] * 3), 1, *([DUMMY] * 3), 1, None) == -2
    assert lib.nc_qk_norm_rope_append_fp8(DUMMY, 128 * 5, 1, 1, 4, 1, *([DUMMY] * 6), 0, DUMMY, DUMMY, 1,
                                          *([DUMMY] * 3), 1, None) == -2


def test_qkp_forward_reports_errors(lib):
    lib.qkp_forward(None, *([DUMMY] * 7), 6, 6, 1, None)
    assert lib.nc_last_error() == -1
    lib.qkp_forward(*([DUMMY] * 8), 7, 6, 1, None)
    assert lib.nc_last_error() == -2


def test_qkp_backward_reports_errors(lib):
    assert lib.qkp_backward_blocks() == 512
    lib.qkp_backward(*([DUMMY] * 10), None, DUMMY, DUMMY, 6, 6, 1, None)
    assert lib.nc_last_error() == -1
    lib.qkp_backward(*([DUMMY] * 13), 7, 6, 1, None)
    assert lib.nc_last_error() == -2
    lib.qkp_backward(*([DUMMY] * 13), 6, 6, 0, None)
    assert lib.nc_last_error() == -2


DECODE_HEADER = HEADER.parent / "nanochat_decode.h"

# the reference's decoder ABI (decode.cu:904-1131): every symbol inference/decoder.py binds
REFERENCE_DEC = {"dec_create", "dec_batch", "dec_set_prompt", "dec_prefill_rows", "dec_prefill", "dec_save_prompt",
                 "dec_load_prompt", "dec_masks", "dec_set_active", "dec_launch_body", "dec_launch_head", "dec_tokens",
                 "dec_take_alt", "dec_destroy"}


def decode_declared():
    text = re.sub(r"/\*.*?\*/", "", DECODE_HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*;", text))


def test_ve_gate_reports_errors(lib):
    """The value-embedding entry points check every argument before a device call."""
    # general entry points: status codes
    assert lib.nc_ve_forward(None, None, 768, None, None, 10, None, None, None, 0, 6, None) == 0   # no rows
    assert lib.nc_ve_forward(None, None, 768, None, None, 10, None, None, None, 4, 6, None) == -1
    assert lib.nc_ve_forward(None, None, 768, None, None, 10, None, None, None, 4, 17, None) == -2   # heads
    assert lib.nc_ve_forward(None, None, 768, None, None, 10, None, None, None, 4, 0, None) == -2
    assert lib.nc_ve_forward(None, None, 700, None, None, 10, None, None, None, 4, 6, None) == -2    # v_stride < C
    assert lib.nc_ve_forward(None, None, 772, None, None, 10, None, None, None, 4, 6, None) == -2    # not x8
    assert lib.nc_ve_forward(None, None, 768, None, None, 0, None, None, None, 4, 6, None) == -2     # vocab
    assert lib.nc_ve_forward(None, None, 768, None, None, 10, None, None, None, -1, 6, None) == -2
    assert lib.nc_ve_backward(None, 768, None, None, None, 10, None, None, None, None, None, 0, 6, None) == 0
    assert lib.nc_ve_backward(None, 768, None, None, None, 10, None, None, None, None, None, 3, 6, None) == -1
    assert lib.nc_ve_backward(None, 100, None, None, None, 10, None, None, None, None, None, 3, 6, None) == -2
    # misaligned operands (fake, never dereferenced addresses)
    p, q, r = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1008), ctypes.c_void_p(0x1004)
    assert lib.nc_ve_forward(q, p, 768, p, p, 10, p, p, p, 4, 6, None) == -2          # n not 16-byte aligned
    assert lib.nc_ve_backward(p, 768, p, r, p, 10, p, p, p, p, p, 4, 6, None) == -2   # order not 8-byte aligned
    # the reference-signature symbols (H = 6): nc_last_error
    lib.ve_forward(None, None, 768, None, None, None, None, None, 5, None)
    assert lib.nc_last_error() == -1
    lib.ve_forward(None, None, 768, None, None, None, None, None, 0, None)
    assert lib.nc_last_error() == 0
    lib.ve_backward(None, 760, None, None, None, None, None, None, None, None, 5, None)
    assert lib.nc_last_error() == -2


def test_flash_attn_reports_errors(lib):
    """Shape, NULL and alignment checks before any device call; nothing to do returns 0 without launching."""
    p, q = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1008)
    fwd = lib.nc_flash_attn_fwd
    assert fwd(None, None, None, 384, 384, 384, None, 0, 100, 3, -1, 0.1, None, None, 0, None) == 0   # no segments
    assert fwd(None, None, None, 384, 384, 384, None, 2, 0, 3, -1, 0.1, None, None, 0, None) == 0     # max_seqlen 0
    assert fwd(None, None, None, 384, 384, 384, None, 2, 100, 3, -1, 0.1, None, None, 0, None) == -1
    assert fwd(p, p, p, 384, 384, 384, p, 2, 100, 0, -1, 0.1, p, p, 0, None) == -2                   # heads
    assert fwd(p, p, p, 383, 384, 384, p, 2, 100, 3, -1, 0.1, p, p, 0, None) == -2                   # stride < row
    assert fwd(p, p, p, 392, 384, 388, p, 2, 100, 3, -1, 0.1, p, p, 0, None) == -2                   # not x8
    assert fwd(q, p, p, 384, 384, 384, p, 2, 100, 3, -1, 0.1, p, p, 0, None) == -2                   # alignment
    assert fwd(p, p, p, 384, 384, 384, p, 2, 100, 3, -1, 0.0, p, p, 0, None) == -2                   # scale
    bwd = lib.nc_flash_attn_bwd
    args = [p, p, p, p, 384, 384, 384, 384, p, 0, p, p, 2, 100, 3, -1, 0.1, p, p, p, 384, 384, 384, None]
    bad = list(args)
    bad[3] = None
    assert bwd(*bad) == -1
    bad = list(args)
    bad[22] = 380
    assert bwd(*bad) == -2
    bad = list(args)
    bad[19] = q
    assert bwd(*bad) == -2
    rows = lib.nc_flash_attn_bwd_rows
    assert rows(None, 384, None, 384, 0, 3, None, None) == 0
    assert rows(None, 384, None, 384, 5, 3, None, None) == -1
    assert rows(p, 380, p, 384, 5, 3, p, None) == -2


def test_decode_header_covers_the_reference_abi():
    from nanochat_amd.native import DECODE_SIGNATURES

    assert REFERENCE_DEC <= decode_declared()
    assert decode_declared() == set(DECODE_SIGNATURES)


def test_decode_library_exports_every_declared_symbol():
    from nanochat_amd.native import DECODE_LIBRARY, hip_library

    if not DECODE_LIBRARY.exists():
        pytest.fail(f"{DECODE_LIBRARY} is not built: run python -m nanochat_amd.native")
    dec = hip_library("decode")
    for name in decode_declared():
        assert hasattr(dec, name), name
    # the kernel entry points ride along in the decoder library
    for name in declared():
        assert hasattr(dec, name), name
    assert dec.dec_prefill_rows(None) == 16384


def test_decode_argtypes_match_the_reference_binding():
    """decoder.py:132-148's argtypes for the 14 symbols, restated as ctypes types."""
    from nanochat_amd.native import DECODE_SIGNATURES

    P, I = ctypes.c_void_p, ctypes.c_int
    expected = {
        "dec_create": [P] * 5, "dec_batch": [P],
        "dec_set_prompt": [P, I, ctypes.c_int32, ctypes.c_int32, ctypes.c_float, ctypes.c_float, ctypes.c_ulonglong],
        "dec_prefill_rows": [P], "dec_prefill": [P, I, P], "dec_save_prompt": [P, I, I, I, I],
        "dec_load_prompt": [P, I, I, I, I], "dec_masks": [P], "dec_set_active": [P, P], "dec_launch_body": [P],
        "dec_launch_head": [P], "dec_destroy": [P], "dec_tokens": [P, P], "dec_take_alt": [P, I],
    }
    for name, argtypes in expected.items():
        assert DECODE_SIGNATURES[name][0] == argtypes, name
    assert DECODE_SIGNATURES["dec_create"][1] is P
    assert DECODE_SIGNATURES["dec_masks"][1] == ctypes.POINTER(ctypes.c_uint32)


def test_slot_gemm_declines_without_launching():
    """Shapes, slice counts and missing operands the step GEMM cannot take return -2 before any device call; long K is
    cut into slices of at most 2,048 (16 chunks of 128), short K is never split."""
    from nanochat_amd.native import hip_library

    lib = hip_library("decode")
    F32, RELU2 = 4, 2
    args = (DUMMY, 1664, 6656, DUMMY, 128, DUMMY, DUMMY, DUMMY, DUMMY)
    assert lib.dec_debug_slot_gemm(F32, DUMMY, 1664, 6656, DUMMY, 129, None, DUMMY, None, None, 1, None, None) == -2
    assert lib.dec_debug_slot_gemm(F32, DUMMY, 1664, 6600, DUMMY, 128, None, DUMMY, None, None, 1, None, None) == -2
    assert lib.dec_debug_slot_gemm(F32, DUMMY, 1662, 6656, DUMMY, 128, None, DUMMY, None, None, 1, None, None) == -2
    assert lib.dec_debug_slot_gemm(F32, *args, 53, DUMMY, None) == -2           # more slices than chunks
    assert lib.dec_debug_slot_gemm(F32, *args, 14, None, None) == -2            # partials need a buffer
    assert lib.dec_debug_slot_gemm(RELU2, DUMMY, 1664, 6656, DUMMY, 128, DUMMY, None, None, None, 1, None,
                                   None) == -2                                   # ReLU^2 needs rstd
    assert lib.dec_debug_slot_gemm(7, *args, 1, None, None) == -2               # no such epilogue
    for R, K, S in ((4992, 1664, 1), (1664, 1664, 1), (6656, 1664, 1), (1664, 6656, 4), (65536, 1664, 1),
                    (100, 128, 1), (768, 2048, 1), (768, 2176, 2)):
        assert lib.dec_debug_slot_gemm_slices(R, K) == S, (R, K)
    assert lib.dec_debug_slot_gemm_part_bytes(1664, 128, 1) == 0
    assert lib.dec_debug_slot_gemm_part_bytes(1664, 128, 4) == 4 * 128 * 1664 * 4


def test_slot_gemm_tiles():
    """The workgroup tile (RT 16-row weight tiles, CT 16-slot tiles, as 100 RT + CT) is the one whose busiest CU takes
    in the fewest bytes, ceil(workgroups / 256) x stages x (RT + CT): at config 5's 128 slots qkv splits the slots into
    two groups of 64 with 48 weight rows a workgroup (208 workgroups), o into four groups of 32 (208), fc and proj into
    two of 64 with 64 rows (208), and lm_head keeps all 128 slots with 64 rows (1,024). The GPU tests' shapes cover every
    tile built."""
    from nanochat_amd.native import hip_library
    from tests.test_gpu_slot_gemm import SHAPES

    lib = hip_library("decode")
    tiles = {(4992, 1664): 304, (1664, 1664): 202, (6656, 1664): 404, (1664, 6656): 404, (65536, 1664): 408}
    for (R, K), t in tiles.items():
        assert lib.dec_debug_slot_gemm_tile(R, K, 128, 0) == t, (R, K)

    def cost(R, K, N, S, rt, ct):
        wgs = -(-R // (16 * rt)) * S * -(-N // (16 * ct))
        return -(-wgs // 256) * (K // 128 // S) * (rt + ct)

    built = (202, 304, 404, 408)
    seen = set()
    for R, K, N in SHAPES:
        for S in (1, 2, 3):
            if S > K // 128:
                continue
            t = lib.dec_debug_slot_gemm_tile(R, K, N, S)
            costs = [cost(R, K, N, S, b // 100, b % 100) for b in built]
            assert t == built[costs.index(min(costs))], (R, K, N, S)
            seen.add(t)
    assert seen == set(built)
    assert lib.dec_debug_slot_gemm_tile(1664, 6600, 128, 0) == -2     # K not a multiple of 128
    assert lib.dec_debug_slot_gemm_tile(1664, 1664, 129, 0) == -2     # more than 128 slots
    assert lib.dec_debug_slot_gemm_tile(1664, 256, 128, 3) == -2      # more slices than chunks


def test_nucleus_cut_declines_shapes():
    """The nucleus-threshold hook refuses an empty or too large vocabulary and a negative row count before any device
    call; zero rows is a no-op."""
    from nanochat_amd.native import hip_library

    lib = hip_library("decode")
    assert lib.dec_debug_nucleus_cut(DUMMY, 1, 0, DUMMY, DUMMY, None) == -2
    assert lib.dec_debug_nucleus_cut(DUMMY, -1, 64, DUMMY, DUMMY, None) == -2
    assert lib.dec_debug_nucleus_cut(DUMMY, 1, 1 << 25, DUMMY, DUMMY, None) == -2
    assert lib.dec_debug_nucleus_cut(DUMMY, 0, 64, DUMMY, DUMMY, None) == 0


def test_prefill_gemm_declines_without_launching():
    """Shapes and missing operands the prefill GEMM cannot take return -2 before any device call; M = 0 is a no-op."""
    from nanochat_amd.native import hip_library

    lib = hip_library("decode")
    STORE, RELU2, RESID, F32 = 0, 2, 3, 4
    assert lib.dec_debug_prefill_gemm(STORE, DUMMY, 4992, 1600, DUMMY, 8, DUMMY, None, None, None, None) == -2   # K
    assert lib.dec_debug_prefill_gemm(STORE, DUMMY, 4990, 1664, DUMMY, 8, DUMMY, None, None, None, None) == -2   # N
    assert lib.dec_debug_prefill_gemm(STORE, DUMMY, 4992, 1664, DUMMY, 8, None, None, None, None, None) == -2    # out
    assert lib.dec_debug_prefill_gemm(F32, DUMMY, 4992, 1664, DUMMY, 8, DUMMY, None, None, None, None) == -2     # fp32
    assert lib.dec_debug_prefill_gemm(RESID, DUMMY, 1664, 1664, DUMMY, 8, DUMMY, None, None, None, None) == -2   # res
    assert lib.dec_debug_prefill_gemm(RELU2, DUMMY, 6656, 1664, DUMMY, 8, DUMMY, None, None, None, None) == -2   # rstd
    assert lib.dec_debug_prefill_gemm(1, DUMMY, 1664, 1664, DUMMY, 8, DUMMY, DUMMY, DUMMY, DUMMY, None) == -2    # kind
    assert lib.dec_debug_prefill_gemm(STORE, DUMMY, 4992, 1664, DUMMY, 0, DUMMY, None, None, None, None) == 0


def test_append_runs_declines_without_launching():
    """The prefill append hook refuses NULL operands and shapes it cannot take with -2 before any device call; no runs
    is a no-op."""
    from nanochat_amd.native import hip_library

    lib = hip_library("decode")
    D = DUMMY

    def call(qkv=D, stride=6 * 128, runs=1, max_count=4, Hq=2, Hkv=2, rope_len=64, max_pages=4, num_pages=8, ve=None,
             ve_h=None, gate=None, tokens=None, C=256):
        return lib.dec_debug_append_runs(qkv, stride, runs, max_count, D, D, D, D, Hq, Hkv, D, D, D, D, rope_len, D, D,
                                         max_pages, D, D, D, num_pages, ve_h, ve, gate, tokens, C, None)

    assert call(qkv=None) == -2
    assert call(stride=5 * 128) == -2                     # shorter than a token's q, k and v
    assert call(Hq=3, Hkv=2) == -2                        # q heads not a multiple of KV heads
    assert call(rope_len=0) == -2
    assert call(ve=D) == -2                               # value embeddings without their stream, gate and tokens
    assert call(ve=D, ve_h=D, gate=D, tokens=D, C=255) == -2   # C narrower than the KV heads' rows
    assert call(runs=0) == 0
