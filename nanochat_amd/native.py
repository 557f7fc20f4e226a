"""The HIP libraries of the fp8 KV path: their hipcc build for gfx950 and their ctypes bindings.

Mirrors the reference's loader (native.py:43-65: `pointer`, `stream`, `cuda_library`) with one
difference in build policy: the libraries are compiled ahead of time into the package (by `build()` or
`python -m nanochat_amd.native`) and only loaded at run time, so a GPU host never compiles. Loading a
missing library builds both once.

    libnanochat_kv.so      the kernel entry points of include/nanochat_amd.h
    libnanochat_decode.so  the decoder runtime of include/nanochat_decode.h (the same kernels, plus the
                           dec_* runtime and its hand-written step and prefill GEMMs);
                           hip_library("decode") loads it, as the reference's cuda_library("decode")
                           loads decode.cu
"""

import ctypes
import functools
import os
import subprocess
import sys
import tempfile
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
INCLUDE = PACKAGE.parent / "include"
LIB_DIR = PACKAGE / "lib"
LIBRARY = LIB_DIR / "libnanochat_kv.so"
DECODE_LIBRARY = LIB_DIR / "libnanochat_decode.so"
KERNEL_SOURCES = [CSRC / "kv_append.hip", CSRC / "attention.hip", CSRC / "ve_gate.hip", CSRC / "flash_attn.hip"]
DECODE_SOURCES = [CSRC / "decoder.hip", CSRC / "slot_gemm.hip", CSRC / "prefill_gemm.hip"]
SOURCES = KERNEL_SOURCES + DECODE_SOURCES
HEADERS = [CSRC / "nc_device.h", CSRC / "nc_internal.h", INCLUDE / "nanochat_amd.h", INCLUDE / "nanochat_decode.h"]
HEAD_DIM = 128

# -ffp-contract=off: the append's fp32 order is part of its bit-exact contract (no implicit FMAs).
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in any kernel.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-DHEAD_DIM={HEAD_DIM}", f"-I{INCLUDE}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{' '.join(cmd)}\n{result.stderr}")


def build() -> tuple[Path, Path]:
    """Compile every source once, then link both libraries (each written to a temporary file, then renamed)."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(dir=LIB_DIR) as tmp:
        objects = {}
        for src in SOURCES:
            objects[src] = Path(tmp) / (src.stem + ".o")
            _run([hipcc(), *HIPCC_FLAGS, "-c", "-o", str(objects[src]), str(src)])
        for output, sources, libs in ((LIBRARY, KERNEL_SOURCES, []), (DECODE_LIBRARY, KERNEL_SOURCES + DECODE_SOURCES, [])):
            built = Path(tmp) / output.name
            _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(built),
                  *(str(objects[s]) for s in sources), *libs])
            built.replace(output)
    return LIBRARY, DECODE_LIBRARY


c_void_p, c_int, c_longlong, c_float, c_size_t = (ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float,
                                                   ctypes.c_size_t)

# argtypes of every entry point of include/nanochat_amd.h
SIGNATURES = {
    "nc_status_string": ([c_int], ctypes.c_char_p),
    "nc_abi_version": ([], c_int),
    "nc_last_error": ([], c_int),
    "qkp_forward": ([c_void_p] * 8 + [c_longlong, c_int, c_int, c_void_p], None),
    "qkp_backward": ([c_void_p] * 13 + [c_longlong, c_int, c_int, c_void_p], None),
    "qkp_backward_blocks": ([], c_int),
    "nc_kv_append_fp8": ([c_void_p, c_void_p, c_longlong, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int,
                          c_void_p, c_void_p, c_void_p, c_int, c_void_p], c_int),
    "nc_qk_norm_rope_append_fp8": ([c_void_p, c_longlong, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                    c_void_p, c_int, c_void_p], c_int),
    "nc_decode_workspace_bytes": ([c_int, c_int, c_int, c_int, c_int], c_size_t),
    "nc_decode_attn_fp8": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_int,
                            c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p, c_size_t, c_void_p], c_int),
    "nc_decode_step_fp8": ([c_void_p, c_longlong, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                            c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p,
                            c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_int, c_void_p,
                            c_void_p, c_size_t, c_void_p], c_int),
    "nc_decode_attn_fp8_noalloc": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int,
                                    c_int, c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p], c_int),
    "nc_prefill_attn_fp8": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_int,
                             c_int, c_int, c_int, c_float, c_void_p, c_void_p], c_int),
    "nc_debug_read_pages": ([c_void_p, c_longlong, c_void_p, c_int, c_int, c_void_p, c_void_p], c_int),
    "ve_forward": ([c_void_p, c_void_p, c_longlong] + [c_void_p] * 5 + [c_longlong, c_void_p], None),
    "ve_backward": ([c_void_p, c_longlong] + [c_void_p] * 8 + [c_longlong, c_void_p], None),
    "nc_ve_forward": ([c_void_p, c_void_p, c_longlong, c_void_p, c_void_p, c_longlong, c_void_p, c_void_p, c_void_p,
                       c_longlong, c_int, c_void_p], c_int),
    "nc_ve_backward": ([c_void_p, c_longlong, c_void_p, c_void_p, c_void_p, c_longlong, c_void_p, c_void_p, c_void_p,
                        c_void_p, c_void_p, c_longlong, c_int, c_void_p], c_int),
    "nc_flash_attn_fwd": ([c_void_p] * 3 + [c_longlong] * 3 + [c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p,
                                                                c_void_p, c_longlong, c_void_p], c_int),
    "nc_flash_attn_bwd": ([c_void_p] * 4 + [c_longlong] * 4 + [c_void_p, c_longlong, c_void_p, c_void_p, c_int, c_int,
                                                                c_int, c_int, c_float, c_void_p, c_void_p, c_void_p,
                                                                c_longlong, c_longlong, c_longlong, c_void_p], c_int),
    "nc_flash_attn_bwd_rows": ([c_void_p, c_longlong, c_void_p, c_longlong, c_longlong, c_int, c_void_p, c_void_p],
                               c_int),
}


# argtypes of every entry point of include/nanochat_decode.h (the reference's binding: decoder.py:132-148)
DECODE_SIGNATURES = {
    "dec_create": ([c_void_p] * 5, c_void_p),
    "dec_create_slots": ([c_void_p] * 5 + [c_int], c_void_p),
    "dec_create_pool": ([c_void_p] * 5 + [c_int, c_longlong], c_void_p),
    "dec_release": ([c_void_p, c_int], None),
    "dec_debug_pages": ([c_void_p, c_void_p], None),
    "dec_batch": ([c_void_p], c_int),
    "dec_set_prompt": ([c_void_p, c_int, ctypes.c_int32, ctypes.c_int32, c_float, c_float, ctypes.c_ulonglong], None),
    "dec_prefill_rows": ([c_void_p], c_int),
    "dec_prefill": ([c_void_p, c_int, c_void_p], None),
    "dec_save_prompt": ([c_void_p, c_int, c_int, c_int, c_int], None),
    "dec_load_prompt": ([c_void_p, c_int, c_int, c_int, c_int], None),
    "dec_masks": ([c_void_p], ctypes.POINTER(ctypes.c_uint32)),
    "dec_set_active": ([c_void_p, c_void_p], None),
    "dec_launch_body": ([c_void_p], None),
    "dec_launch_head": ([c_void_p], None),
    "dec_tokens": ([c_void_p, c_void_p], None),
    "dec_take_alt": ([c_void_p, c_int], None),
    "dec_destroy": ([c_void_p], None),
    "dec_debug_logits": ([c_void_p, c_void_p, c_int], None),
    "dec_debug_cache": ([c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p], None),
    "dec_debug_table": ([c_void_p, c_int, c_void_p], None),
    "dec_debug_set_split": ([c_void_p, c_int], None),
    "dec_debug_set_graphs": ([c_void_p, c_int], None),
    "dec_debug_slot_gemm": ([c_int, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                             c_int, c_void_p, c_void_p], c_int),
    "dec_debug_slot_gemm_slices": ([c_int, c_int], c_int),
    "dec_debug_slot_gemm_part_bytes": ([c_int, c_int, c_int], c_longlong),
    "dec_debug_slot_gemm_tile": ([c_int, c_int, c_int, c_int], c_int),
    "dec_debug_slot_gemm_ssq": ([c_int, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                 c_void_p], c_int),
    "dec_debug_nucleus_cut": ([c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p], c_int),
    "dec_debug_prefill_gemm": ([c_int, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p], c_int),
    "dec_debug_append_runs": ([c_void_p, c_longlong, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                               c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p,
                               c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p],
                              c_int),
}

LIBRARIES = {"nanochat_kv": (LIBRARY, SIGNATURES), "decode": (DECODE_LIBRARY, DECODE_SIGNATURES)}


@functools.cache
def hip_library(name: str = "nanochat_kv") -> ctypes.CDLL:
    """A prebuilt library (both built here first if absent) with every entry point's argtypes set; once per process.
    "nanochat_kv": the kernel entry points; "decode": the dec_* decoder runtime."""
    if name not in LIBRARIES:
        raise ValueError(f"unknown library {name!r}: expected one of {sorted(LIBRARIES)}")
    path, signatures = LIBRARIES[name]
    if not path.exists():
        build()
    lib = ctypes.CDLL(str(path))
    for symbol, (argtypes, restype) in signatures.items():
        fn = getattr(lib, symbol)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


class NativeError(RuntimeError):
    """A nonzero status from an entry point of the library."""


def check(status: int) -> None:
    if status != 0:
        text = hip_library().nc_status_string(status).decode()
        raise NativeError(f"nanochat_kv status {status}: {text}")


def pointer(t) -> int:
    """A tensor's device address (reference native.py:43-44), as the integer the entry points' c_void_p argtypes take
    (a ctypes object per argument costs a decode step's launch from Python about 0.2 us each)."""
    return t.data_ptr()


def stream() -> int:
    """The current torch stream of the current device (a hipStream_t), which the kernels launch on (reference
    native.py:47-51). Read through torch's raw-stream getter where it exists, which builds no Stream object (about
    2 us a call less); torch.cuda.current_stream() otherwise."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return torch.cuda.current_stream().cuda_stream
    torch.cuda._lazy_init()
    return raw(torch._C._cuda_getDevice())


if __name__ == "__main__":
    print(build())
    sys.exit(0)
