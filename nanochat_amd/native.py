"""The HIP library of the fp8 KV path: its hipcc build for gfx950 and its ctypes binding.

Mirrors the reference's loader (native.py:43-65: `pointer`, `stream`, `cuda_library`) with one
difference in build policy: the library is compiled ahead of time into the package
(`nanochat_amd/lib/libnanochat_kv.so`, by `build()` or `python -m nanochat_amd.native`) and only
loaded at run time, so a GPU host never compiles. Loading a missing library builds it once.
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
SOURCES = [CSRC / "kv_append.hip", CSRC / "attention.hip"]
HEADERS = [CSRC / "nc_device.h", INCLUDE / "nanochat_amd.h"]
HEAD_DIM = 128

# -ffp-contract=off: the append's fp32 order is part of its bit-exact contract (no implicit FMAs).
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in any kernel.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-DHEAD_DIM={HEAD_DIM}", f"-I{INCLUDE}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def build(output: Path = LIBRARY) -> Path:
    """Compile every kernel source into one shared library (written to a temporary file, then renamed)."""
    output.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(dir=output.parent) as tmp:
        built = Path(tmp) / output.name
        cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(built), *map(str, SOURCES)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"hipcc failed ({result.returncode}):\n{' '.join(cmd)}\n{result.stderr}")
        built.replace(output)
    return output


c_void_p, c_int, c_longlong, c_float, c_size_t = (ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float,
                                                   ctypes.c_size_t)

# argtypes of every entry point of include/nanochat_amd.h
SIGNATURES = {
    "nc_status_string": ([c_int], ctypes.c_char_p),
    "nc_abi_version": ([], c_int),
    "nc_last_error": ([], c_int),
    "qkp_forward": ([c_void_p] * 8 + [c_longlong, c_int, c_int, c_void_p], None),
    "nc_kv_append_fp8": ([c_void_p, c_void_p, c_longlong, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int,
                          c_void_p, c_void_p, c_void_p, c_int, c_void_p], c_int),
    "nc_qk_norm_rope_append_fp8": ([c_void_p, c_longlong, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                    c_void_p, c_int, c_void_p], c_int),
    "nc_decode_workspace_bytes": ([c_int, c_int, c_int, c_int, c_int, c_int], c_size_t),
    "nc_decode_attn_fp8": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_int,
                            c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p, c_size_t, c_void_p], c_int),
    "nc_prefill_attn_fp8": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_int,
                             c_int, c_int, c_int, c_float, c_void_p, c_void_p], c_int),
}


@functools.cache
def hip_library(name: str = "nanochat_kv") -> ctypes.CDLL:
    """The prebuilt library (built here first if absent), with every entry point's argtypes set; once per process."""
    if name != "nanochat_kv":
        raise ValueError(f"unknown library {name!r}: the fp8 KV path ships one library, 'nanochat_kv'")
    if not LIBRARY.exists():
        build()
    lib = ctypes.CDLL(str(LIBRARY))
    for symbol, (argtypes, restype) in SIGNATURES.items():
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


def pointer(t) -> ctypes.c_void_p:
    """A tensor's device address (reference native.py:43-44)."""
    return ctypes.c_void_p(t.data_ptr())


def stream() -> ctypes.c_void_p:
    """The current torch stream (a hipStream_t), which the kernels launch on (reference native.py:47-51)."""
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


if __name__ == "__main__":
    print(build())
    sys.exit(0)
