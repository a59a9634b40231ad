"""ctypes binding of libmamba_int.so (the C ABI declared in include/mamba_int.h).

Loaded once per process, with explicit argtypes/restype, like the reference's
``_load_library`` (``src/triton_kernels/warp_scan.py:16-56``).  Unlike the
reference there is no silent fallback: a missing library raises, and every
entry point's status is checked (``MIError`` carries ``mi_last_error_string``).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("MAMBA_INT_LIB", os.path.join(PKG_ROOT, "libmamba_int.so"))

MI_OK, MI_ERR_NULL_POINTER, MI_ERR_BAD_DIM, MI_ERR_BAD_ALIGNMENT, MI_ERR_BAD_ARG, MI_ERR_HIP = range(6)
OUT_INT32, OUT_INT8, OUT_DECAY_MOD, OUT_RESIDUAL, OUT_FLOAT = range(5)

P = ctypes.c_void_p
I = ctypes.c_int
I32 = ctypes.c_int32
F = ctypes.c_float

# name -> argtypes, in the order of include/mamba_int.h
SIGNATURES = {
    "mi_dyadic_scan": [P, P, P, P, I, P, P, P, I, I, I, I, P],
    "mi_dyadic_scan_f32": [P, P, P, P, I, I, I, I, P],
    "mi_dyadic_scan_elementwise": [P, P, I, P, P, P, I, I, I, P],
    "mi_dyadic_chunked_scan": [P, P, I, I, P, P, P, P, P, I, I, I, P],
    "mi_ssd_chunked_scan": [P, P, P, P, I, P, P, P, P, I, I, I, I, I, I, P],
    "mi_pack_ternary": [P, P, I, I, P],
    "mi_act_quant_f32": [P, P, P, I, I, P],
    "mi_bitlinear": [P, I, P, P, I, I, I, I, I, I, I32, I, I32, P, F, P, P],
    "mi_bitlinear_gemm": [P, I, P, P, I, I, I, I, I, I, I32, I, I32, P, F, P, P],
    "mi_bitlinear_gemv": [P, I, P, P, I, I, I, I, I, I, I32, I, I32, P, F, P, P],
    "mi_bitlinear_residual_parts": [P, I, P, P, I, I, I, I, I32, I, I32, P, P],
    "mi_bitshift_norm": [P, P, P, I, I, P, P],
    "mi_embed": [P, P, P, I, I, I, P, I, P],
    "mi_conv_squareplus": [P, I, P, P, P, P, P, I, I, I, P],
    "mi_in_proj_conv": [P, I, P, I, P, P, P, P, P, P, I, I, I, I, I, P],
    "mi_block_scan": [P, P, P, I, I, P, I, I, P, I, I, P, P, P, I, I, I, I, P],
    "mi_bitshift_norm_v2": [P, P, P, I, I, P, P],
    "mi_ssd_block_scan": [P, P, I, P, I, I, P, I, I, P, P, P, I, I, I, I, P],
    "mi_argmax_i32": [P, I, P, I, I, P],
    "mi_norm_bitlinear": [P, P, I, P, P, P, I, I, I, I, I, I, P],
    "mi_norm_in_proj_conv": [P, P, I, P, P, I, P, P, P, P, P, I, I, I, P],
    "mi_norm_v2_in_proj_conv": [P, P, I, P, P, I, P, P, P, P, P, I, I, I, P],
    "mi_dt_scan_step": [P, I, I, P, I, P, P, I, I, P, I, I, P, P, I, I, I, P],
    "mi_xproj_dt_scan_step": [P, P, I, I, P, I, P, I, I, P, I, I, P, P, I, I, I, P],
    "mi_norm_in_proj_conv_xpart": [P, P, I, P, P, I, P, P, P, P, P, P, I, P, I, I, I, P],
    "mi_xpart_dt_scan_step": [P, I, I, I, P, I, P, P, I, I, P, I, I, P, P, I, I, I, P],
    "mi_bitshift_norm_parts": [P, P, P, I, I, P, I, I, P],
    "mi_conv_step_xproj": [P, I, P, P, P, P, P, I, I, P, I, I, I, P],
    "mi_conv_step_xpart": [P, I, P, P, P, P, P, I, P, I, I, P],
    "mi_norm_bitlinear_argmax": [P, P, I, P, P, P, I, P, I, I, I, P],
    "mi_argmax_keys": [P, I, P, I, P],
    "mi_embed_argmax": [P, I, P, P, P, I, I, I, P, I, P],
    "mi_decode_workspace_size": [P, I, P],
    "mi_decode_step": [P, I, P, P, P, I, P, P, P, ctypes.c_size_t, P],
    "mi_decode_step_static": [P, I, P, P, P, I, P, P, P],
    "mi_checkpoint_open": [ctypes.c_char_p, P],
    "mi_checkpoint_get_info": [P, P],
    "mi_checkpoint_upload": [P, P, ctypes.c_size_t, P, P, I, P],
}


class MIError(RuntimeError):
    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libmamba_int.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libmamba_int.so not found at {LIB_PATH}; build it first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        # torch first: it and this library then share torch's HIP runtime
        # (both link libamdhip64.so.7; the one loaded first serves the process,
        # and a library call made through a runtime loaded before torch's
        # finds no device)
        import torch  # noqa: F401
        lib = ctypes.CDLL(LIB_PATH)
        lib.mi_version.restype = ctypes.c_char_p
        lib.mi_version.argtypes = []
        lib.mi_last_error_string.restype = ctypes.c_char_p
        lib.mi_last_error_string.argtypes = []
        lib.mi_checkpoint_close.restype = None
        lib.mi_checkpoint_close.argtypes = [P]
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _lib = lib
    return _lib


def version() -> str:
    return load().mi_version().decode()


def call(name: str, *args) -> None:
    lib = load()
    st = getattr(lib, name)(*args)
    if st != MI_OK:
        raise MIError(name, st, lib.mi_last_error_string().decode())


def raw(name: str, *args) -> int:
    """Call without raising; returns the mi_status (used by ABI tests)."""
    return getattr(load(), name)(*args)


def last_error() -> str:
    return load().mi_last_error_string().decode()
