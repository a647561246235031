"""ctypes binding of the C ABI in include/mamba3_scan.h.

The library is loaded once, after ``import torch`` so that it binds to the HIP
runtime torch already loaded (both carry the soname libamdhip64.so.7).  There
is no fallback: if the library is missing or does not export the ABI, every
entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (load torch's HIP runtime first)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmamba3_rocm.so")
# return codes of the C ABI (include/mamba3_scan.h)
M3_OK, M3_E_ARG, M3_E_ALIGN, M3_E_UNSUPPORTED, M3_E_LAUNCH = 0, 1, 2, 3, 4
# activations of m3_block_act (include/mamba3_layer.h)
M3_ACT_GELU, M3_ACT_FULL_GLU, M3_ACT_HALF_GLU1, M3_ACT_HALF_GLU2 = 0, 1, 2, 3

DTYPE_F32 = 0
DTYPE_BF16 = 1
IMPL_NONE, IMPL_CHUNKED_MFMA, IMPL_GENERIC = 0, 1, 2

EXPORTS = ("m3_abi_version", "m3_last_error", "m3_chunk_scan_impl", "m3_chunk_scan_fwd",
           "m3_chunk_scan_fwd_carry", "m3_chunk_scan_ws_bytes", "m3_chunk_scan_fwd_ws",
           "m3_chunk_scan_fwd_noalloc",
           "m3_chunk_scan_bwd_ws_bytes", "m3_chunk_scan_bwd", "m3_chunk_scan_fwd_shared",
           "m3_chunk_scan_bwd_shared_ws_bytes", "m3_chunk_scan_bwd_shared", "m3_chunk_scan_saved_bytes",
           "m3_chunk_scan_fwd_train", "m3_chunk_scan_bwd_saved_ws_bytes", "m3_chunk_scan_bwd_saved",
           "m3_chunk_scan_fwd_train_shared", "m3_chunk_scan_bwd_saved_shared_ws_bytes",
           "m3_chunk_scan_bwd_saved_shared",
           "m3_decode_step",
           "m3_layer_pre", "m3_layer_scan", "m3_layer_scan_carry", "m3_layer_scan_train", "m3_layer_scan_bwd",
           "m3_layer_decode_step", "m3_split_bf16x3",
           "m3_layer_post",
           "m3_layer_post_bwd_ws_bytes", "m3_layer_post_bwd",
           "m3_layer_pre_bwd_ws_bytes", "m3_layer_pre_bwd",
           "m3_block_norm", "m3_block_gelu", "m3_block_act", "m3_block_act_norm",
           "m3_log_softmax", "m3_block_act_bwd", "m3_block_gelu_bwd", "m3_block_norm_bwd_ws_bytes",
           "m3_block_norm_bwd", "m3_log_softmax_nll")

_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGS = {
    "m3_abi_version": ([], _I),
    "m3_last_error": ([], ctypes.c_char_p),
    "m3_chunk_scan_impl": ([_I] * 5, _I),
    "m3_chunk_scan_fwd": ([_P] * 12 + [_I] * 9 + [_P], _I),
    "m3_chunk_scan_fwd_carry": ([_P] * 20 + [_I] * 9 + [_P], _I),
    "m3_chunk_scan_ws_bytes": ([_I] * 8, ctypes.c_size_t),
    "m3_chunk_scan_fwd_ws": ([_P] * 20 + [_I] * 9 + [_P, ctypes.c_size_t, _P], _I),
    "m3_chunk_scan_fwd_noalloc": ([_P] * 20 + [_I] * 9 + [_P], _I),
    "m3_chunk_scan_bwd_ws_bytes": ([_I] * 9, ctypes.c_size_t),
    "m3_chunk_scan_bwd": ([_P] * 23 + [_I] * 9 + [_P, ctypes.c_size_t, _P], _I),
    "m3_chunk_scan_fwd_shared": ([_P] * 12 + [_I] * 8 + [_P, ctypes.c_size_t, _P], _I),
    "m3_chunk_scan_bwd_shared_ws_bytes": ([_I] * 8, ctypes.c_size_t),
    "m3_chunk_scan_bwd_shared": ([_P] * 23 + [_I] * 8 + [_P, ctypes.c_size_t, _P], _I),
    "m3_chunk_scan_saved_bytes": ([_I] * 7, ctypes.c_size_t),
    "m3_chunk_scan_fwd_train": ([_P] * 12 + [_I] * 9 + [_P, ctypes.c_size_t, _P, ctypes.c_size_t, _P], _I),
    "m3_chunk_scan_bwd_saved_ws_bytes": ([_I] * 9, ctypes.c_size_t),
    "m3_chunk_scan_bwd_saved": ([_P] * 23 + [_I] * 9 + [_P, ctypes.c_size_t, _P, ctypes.c_size_t, _P], _I),
    "m3_chunk_scan_fwd_train_shared": ([_P] * 12 + [_I] * 8 + [_P, ctypes.c_size_t, _P, ctypes.c_size_t, _P], _I),
    "m3_chunk_scan_bwd_saved_shared_ws_bytes": ([_I] * 8, ctypes.c_size_t),
    "m3_chunk_scan_bwd_saved_shared": ([_P] * 23 + [_I] * 8 + [_P, ctypes.c_size_t, _P, ctypes.c_size_t, _P], _I),
    "m3_layer_pre": ([_P] * 12 + [_I] * 6 + [ctypes.c_float, ctypes.c_float, _I, _P], _I),
    "m3_layer_decode_step": ([_P] * 12 + [_I] * 5 + [ctypes.c_float] * 2 + [_I] * 3 + [_P], _I),
    "m3_split_bf16x3": ([_P] * 4 + [ctypes.c_long, _I, ctypes.c_long, _P], _I),
    "m3_layer_scan": ([_P] * 3 + [_I] + [_P] * 8 + [_I] * 8 + [_P, ctypes.c_size_t, _P], _I),
    "m3_layer_scan_carry": ([_P] * 3 + [_I] + [_P] * 16 + [_I] * 8 + [_P, ctypes.c_size_t, _P], _I),
    "m3_layer_scan_train": ([_P] * 3 + [_I] + [_P] * 8 + [_I] * 8 + [_P, ctypes.c_size_t] * 2 + [_P], _I),
    "m3_layer_scan_bwd": ([_P] * 3 + [_I] + [_P] * 18 + [_I] * 8 + [_P, ctypes.c_size_t] * 2 + [_P], _I),
    "m3_layer_post": ([_P] * 3 + [_I] * 3 + [ctypes.c_float, _I, _P], _I),
    "m3_layer_post_bwd_ws_bytes": ([_I] * 3, ctypes.c_size_t),
    "m3_layer_post_bwd": ([_P] * 5 + [_I] * 3 + [ctypes.c_float, _I, _P, ctypes.c_size_t, _P], _I),
    "m3_layer_pre_bwd_ws_bytes": ([_I] * 4, ctypes.c_size_t),
    "m3_layer_pre_bwd": ([_P] * 16 + [_I] * 6 + [ctypes.c_float] * 2 + [_I, _P, ctypes.c_size_t, _P], _I),
    "m3_block_norm": ([_P] * 4 + [_I] * 3 + [ctypes.c_float, _I, _P], _I),
    "m3_block_gelu": ([_P] * 2 + [_I] * 4 + [_P], _I),
    "m3_block_act": ([_P] * 5 + [_I] * 5 + [_P], _I),
    "m3_block_act_norm": ([_P] * 8 + [_I] * 3 + [ctypes.c_float] + [_I] * 3 + [_P], _I),
    "m3_log_softmax": ([_P] * 2 + [_I] * 3 + [_P], _I),
    "m3_block_act_bwd": ([_P] * 6 + [_I] * 5 + [_P], _I),
    "m3_block_gelu_bwd": ([_P] * 4 + [_I] * 5 + [_P], _I),
    "m3_block_norm_bwd_ws_bytes": ([_I] * 3, ctypes.c_size_t),
    "m3_block_norm_bwd": ([_P] * 7 + [_I] * 3 + [ctypes.c_float, _I, _P, ctypes.c_size_t, _P], _I),
    "m3_log_softmax_nll": ([_P] * 3 + [_I] * 3 + [ctypes.c_float, _P], _I),
    "m3_decode_step": ([_P] * 16 + [_I] * 9 + [_P], _I),
}

_lock = threading.Lock()
_lib = None


class Mamba3LibraryError(RuntimeError):
    """The HIP library is missing, stale, or a call into it failed."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises Mamba3LibraryError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise Mamba3LibraryError(
                    f"{LIB_PATH} is not built; run `python sigma-0_amd/build.py` (hipcc, gfx950)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in _SIGS.items():
                fn = getattr(lib, name, None)
                if fn is None:
                    raise Mamba3LibraryError(f"{LIB_PATH} does not export {name}")
                fn.argtypes = args
                fn.restype = res
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().m3_last_error().decode(errors="replace")
        raise Mamba3LibraryError(f"{what} failed (code {rc}): {msg}")


def impl_for(io_dtype: int, N: int, P: int, R: int, chunk_size: int) -> int:
    return load().m3_chunk_scan_impl(io_dtype, N, P, R, chunk_size)
