"""ctypes binding of liba8attn.so, the gfx950 HIP library behind include/a8attn.h.

The library is loaded on first use, after torch (so that it binds to the HIP runtime torch already
loaded: both name the runtime by the soname libamdhip64.so.7). There is no fallback: a missing
library or a non-zero status raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded first: the library then shares torch's HIP runtime)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liba8attn.so")

A8_EINVAL, A8_EALIGN, A8_EUNSUP, A8_EWSPACE = -1, -2, -3, -4

_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_IP = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); mirrors include/a8attn.h
SIGNATURES = {
    "a8_version": (ctypes.c_char_p, []),
    "a8_last_error": (ctypes.c_char_p, []),
    "a8_hip_runtime_path": (ctypes.c_char_p, []),
    "a8_bias_rope_store": (_I, [_P, _L, _P, _P, _P, _L, _I, _P, _P, _I, _P, _L, _L,
                                _P, _P, _L, _L, _L, _I, _I, _I, _I, _I, _I, _P]),
    "a8_decode_attn": (_I, [_P, _L, _L, _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L,
                            _P, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "a8_decode_attn_noalloc": (_I, [_P, _L, _L, _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L,
                                    _I, _I, _I, _I, _I, _I, _F, _P]),
    "a8_decode_choose": (_I, [_I, _I, _I, _I, _I, _L, _I, _IP, _IP]),
    "a8_decode_attn_stream": (_I, [_P, _L, _L, _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L,
                                   _P, _P, _L, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "a8_decode_choose_stream": (_I, [_I, _I, _I, _L, _I, _IP, _IP, _IP]),
    "a8_store_decode_stream": (_I, [_P, _L, _P, _P, _P, _L, _I, _P, _P, _P, _L, _L,
                                    _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L,
                                    _P, _P, _L, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "a8_store_decode_split": (_I, [_P, _L, _P, _P, _P, _L, _I, _P, _P, _P, _L, _L,
                                   _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L,
                                   _P, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "a8_decode_attn_flat": (_I, [_P, _L, _L, _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L,
                                 _P, _P, _L, _P, _L, _I, _I, _I, _I, _I, _F, _P]),
    "a8_rmsnorm": (_I, [_P, _L, _P, _L, _P, _P, _L, _P, _L, _I, _I, _F, _P]),
    "a8_silu_mul": (_I, [_P, _L, _P, _L, _I, _I, _P]),
    "a8_gemm_small": (_I, [_P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _P]),
    "a8_conv_cl": (_I, [_P, _L, _L, _P, _L, _L, _L, _I, _P, _P, _L, _L, _P, _L, _L, _P, _P,
                        _I, _I, _I, _I, _I, _I, _I, _I, _P, _L, _P]),
    "a8_conv_cl_ws_bytes": (_L, [_I, _I, _I, _I, _I, _I]),
    "a8_snake_cat": (_I, [_P, _L, _L, _P, _L, _L, _P, _P, _P, _L, _L, _I, _I, _I, _I, _P]),
    "a8_snake_cat_refresh": (_I, [_P, _L, _L, _P, _L, _L, _P, _P, _P, _L, _L, _I, _I, _I, _I, _P]),
    "a8_decode_attn_f32q": (_I, [_P, _L, _L, _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L, _I, _I, _I, _I, _I,
                                 _F, _P]),
    "a8_gemm_silu_small": (_I, [_P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _P]),
    "a8_conv_out_tanh": (_I, [_P, _L, _L, _P, _L, _L, _P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P]),
    "a8_gemm_small_norm": (_I, [_P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _F, _P]),
    "a8_gemm_small_norm_pf": (_I, [_P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _F,
                                   _P, _L, _P, _I, _P]),
    "a8_ru_cl": (_I, [_P, _L, _L, _P, _L, _L, _P, _P, _P, _P, _P, _P, _L, _L, _P, _L, _L, _I, _I, _I, _I, _I, _I,
                      _P]),
    "a8_prefix_copy": (_I, [_P, _P, _L, _L, _L, _P, _P, _L, _L, _L, _L, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "a8_decode_choose_flat": (_I, [_I, _I, _I, _L, _I, _IP]),
    "a8_store_decode_flat": (_I, [_P, _L, _P, _P, _P, _L, _I, _P, _P, _P, _L, _L,
                                  _P, _P, _L, _L, _L, _I, _I, _P, _P, _P, _L, _L,
                                  _P, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I, _F, _P]),
    "a8_prefill_attn": (_I, [_P, _L, _L, _I, _P, _P, _L, _L, _L, _I, _I, _P, _L, _L,
                             _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
    "a8_prefill_attn_qkv": (_I, [_P, _L, _P, _P, _P, _L, _I, _I, _P, _P, _L, _L, _L, _I, _I, _P, _L, _L,
                                 _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
}

_lock = threading.Lock()
_lib = None


class A8Error(RuntimeError):
    """A HIP launch of the library failed (positive hipError_t status)."""


def load() -> ctypes.CDLL:
    """The loaded library (loads it on the first call). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(f"{LIB_PATH} is missing: build it with `python __graft_entry__.py build` "
                                  "(or __graft_entry__.build()) before using the HIP kernels")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Raise the Python error matching a C-ABI status (0 = ok)."""
    if status == 0:
        return
    if status < 0:
        msg = load().a8_last_error().decode(errors="replace")
        if status == A8_EUNSUP:
            raise NotImplementedError(f"{what}: {msg}")
        if status == A8_EWSPACE:
            raise AssertionError(f"{what}: {msg}")
        raise ValueError(f"{what}: {msg}")
    raise A8Error(f"{what}: HIP error {status}")


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t (as an int) of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def version() -> str:
    return load().a8_version().decode()


def runtime_path() -> str:
    return load().a8_hip_runtime_path().decode()
