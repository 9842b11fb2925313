"""ctypes binding of libgdn2_hip.so (the C ABI in include/gdn2_hip.h).

The library is loaded lazily on first use. If it is missing the call raises
immediately -- there is no fallback path on the GPU.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libgdn2_hip.so")
_lock = threading.Lock()
_lib = None

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

# name -> (restype, argtypes); must match include/gdn2_hip.h
_P, _I, _L, _F, _S = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "gdn2_hip_version": (_I, []),
    "gdn2_hip_status_string": (ctypes.c_char_p, [_I]),
    "gdn2_hip_decode": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _L, _L, _L, _F, _P]),
    "gdn2_hip_prefill_workspace_bytes": (_S, [_I, _I, _I, _L]),
    "gdn2_hip_chunk_local": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _L, _L, _L, _F, _P]),
    "gdn2_hip_prefill_scan": (_I, [_P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _L, _L, _L, _P]),
    "gdn2_hip_prefill_chunks": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I,
                                     _L, _L, _L, _F, _P]),
    "gdn2_hip_prefill_chunks_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                             _L, _L, _L, _F, _P]),
    "gdn2_hip_prefill_varlen_workspace_bytes": (_S, [_I, _I, _I, _L]),
    "gdn2_hip_prefill_varlen": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I,
                                     _L, _F, _P]),
    "gdn2_hip_layer_prologue": (_I, [_P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _L, _I, _P, _P, _I, _P, _P,
                                     _P, _P, _F, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _I, _P]),
    "gdn2_hip_layer_prologue_varlen": (_I, [_P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _L, _I, _P, _P, _I, _P,
                                            _P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _I,
                                            _P]),
    "gdn2_hip_layer_epilogue": (_I, [_P, _I, _P, _L, _P, _F, _P, _I, _L, _I, _L, _I, _I, _P]),
    "gdn2_hip_gemv": (_I, [_P, _L, _P, _P, _L, _I, _I, _I, _I, _P]),
    "gdn2_hip_layer_decode_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _I, _I]),
    "gdn2_hip_backward_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _L]),
    "gdn2_hip_backward": (_I, [_P, _P, _P, _P, _P, _P, _I, _F, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _I, _L, _I, _I, _I, _I, _P]),
    "gdn2_hip_backward_varlen_workspace_bytes": (_S, [_I, _I, _I, _I, _I, _L]),
    "gdn2_hip_backward_varlen": (_I, [_P, _P, _P, _P, _P, _P, _I, _F, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                                      _P, _P, _I, _L, _I, _I, _I, _I, _P]),
    "gdn2_hip_layer_decode": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _P, _F, _P, _P, _F, _P, _P, _P, _I, _I,
                                   _I, _I, _I, _I, _I, _I, _F, _P]),
}


def library_path() -> str:
    return _LIB_PATH


def lib():
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(_LIB_PATH):
                    raise RuntimeError(
                        f"{_LIB_PATH} is missing: build it with `python -m gdt2_tilelang_amd.build` "
                        "(the hip backend has no fallback)")
                handle = ctypes.CDLL(_LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().gdn2_hip_status_string(status).decode()
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; use float16, bfloat16 or float32") from None
