"""ctypes binding to libvbhip.so (the C ABI declared in include/vbhip.h).

There is no CPU fallback: if the library is missing or no gfx950 GPU is
visible, every op raises.  ``ctypes.CDLL`` releases the GIL during calls.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvbhip.so")

VB_OK = 0
VB_E_INVAL = -1
VB_E_UNSUPPORTED = -2
VB_E_HIP = -3
VB_E_NOMEM = -4

_vp, _i64, _i32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t

# name -> (restype, argtypes); every symbol here is declared in include/vbhip.h
SIGNATURES = {
    "vb_last_error": (ctypes.c_char_p, []),
    "vb_version": (ctypes.c_int, []),
    "vb_row_bytes": (_i64, [_i32, _i64]),
    "vb_init": (ctypes.c_int, [ctypes.c_int]),
    "vb_tuning_reload": (ctypes.c_int, []),
    "vb_malloc": (ctypes.c_int, [ctypes.POINTER(_vp), _sz]),
    "vb_free": (ctypes.c_int, [_vp]),
    "vb_memcpy_h2d": (ctypes.c_int, [_vp, _vp, _sz, _vp]),
    "vb_memcpy_d2h": (ctypes.c_int, [_vp, _vp, _sz, _vp]),
    "vb_stream_create": (ctypes.c_int, [ctypes.POINTER(_vp)]),
    "vb_stream_sync": (ctypes.c_int, [_vp]),
    "vb_stream_destroy": (ctypes.c_int, [_vp]),
    "vb_dequant_rows": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _vp]),
    "vb_quantize_rows": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _vp]),
    "vb_embed_rows": (ctypes.c_int, [_vp, _i32, _i64, _i64, _vp, _i64, _vp, _vp]),
    "vb_gemv": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "vb_gemm": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i64, _i64, _i64, _i32, _i32, _vp]),
    "vb_gemm_workspace": (_i64, [_i64, _i64, _i64, _i32, _i32, _i32]),
    "vb_stream_read": (ctypes.c_int, [_vp, _i64, _i64, _i32, _vp, _vp]),
    "vb_gemm_ws": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i64, _i64, _i64, _i32, _i32, _vp, _sz, _vp]),
    "vb_sparse_ffn_workspace": (_i64, [_i64, _i64, _i32, _i32]),
    "vb_sparse_ffn": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _vp, _i64, _i64, _i32,
                                     _vp, _sz, _vp]),
    "vb_sparse_ffn_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _vp, _i64, _i64, _i32,
                                             _vp]),
    "vb_ffn_block_workspace": (_i64, [_i64, _i64]),
    "vb_ffn_block": (ctypes.c_int, [_vp, _vp, ctypes.c_float, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i32,
                                    _i32, _vp, _vp, _sz, _vp]),
    "vb_sparse_ffn_block": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _vp, ctypes.c_float, _vp, _i32, _vp, _i32,
                                           _i32, _vp, _i64, _i64, _i32, _vp, _sz, _vp]),
    "vb_ema_update": (ctypes.c_int, [_vp, _i64, _vp, ctypes.c_double, _vp]),
    "vb_ema_predict": (ctypes.c_int, [_vp, _vp, _i64, _i32, ctypes.c_float, _i32, _i32, _vp, _vp, _vp, _vp]),
    "vb_topk_indices": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp]),
    "vb_moe_workspace": (_i64, [_i32, _i32, _i64, _i64]),
    "vb_moe_grouped_ffn": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _i64,
                                          _i64, _i32, _vp, _sz, _vp]),
    "vb_moe_grouped_ffn_types": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp,
                                                _i64, _i64, _i32, _i32, _vp, _sz, _vp]),
    "vb_moe_route": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "vb_activation": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp]),
    "vb_rms_norm": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp]),
    "vb_softmax": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp]),
    "vb_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "vb_gguf_close": (ctypes.c_int, [_vp]),
    "vb_gguf_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64),
                                    ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "vb_gguf_n_tensors": (_i64, [_vp]),
    "vb_gguf_find_tensor": (_i64, [_vp, ctypes.c_char_p]),
    "vb_gguf_tensor_info": (ctypes.c_int, [_vp, _i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i32),
                                           ctypes.POINTER(_i32), ctypes.POINTER(_i64),
                                           ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "vb_gguf_tensor_data": (ctypes.c_int, [_vp, _i64, ctypes.POINTER(_vp)]),
    "vb_gguf_upload": (ctypes.c_int, [_vp, _i64, _vp, _vp]),
    "vb_gguf_n_kv": (_i64, [_vp]),
    "vb_gguf_find_kv": (_i64, [_vp, ctypes.c_char_p]),
    "vb_gguf_kv_info": (ctypes.c_int, [_vp, _i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i32),
                                       ctypes.POINTER(_i32), ctypes.POINTER(ctypes.c_uint64)]),
    "vb_gguf_kv_int": (ctypes.c_int, [_vp, _i64, ctypes.c_uint64, ctypes.POINTER(_i64)]),
    "vb_gguf_kv_float": (ctypes.c_int, [_vp, _i64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)]),
    "vb_gguf_kv_str": (ctypes.c_int, [_vp, _i64, ctypes.c_uint64, ctypes.POINTER(_vp),
                                      ctypes.POINTER(ctypes.c_uint64)]),
}

_lib = None
_lock = threading.Lock()
_inited = set()


class VBError(RuntimeError):
    """A libvbhip call failed (the reference raises RuntimeError for the same
    conditions: cpp/src/dequant.cpp:423, cpp/src/cuda_kernels.cu:24-31)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load libvbhip.so; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m vibeblade_amd.build`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    return load().vb_last_error().decode(errors="replace")


def check(fn_name: str, rc: int) -> None:
    if rc != VB_OK:
        err = last_error()
        if rc == VB_E_INVAL:
            raise ValueError(f"{fn_name}: {err}")
        raise VBError(fn_name, rc, err)


def call(fn_name: str, *args) -> None:
    check(fn_name, getattr(load(), fn_name)(*args))


def init(device: int = 0) -> None:
    """vb_init once per device (checks that it is a gfx950)."""
    if device in _inited:
        return
    call("vb_init", device)
    _inited.add(device)
