"""ctypes binding of libhiggs_qmm.so (the C ABI in include/higgs_qmm.h).

The library is the product; there is no fallback. If the .so is missing,
loading raises immediately (build it with ``python -m higgs_amd.build`` or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhiggs_qmm.so")

HQ_OK = 0
HQ_ERR_INVALID_ARGUMENT = 1
HQ_ERR_UNSUPPORTED = 2
HQ_ERR_HIP = 3

DTYPE_FLOAT32, DTYPE_FLOAT16, DTYPE_BFLOAT16 = 0, 1, 2

# Every symbol include/higgs_qmm.h declares, with its ctypes signature.
_vp, _i64, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "hq_version": (ctypes.c_char_p, []),
    "hq_last_error": (ctypes.c_char_p, []),
    "hq_result_dtype": (_int, [_int, _int]),
    "hq_quantized_matmul": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int,
                                   _int, _int, _int, _vp]),
    "hq_gather_qmm": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                             _i64, _int, _int, _int, _int, _int, _int, _vp]),
    "hq_quantized_linear": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int,
                                   _int, _int, _int, _vp]),
    "hq_dequantize": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _int, _vp]),
    "hq_quantize": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _int, _vp]),
    "hq_embedding_dequantize": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int,
                                       _int, _vp]),
    "hq_quantized_matmul_swiglu": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                          _i64, _int, _int, _int, _int, _vp]),
    "hq_gather_qmm_swiglu": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                    _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _vp]),
    "hq_swiglu": (_int, [_vp, _vp, _vp, _i64, _int, _vp]),
    "hq_moe_sort": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "hq_moe_combine": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp]),
}


class HiggsQmmError(RuntimeError):
    """A call through the C ABI failed; ``status`` is the hq_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(
                        f"{LIB_PATH} is missing: build the HIP library first "
                        "(python -m higgs_amd.build)")
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def last_error() -> str:
    return lib().hq_last_error().decode()


def check(status: int) -> None:
    if status != HQ_OK:
        raise HiggsQmmError(status, last_error())


def version() -> str:
    return lib().hq_version().decode()
