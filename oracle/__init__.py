"""CPU oracle for the MLX affine group-quantized linear path (ctypes + numpy).

TEST INFRASTRUCTURE ONLY. This package is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and never as the thing measured or shipped. The product path
(``higgs_amd``) does not import it.

The C restatement lives in ``oracle/hq_oracle.c``; each function there cites the
reference file:line it follows. This wrapper only moves numpy arrays across
the C boundary. Arrays of bfloat16 / float16 values are carried as ``uint16``
bit patterns (numpy has no bfloat16); ``dtype`` codes are 0 = float32,
1 = float16, 2 = bfloat16, as in ``include/higgs_qmm.h``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

F32, F16, BF16 = 0, 1, 2

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libhq_oracle.so")
_lib = None

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p


def build() -> None:
    """Compile oracle/hq_oracle.c into oracle/libhq_oracle.so."""
    subprocess.check_call([os.path.join(_HERE, "build_oracle.sh")])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.hqo_f32_to_bf16.restype = ctypes.c_uint16
        L.hqo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.hqo_f32_to_f16.restype = ctypes.c_uint16
        L.hqo_f32_to_f16.argtypes = [ctypes.c_float]
        L.hqo_bf16_to_f32.restype = ctypes.c_float
        L.hqo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.hqo_f16_to_f32.restype = ctypes.c_float
        L.hqo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.hqo_round_f64.restype = ctypes.c_float
        L.hqo_round_f64.argtypes = [ctypes.c_double, _int]
        L.hqo_to_f32.argtypes = [_vp, _int, _i64, _vp]
        L.hqo_from_f32.argtypes = [_vp, _i64, _int, _vp]
        L.hqo_pack.argtypes = [_vp, _i64, _i64, _int, _vp]
        L.hqo_unpack.argtypes = [_vp, _i64, _i64, _int, _vp]
        L.hqo_dequantize.argtypes = [_vp, _vp, _vp, _i64, _i64, _int, _int, _int, _int, _vp]
        L.hqo_qmm_f64.argtypes = [_vp, _int, _vp, _vp, _vp, _int, _i64, _i64, _i64,
                                  _int, _int, _int, _vp]
        L.hqo_qmm_mlx.argtypes = [_vp, _int, _vp, _vp, _vp, _int, _i64, _i64, _i64,
                                  _int, _int, _int, _vp]
        L.hqo_gather_qmm_f64.argtypes = [_vp, _int, _vp, _vp, _vp, _int, _vp, _vp,
                                         _i64, _i64, _i64, _i64, _i64, _i64, _int,
                                         _int, _int, _vp]
        L.hqo_gather_sort.argtypes = [_vp, _i64, _i64, _vp, _vp, _vp, _vp]
        L.hqo_swiglu.argtypes = [_vp, _vp, _int, _i64, _vp]
        L.hqo_moe_combine.argtypes = [_vp, _int, _vp, _vp, _int, _i64, _i64, _i64, _vp]
        L.hqo_quantize.argtypes = [_vp, _int, _i64, _i64, _int, _int, _vp, _vp, _vp]
        L.hqo_num_threads.restype = _int
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(_vp)


def _dt_of(a: np.ndarray, dtype: int | None) -> int:
    if dtype is not None:
        return dtype
    if a.dtype == np.float32:
        return F32
    raise ValueError("16-bit arrays are uint16 bit patterns: pass dtype explicitly")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (rc={rc})")


# --- conversions -----------------------------------------------------------

def to_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, np.float32)
    lib().hqo_to_f32(_p(a), dtype, a.size, _p(out))
    return out


def from_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.float32 if dtype == F32 else np.uint16)
    lib().hqo_from_f32(_p(a), a.size, dtype, _p(out))
    return out


def round_f64(v: float, dtype: int) -> float:
    return float(lib().hqo_round_f64(float(v), dtype))


# --- packing ---------------------------------------------------------------

def pack(q: np.ndarray, bits: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint32)
    rows, cols = q.reshape(-1, q.shape[-1]).shape
    if (cols * bits) % 32:
        raise ValueError("cols*bits must be a multiple of 32")
    w = np.empty(q.shape[:-1] + (cols * bits // 32,), np.uint32)
    lib().hqo_pack(_p(q), rows, cols, bits, _p(w))
    return w


def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    P = w.shape[-1]
    cols = P * 32 // bits
    rows = w.size // P if P else 0
    q = np.empty(w.shape[:-1] + (cols,), np.uint32)
    lib().hqo_unpack(_p(w), rows, cols, bits, _p(q))
    return q


# --- dequantize / matmul ---------------------------------------------------

def dequantize(w, scales, biases, group_size, bits, dtype, fused=False) -> np.ndarray:
    """Returns the dequantized matrix in `dtype` (uint16 bits for 16-bit)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = np.ascontiguousarray(biases)
    K = w.shape[-1] * 32 // bits
    rows = w.size // w.shape[-1]
    out = np.empty(w.shape[:-1] + (K,), np.float32 if dtype == F32 else np.uint16)
    _check(lib().hqo_dequantize(_p(w), _p(scales), _p(biases), rows, K, group_size,
                                bits, dtype, int(fused), _p(out)), "dequantize")
    return out


def qmm_f64(x, x_dtype, w, scales, biases, s_dtype, group_size, bits, transpose=True):
    """Exact fp64 reference of quantized_matmul for x [M, K] (2-D)."""
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = np.ascontiguousarray(biases)
    M, K = x.shape
    if transpose:
        N = w.shape[0]
    else:
        N = w.shape[1] * 32 // bits
    y = np.empty((M, N), np.float64)
    _check(lib().hqo_qmm_f64(_p(x), x_dtype, _p(w), _p(scales), _p(biases), s_dtype,
                             M, N, K, int(transpose), group_size, bits, _p(y)), "qmm_f64")
    return y


def result_dtype(x_dtype: int, s_dtype: int) -> int:
    return x_dtype if x_dtype == s_dtype else F32


def qmm_mlx(x, x_dtype, w, scales, biases, s_dtype, group_size, bits, threads=0):
    """MLX-CPU-style quantized_matmul (transpose=True), the timed CPU baseline."""
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = np.ascontiguousarray(biases)
    M, K = x.shape
    N = w.shape[0]
    T = result_dtype(x_dtype, s_dtype)
    y = np.empty((M, N), np.float32 if T == F32 else np.uint16)
    _check(lib().hqo_qmm_mlx(_p(x), x_dtype, _p(w), _p(scales), _p(biases), s_dtype,
                             M, N, K, group_size, bits, threads, _p(y)), "qmm_mlx")
    return y


def gather_qmm_f64(x, x_dtype, w, scales, biases, s_dtype, lhs, rhs, M, N, K,
                   group_size, bits, transpose=True, x_batch=None, w_batch=None):
    """fp64 gather_qmm with flattened, already-broadcast indices.

    x: [x_batch, M, K]; w: [w_batch, rows, P]; rhs: [batch] u32; lhs: [batch]
    u32 or None (None = x batch element i // (batch // x_batch)). Returns
    [batch, M, N] float64 (NaN rows for out-of-range indices).
    """
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = np.ascontiguousarray(biases)
    rhs = np.ascontiguousarray(rhs, dtype=np.uint32)
    if lhs is not None:
        lhs = np.ascontiguousarray(lhs, dtype=np.uint32)
    batch = rhs.size
    if x_batch is None:
        x_batch = x.size // (M * K)
    if w_batch is None:
        w_batch = w.shape[0]
    y = np.empty((batch, M, N), np.float64)
    _check(lib().hqo_gather_qmm_f64(_p(x), x_dtype, _p(w), _p(scales), _p(biases),
                                    s_dtype, _p(lhs), _p(rhs), batch, x_batch, w_batch,
                                    M, N, K, int(transpose), group_size, bits, _p(y)),
           "gather_qmm_f64")
    return y


def gather_sort(idx: np.ndarray, top_k: int):
    """Returns (order, inv_order, idx_sorted, token_idx) as uint32 arrays."""
    idx = np.ascontiguousarray(idx, dtype=np.uint32).reshape(-1)
    n = idx.size
    order = np.empty(n, np.uint32)
    inv = np.empty(n, np.uint32)
    srt = np.empty(n, np.uint32)
    tok = np.empty(n, np.uint32)
    lib().hqo_gather_sort(_p(idx), n, top_k, _p(order), _p(inv), _p(srt), _p(tok))
    return order, inv, srt, tok


def swiglu(gate: np.ndarray, up: np.ndarray, dtype: int) -> np.ndarray:
    gate = np.ascontiguousarray(gate)
    up = np.ascontiguousarray(up)
    out = np.empty(gate.shape, gate.dtype)
    lib().hqo_swiglu(_p(gate), _p(up), dtype, gate.size, _p(out))
    return out


def moe_combine(y: np.ndarray, dtype: int, inv: np.ndarray, scores: np.ndarray,
                sdtype: int) -> np.ndarray:
    """out[t] = round(sum_j round(scores[t, j] * y[inv[t*k + j]])); y [n, D]
    (bit patterns of dtype), scores [tokens, k]. Returns [tokens, D] of dtype."""
    y = np.ascontiguousarray(y)
    scores = np.ascontiguousarray(scores)
    inv = np.ascontiguousarray(inv, dtype=np.uint32).reshape(-1)
    tokens, top_k = scores.shape
    D = y.shape[-1]
    out = np.empty((tokens, D), y.dtype)
    lib().hqo_moe_combine(_p(y), dtype, _p(inv), _p(scores), sdtype, tokens, top_k, D, _p(out))
    return out


def quantize(w: np.ndarray, dtype: int, group_size: int, bits: int):
    """MLX affine quantize of w [..., K] (float32 values, or uint16 bit patterns
    of a 16-bit dtype). Returns (wq u32 [..., K*bits/32], scales, biases
    [..., K/group_size] in dtype)."""
    w = np.ascontiguousarray(w)
    K = w.shape[-1]
    rows = w.size // K if K else 0
    G = K // group_size
    wq = np.empty(w.shape[:-1] + (K * bits // 32,), np.uint32)
    sdt = np.float32 if dtype == F32 else np.uint16
    s = np.empty(w.shape[:-1] + (G,), sdt)
    b = np.empty(w.shape[:-1] + (G,), sdt)
    _check(lib().hqo_quantize(_p(w), dtype, rows, K, group_size, bits, _p(wq), _p(s), _p(b)),
           "quantize")
    return wq, s, b


def num_threads() -> int:
    return int(lib().hqo_num_threads())
