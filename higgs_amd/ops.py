"""Host-side facade of the quantized-linear path over the C ABI.

Mirrors the mlx-rs operator interface that higgs' model layers call, with the
same argument names, meanings and validation messages:

* ``quantized_matmul(x, w, scales, biases, transpose, group_size, bits)`` --
  mlx-rs ``ops::quantized_matmul`` (crates/higgs-models/src/qwen3_next.rs:
  218-227; every mlx-rs ``QuantizedLinear``, transformer.rs:148-157).
* ``gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices, transpose,
  group_size, bits, sorted_indices)`` -- ``mlx_gather_qmm`` as wrapped by
  higgs' ``gather_qmm`` (qwen3_next.rs:509-578).
* ``dequantize(w, scales, biases, group_size, bits)`` -- mlx-rs
  ``ops::dequantize`` (qwen3_next.rs:314).
* ``quantize(w, group_size, bits)`` -- mlx-rs ``ops::quantize``
  (qwen3_next.rs:4305-4307, 12942; ``nn::quantize`` at transformer.rs:954-965).
* ``quantized_linear(x, w, scales, biases, bias, group_size, bits)`` -- mlx-rs
  ``QuantizedLinear::forward`` (quantized_matmul, then + bias when the layer
  has one: the Qwen2 q/k/v projections, transformer.rs:180-191).
* ``dense_hidden_fused`` -- ``FfnBlock::dense_hidden_fused``
  (qwen3_next.rs:2539-2585): gate/up projection and SwiGLU in one launch.
* ``forward_gather_global_sort`` / ``moe_block`` -- the MoE experts on the
  global-sort path (qwen3_next.rs:1731-1809; qwen3_moe.rs:353-357), from the
  building blocks ``moe_sort``, ``gather_qmm_swiglu``, ``gather_qmm`` and
  ``moe_combine``.

Tensors are torch tensors on the GPU: torch provides device memory and the
current HIP stream, and the arithmetic runs in libhiggs_qmm.so. Packed weights
are ``torch.uint32`` or ``torch.int32`` (same bits). There is no CPU fallback:
CPU tensors are rejected.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import HiggsQmmError

_DT = {torch.float32: _lib.DTYPE_FLOAT32, torch.float16: _lib.DTYPE_FLOAT16,
       torch.bfloat16: _lib.DTYPE_BFLOAT16}
_TORCH_DT = {v: k for k, v in _DT.items()}
_WORD_DTYPES = (torch.int32, getattr(torch, "uint32", torch.int32))
_INDEX_DTYPES = (torch.int32, getattr(torch, "uint32", torch.int32), torch.int64)

SUPPORTED_BITS = (2, 3, 4, 5, 6, 8)
SUPPORTED_GROUP_SIZES = (32, 64, 128)


def _err(msg: str, status: int = _lib.HQ_ERR_INVALID_ARGUMENT) -> HiggsQmmError:
    return HiggsQmmError(status, msg)


def _shape(t: torch.Tensor) -> str:
    return "(" + ",".join(str(d) for d in t.shape) + ")"


def _dt_name(t: torch.Tensor) -> str:
    return str(t.dtype).replace("torch.", "")


def _check_params(tag: str, group_size: int, bits: int) -> None:
    if bits not in SUPPORTED_BITS:
        raise _err(f"[{tag}] The requested number of bits {bits} is not supported. "
                   "The supported bits are 2, 3, 4, 5, 6 and 8.")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise _err(f"[{tag}] The requested group size {group_size} is not supported. "
                   "The supported group sizes are 32, 64, and 128.")


def _check_device(tag: str, *ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise _err(f"[{tag}] All arrays must live on the GPU (got a tensor on {t.device}).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise _err(f"[{tag}] All arrays must be on the same device.")
    return dev


def _words(tag: str, w: torch.Tensor) -> torch.Tensor:
    if w.dtype not in _WORD_DTYPES:
        raise _err(f"[{tag}] The weight matrix should be uint32 but received {_dt_name(w)}")
    return w.contiguous()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def result_dtype(x_dtype: torch.dtype, s_dtype: torch.dtype) -> torch.dtype:
    """MLX promotion of the activation and scale dtypes (mixed -> float32)."""
    return x_dtype if x_dtype == s_dtype else torch.float32


def _extract_dims(tag, x, w, scales, biases, transpose, group_size, bits):
    """MLX's extract_quantized_matmul_dims: returns (w_inner, w_outer)."""
    w = _words(tag, w)
    if scales.shape != biases.shape:
        raise _err(f"[{tag}] Scales and biases should have the same shape. Received scales "
                   f"with shape {_shape(scales)} and biases with {_shape(biases)}.")
    if w.dim() < 2 or scales.dim() != w.dim() or tuple(w.shape[:-2]) != tuple(scales.shape[:-2]):
        raise _err(f"[{tag}] Weight, scales and biases should have the same batch shape. "
                   f"Received weight with shape {_shape(w)}, scales with {_shape(scales)} "
                   f"and biases with {_shape(biases)}.")
    if w.shape[-1] * 32 // bits != scales.shape[-1] * group_size or \
            w.shape[-1] * 32 % bits or w.shape[-2] != scales.shape[-2]:
        raise _err(f"[{tag}] The shapes of the weight and scales are incompatible based on bits "
                   f"and group_size. w.shape() == {_shape(w)} and scales.shape() == "
                   f"{_shape(scales)} with group_size={group_size} and bits={bits}")
    w_inner = w.shape[-1] * 32 // bits if transpose else w.shape[-2]
    w_outer = w.shape[-2] if transpose else w.shape[-1] * 32 // bits
    if x.shape[-1] != w_inner:
        raise _err(f"[{tag}] Last dimension of first input with shape (..., {x.shape[-1]}) does "
                   f"not match the expanded quantized matrix ({w_inner}, {w_outer}) computed "
                   f"from shape {_shape(w)} with group_size={group_size}, bits={bits} and "
                   f"transpose={str(bool(transpose)).lower()}")
    for t, name in ((x, "x"), (scales, "scales"), (biases, "biases")):
        if t.dtype not in _DT:
            raise _err(f"[{tag}] Only real floating types are supported but x.dtype() == "
                       f"{_dt_name(x)}, scales.dtype() == {_dt_name(scales)} and "
                       f"biases.dtype() == {_dt_name(biases)}")
    if scales.dtype != biases.dtype:
        raise _err(f"[{tag}] scales and biases must share a dtype (got {_dt_name(scales)} and "
                   f"{_dt_name(biases)}).")
    return w, w_inner, w_outer


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, transpose: bool = True, group_size: int = 64,
                     bits: int = 4) -> torch.Tensor:
    """y = x @ deq(w).T (transpose) or x @ deq(w); x is [..., K].

    A 2-D ``w`` is one product with all of x's leading dims flattened into M.
    A batched ``w`` ([..., N, P]) broadcasts its batch dims against x's, as MLX
    does, and runs through the gather kernel with default indices.
    """
    tag = "quantized_matmul"
    _check_params(tag, group_size, bits)
    if x.dim() < 1:
        raise _err(f"[{tag}] x must have at least one dimension.")
    w, w_inner, w_outer = _extract_dims(tag, x, w, scales, biases, transpose, group_size, bits)
    dev = _check_device(tag, x, w, scales, biases)
    out_dtype = result_dtype(x.dtype, scales.dtype)
    if w.dim() > 2:
        if x.dim() < 2:
            x = x.unsqueeze(0)
        return gather_qmm(x, w, scales, biases, None, None, transpose, group_size, bits, False)
    x = x.contiguous()
    scales = scales.contiguous()
    biases = biases.contiguous()
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    y = torch.empty((*x.shape[:-1], w_outer), dtype=out_dtype, device=dev)
    _lib.check(_lib.lib().hq_quantized_matmul(
        _ptr(y), _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), M, w_outer, K,
        int(bool(transpose)), group_size, bits, _DT[x.dtype], _DT[scales.dtype], _stream(dev)))
    return y


def quantized_linear(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, bias: Optional[torch.Tensor] = None,
                     group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """y = x @ deq(w).T + bias for a 2-D ``w`` [N, P]; ``bias`` [N] or None.

    The product is rounded to the output dtype, then the bias is added and the
    sum rounded (mlx-rs QuantizedLinear: quantized_matmul, then add), in the
    kernel's epilogue. The bias must have the product's output dtype.
    """
    tag = "quantized_linear"
    if bias is None:
        return quantized_matmul(x, w, scales, biases, True, group_size, bits)
    _check_params(tag, group_size, bits)
    if x.dim() < 1:
        raise _err(f"[{tag}] x must have at least one dimension.")
    w, w_inner, w_outer = _extract_dims(tag, x, w, scales, biases, True, group_size, bits)
    if w.dim() != 2:
        raise _err(f"[{tag}] The weight of a linear layer is 2-D (got {_shape(w)}).")
    out_dtype = result_dtype(x.dtype, scales.dtype)
    if tuple(bias.shape) != (w_outer,):
        raise _err(f"[{tag}] The bias must have shape ({w_outer},) (got {_shape(bias)}).")
    if bias.dtype != out_dtype:
        raise _err(f"[{tag}] The bias dtype ({_dt_name(bias)}) must be the output dtype "
                   f"{str(out_dtype).replace('torch.', '')}.", _lib.HQ_ERR_UNSUPPORTED)
    dev = _check_device(tag, x, w, scales, biases, bias)
    x = x.contiguous()
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    y = torch.empty((*x.shape[:-1], w_outer), dtype=out_dtype, device=dev)
    _lib.check(_lib.lib().hq_quantized_linear(
        _ptr(y), _ptr(x), _ptr(w), _ptr(scales.contiguous()), _ptr(biases.contiguous()),
        _ptr(bias.contiguous()), M, w_outer, K, group_size, bits, _DT[x.dtype],
        _DT[scales.dtype], _DT[bias.dtype], _stream(dev)))
    return y


def _prefix_broadcast(x_batch_shape: Sequence[int], out_shape: Sequence[int]) -> bool:
    """True if x's batch dims, right-aligned to out_shape, equal a prefix of out_shape
    followed only by 1s -- then x batch element = flat_out_index // (batch/x_batch)."""
    nd = len(out_shape)
    if len(x_batch_shape) > nd:
        return False
    xs = [1] * (nd - len(x_batch_shape)) + list(x_batch_shape)
    j = nd
    while j > 0 and xs[j - 1] == 1:
        j -= 1
    return all(xs[i] == out_shape[i] for i in range(j))


def _as_u32_indices(tag: str, idx: torch.Tensor, name: str) -> torch.Tensor:
    if idx.dtype not in _INDEX_DTYPES:
        raise _err(f"[{tag}] {name} must be an integer array (got {_dt_name(idx)}).")
    if idx.dtype == torch.int64:
        idx = idx.to(torch.int32)
    return idx.contiguous()


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               lhs_indices: Optional[torch.Tensor] = None,
               rhs_indices: Optional[torch.Tensor] = None, transpose: bool = True,
               group_size: int = 64, bits: int = 4,
               sorted_indices: bool = False) -> torch.Tensor:
    """MLX gather_qmm: out[b] = x[lhs[b]] @ deq(w[rhs[b]]).T for the broadcast of
    lhs_indices and rhs_indices; x is [..., M, K], w is [..., N, P].

    Output shape: broadcast(lhs, rhs).shape + [M, N]. Missing indices default to
    an arange over the batch dims of x (lhs) or w (rhs), as MLX does.
    """
    tag = "gather_qmm"
    _check_params(tag, group_size, bits)
    if x.dim() < 2 or w.dim() < 2:
        raise _err(f"[{tag}] x and w must have at least two dimensions.")
    w, w_inner, w_outer = _extract_dims(tag, x, w, scales, biases, transpose, group_size, bits)
    dev = _check_device(tag, x, w, scales, biases, lhs_indices, rhs_indices)
    x_batch_shape = tuple(x.shape[:-2])
    w_batch_shape = tuple(w.shape[:-2])
    x_batch = math.prod(x_batch_shape)
    w_batch = math.prod(w_batch_shape)
    M, K = x.shape[-2], x.shape[-1]
    N = w_outer
    if rhs_indices is None:
        rhs = torch.arange(w_batch, dtype=torch.int32, device=dev).reshape(w_batch_shape)
    else:
        rhs = _as_u32_indices(tag, rhs_indices, "rhs_indices")
    lhs = None if lhs_indices is None else _as_u32_indices(tag, lhs_indices, "lhs_indices")
    lhs_shape = x_batch_shape if lhs is None else tuple(lhs.shape)
    try:
        out_batch = tuple(torch.broadcast_shapes(lhs_shape, tuple(rhs.shape)))
    except RuntimeError:
        raise _err(f"[{tag}] Cannot broadcast lhs indices with shape {lhs_shape} and rhs "
                   f"indices with shape {tuple(rhs.shape)}.") from None
    batch = math.prod(out_batch)
    out_dtype = result_dtype(x.dtype, scales.dtype)
    y = torch.empty((*out_batch, M, N), dtype=out_dtype, device=dev)
    if y.numel() == 0:
        return y
    rhs_flat = rhs.expand(out_batch).contiguous().reshape(-1)
    if lhs is None and _prefix_broadcast(x_batch_shape, out_batch):
        lhs_flat = None
    else:
        if lhs is None:
            lhs = torch.arange(x_batch, dtype=torch.int32, device=dev).reshape(x_batch_shape)
        lhs_flat = lhs.expand(out_batch).contiguous().reshape(-1)
    x = x.contiguous()
    scales = scales.contiguous()
    biases = biases.contiguous()
    _lib.check(_lib.lib().hq_gather_qmm(
        _ptr(y), _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(lhs_flat), _ptr(rhs_flat),
        batch, max(x_batch, 1), max(w_batch, 1), M, N, K, int(bool(transpose)), group_size, bits,
        int(bool(sorted_indices)), _DT[x.dtype], _DT[scales.dtype], _stream(dev)))
    return y


def _check_dequant(tag, w, scales, biases, group_size, bits):
    _check_params(tag, group_size, bits)
    if w.dim() < 2 or scales.dim() < 2 or biases.dim() < 2:
        raise _err(f"[{tag}] The matrix to be quantized must have at least 2 dimension but it "
                   f"has only {w.dim()}.")
    if tuple(w.shape[:-1]) != tuple(scales.shape[:-1]) or \
            tuple(w.shape[:-1]) != tuple(biases.shape[:-1]):
        raise _err(f"[{tag}] Shape of scales and biases does not match the matrix")
    if w.dtype not in _WORD_DTYPES:
        raise _err(f"[{tag}] The matrix should be given as a uint32")
    if w.shape[-1] * 32 // bits != scales.shape[-1] * group_size or w.shape[-1] * 32 % bits:
        raise _err(f"[{tag}] Shape of scales and biases does not match the matrix given the "
                   f"quantization parameters. Provided matrix of shape {_shape(w)} and "
                   f"scales/biases of shape {_shape(scales)} with group_size={group_size} and "
                   f"bits={bits}.")
    if scales.dtype not in _DT or biases.dtype != scales.dtype:
        raise _err(f"[{tag}] scales and biases must be float32, float16 or bfloat16 and share a "
                   "dtype.")


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """deq(w) = scales * q + biases in the scales' dtype; out is w.shape[:-1] + [K]."""
    tag = "dequantize"
    _check_dequant(tag, w, scales, biases, group_size, bits)
    dev = _check_device(tag, w, scales, biases)
    w = w.contiguous()
    scales = scales.contiguous()
    biases = biases.contiguous()
    K = w.shape[-1] * 32 // bits
    rows = w.numel() // w.shape[-1] if w.shape[-1] else 0
    out = torch.empty((*w.shape[:-1], K), dtype=scales.dtype, device=dev)
    if out.numel() == 0:
        return out
    _lib.check(_lib.lib().hq_dequantize(_ptr(out), _ptr(w), _ptr(scales), _ptr(biases), rows, K,
                                        group_size, bits, _DT[scales.dtype], _stream(dev)))
    return out


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """MLX affine quantize of a float matrix w [..., K] on the GPU.

    Returns (wq int32 [..., K*bits/32] (uint32 bit patterns, MLX packing),
    scales, biases [..., K/group_size] in w's dtype), as mlx-rs
    ``ops::quantize(w, group_size, bits)``: per group, the min or max of larger
    magnitude becomes the bias and an exact multiple of the scale, so 0 is
    representable; every operation rounds to w's dtype.
    """
    tag = "quantize"
    _check_params(tag, group_size, bits)
    if w.dim() < 2:
        raise _err(f"[{tag}] The matrix to be quantized must have at least 2 dimension but it "
                   f"has only {w.dim()}.")
    if w.dtype not in _DT:
        raise _err(f"[{tag}] Only real floating types can be quantized (got {_dt_name(w)}).")
    K = w.shape[-1]
    if K % group_size:
        raise _err(f"[{tag}] The last dimension of the matrix needs to be divisible by the "
                   f"quantization group size {group_size}. However the provided matrix has "
                   f"shape {_shape(w)}")
    dev = _check_device(tag, w)
    w = w.contiguous()
    rows = w.numel() // K if K else 0
    wq = torch.empty((*w.shape[:-1], K * bits // 32), dtype=torch.int32, device=dev)
    scales = torch.empty((*w.shape[:-1], K // group_size), dtype=w.dtype, device=dev)
    biases = torch.empty_like(scales)
    if rows:
        _lib.check(_lib.lib().hq_quantize(_ptr(wq), _ptr(scales), _ptr(biases), _ptr(w), rows, K,
                                          group_size, bits, _DT[w.dtype], _stream(dev)))
    return wq, scales, biases


def embedding(indices: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
              biases: torch.Tensor, group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """Quantized embedding lookup, dequantize(w[idx], scales[idx], biases[idx]).

    higgs' QEmbedding::forward (crates/higgs-models/src/qwen3_next.rs:308-318):
    flatten indices, take rows, dequantize, reshape to indices.shape + [K]. Only
    the selected rows are read.
    """
    tag = "embedding"
    _check_dequant(tag, w, scales, biases, group_size, bits)
    if w.dim() != 2:
        raise _err(f"[{tag}] The embedding table must be 2-D (got {_shape(w)}).")
    dev = _check_device(tag, w, scales, biases, indices)
    flat = _as_u32_indices(tag, indices, "indices").reshape(-1)
    K = w.shape[-1] * 32 // bits
    out = torch.empty((*indices.shape, K), dtype=scales.dtype, device=dev)
    if out.numel() == 0:
        return out
    w = w.contiguous()
    scales = scales.contiguous()
    biases = biases.contiguous()
    _lib.check(_lib.lib().hq_embedding_dequantize(
        _ptr(out), _ptr(w), _ptr(scales), _ptr(biases), _ptr(flat), flat.numel(), w.shape[0], K,
        group_size, bits, _DT[scales.dtype], _stream(dev)))
    return out


# --- fused SwiGLU and the MoE global-sort block ---------------------------------

def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """gate * sigmoid(gate) * up, elementwise (qwen3_next.rs:340-342)."""
    tag = "swiglu"
    dev = _check_device(tag, gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype or gate.dtype not in _DT:
        raise _err(f"[{tag}] gate and up must be float arrays of one shape and dtype (got "
                   f"{_shape(gate)} {_dt_name(gate)} and {_shape(up)} {_dt_name(up)}).")
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    if out.numel():
        _lib.check(_lib.lib().hq_swiglu(_ptr(out), _ptr(gate), _ptr(up), out.numel(),
                                        _DT[gate.dtype], _stream(dev)))
    return out


def _split_rows(t: torch.Tensor, n: int):
    return t[..., :n, :], t[..., n:, :]


def dense_hidden_fused(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                       biases: torch.Tensor, intermediate: int, group_size: int = 64,
                       bits: int = 4) -> torch.Tensor:
    """swiglu of a gate/up projection pair stored concatenated along N.

    higgs' FfnBlock::dense_hidden_fused (crates/higgs-models/src/qwen3_next.rs:
    2539-2585): ``w``/``scales``/``biases`` are gate_proj and up_proj
    concatenated on axis 0 ([2*intermediate, P]); the result is
    silu_mul(split(x @ deq(w).T, intermediate)) of shape [..., intermediate].
    Gate and up run in one launch with the SwiGLU in the epilogue; shapes the
    fused kernel does not take run as two quantized_matmul calls and
    ``swiglu``.
    """
    tag = "quantized_matmul_swiglu"
    _check_params(tag, group_size, bits)
    w, w_inner, w_outer = _extract_dims(tag, x, w, scales, biases, True, group_size, bits)
    if w.dim() != 2 or w_outer != 2 * intermediate or intermediate <= 0:
        raise _err(f"[{tag}] The fused weight must be [2*intermediate, P] = "
                   f"[{2 * intermediate}, ...] (got {_shape(w)}).")
    dev = _check_device(tag, x, w, scales, biases)
    wg, wu = _split_rows(w, intermediate)
    sg, su = _split_rows(scales.contiguous(), intermediate)
    bg, bu = _split_rows(biases.contiguous(), intermediate)
    return swiglu_pair(x, (wg, sg, bg), (wu, su, bu), group_size, bits, dev=dev)


def swiglu_pair(x: torch.Tensor, gate: Sequence[torch.Tensor], up: Sequence[torch.Tensor],
                group_size: int = 64, bits: int = 4, dev=None) -> torch.Tensor:
    """swiglu(x @ deq(Wg).T, x @ deq(Wu).T) for separate (w, scales, biases)
    triples of equal shape; x is [..., K], the result [..., N]."""
    tag = "quantized_matmul_swiglu"
    wg, sg, bg = gate
    wu, su, bu = up
    _check_params(tag, group_size, bits)
    wg, K, N = _extract_dims(tag, x, wg, sg, bg, True, group_size, bits)
    wu, _, _ = _extract_dims(tag, x, wu, su, bu, True, group_size, bits)
    if wg.shape != wu.shape or wg.dim() != 2 or sg.dtype != su.dtype:
        raise _err(f"[{tag}] gate and up projections must be 2-D with one shape and dtype.")
    dev = dev or _check_device(tag, x, wg, sg, bg, wu, su, bu)
    sg, bg, su, bu = (t.contiguous() for t in (sg, bg, su, bu))
    x = x.contiguous()
    out_dtype = result_dtype(x.dtype, sg.dtype)
    h = torch.empty((*x.shape[:-1], N), dtype=out_dtype, device=dev)
    M = x.numel() // K if K else 0
    if h.numel() == 0:
        return h
    rc = _lib.lib().hq_quantized_matmul_swiglu(
        _ptr(h), _ptr(x), _ptr(wg), _ptr(sg), _ptr(bg), _ptr(wu), _ptr(su), _ptr(bu),
        M, N, K, group_size, bits, _DT[x.dtype], _DT[sg.dtype], _stream(dev))
    if rc == _lib.HQ_ERR_UNSUPPORTED:
        g = quantized_matmul(x, wg, sg, bg, True, group_size, bits)
        u = quantized_matmul(x, wu, su, bu, True, group_size, bits)
        return swiglu(g, u)
    _lib.check(rc)
    return h


def gather_qmm_swiglu(x: torch.Tensor, gate: Sequence[torch.Tensor], up: Sequence[torch.Tensor],
                      lhs_indices: Optional[torch.Tensor], rhs_indices: torch.Tensor,
                      group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """swiglu(gather_qmm(x, Wg, ...), gather_qmm(x, Wu, ...)) on the sorted path.

    The gate/up pair and SwiGLU of SwitchMlpWeights::forward_gather_global_sort
    (crates/higgs-models/src/qwen3_next.rs:1764-1787) in one launch. x is
    [x_batch, M, K]; Wg/Wu [E, N, P]; rhs_indices are flat, non-decreasing
    expert ids; lhs_indices (optional, flat) pick x's batch element per row.
    Returns [batch, M, N].
    """
    tag = "gather_qmm_swiglu"
    wg, sg, bg = gate
    wu, su, bu = up
    _check_params(tag, group_size, bits)
    wg, K, N = _extract_dims(tag, x, wg, sg, bg, True, group_size, bits)
    wu, _, _ = _extract_dims(tag, x, wu, su, bu, True, group_size, bits)
    if wg.shape != wu.shape or wg.dim() != 3:
        raise _err(f"[{tag}] gate and up weights must both be [E, N, P] (got {_shape(wg)} and "
                   f"{_shape(wu)}).")
    dev = _check_device(tag, x, wg, sg, bg, wu, su, bu, lhs_indices, rhs_indices)
    rhs = _as_u32_indices(tag, rhs_indices, "rhs_indices").reshape(-1)
    lhs = None if lhs_indices is None else _as_u32_indices(tag, lhs_indices, "lhs_indices").reshape(-1)
    if lhs is not None and lhs.numel() != rhs.numel():
        raise _err(f"[{tag}] lhs_indices and rhs_indices must have one length.")
    x = x.contiguous()
    x_batch = x.numel() // (x.shape[-2] * K) if x.numel() else 1
    M = x.shape[-2]
    batch = rhs.numel()
    h = torch.empty((batch, M, N), dtype=result_dtype(x.dtype, sg.dtype), device=dev)
    if h.numel() == 0:
        return h
    rc = _lib.lib().hq_gather_qmm_swiglu(
        _ptr(h), _ptr(x), _ptr(wg), _ptr(sg.contiguous()), _ptr(bg.contiguous()), _ptr(wu),
        _ptr(su.contiguous()), _ptr(bu.contiguous()), _ptr(lhs), _ptr(rhs), batch,
        max(x_batch, 1), wg.shape[0], M, N, K, group_size, bits, _DT[x.dtype], _DT[sg.dtype],
        _stream(dev))
    if rc == _lib.HQ_ERR_UNSUPPORTED:
        # shapes or dtypes the fused grouped kernel does not take (float32
        # activations, mixed dtypes, K % 64 != 0): the reference's own form,
        # two sorted gather_qmm calls and swiglu (qwen3_next.rs:1764-1787)
        xs = x.reshape(-1, M, K)
        if lhs is None:  # the null-lhs broadcast, made explicit
            lhs = (torch.arange(batch, dtype=torch.int64, device=dev) //
                   (batch // max(x_batch, 1))).to(torch.int32)
        g = gather_qmm(xs, wg, sg, bg, lhs, rhs, True, group_size, bits, True)
        u = gather_qmm(xs, wu, su, bu, lhs, rhs, True, group_size, bits, True)
        return swiglu(g, u)
    _lib.check(rc)
    return h


def moe_sort(indices: torch.Tensor, num_experts: int):
    """The index plumbing of forward_gather_global_sort (qwen3_next.rs:1746-1761).

    indices: [..., top_k] expert ids. Returns (order, inv_order, idx_sorted,
    token_idx), each int32 [n] (uint32 bit patterns), n = indices.numel():
    order = stable argsort of the flattened ids, inv_order = argsort(order),
    idx_sorted = ids[order], token_idx = order // top_k.
    """
    tag = "moe_sort"
    dev = _check_device(tag, indices)
    if indices.dim() < 1:
        raise _err(f"[{tag}] indices must have a top_k axis.")
    top_k = indices.shape[-1]
    flat = _as_u32_indices(tag, indices, "indices").reshape(-1)
    n = flat.numel()
    outs = [torch.empty(n, dtype=torch.int32, device=dev) for _ in range(4)]
    if n:
        _lib.check(_lib.lib().hq_moe_sort(*(_ptr(o) for o in outs), _ptr(flat), n, top_k,
                                          num_experts, _stream(dev)))
    return tuple(outs)


def moe_combine(y_sorted: torch.Tensor, inv_order: torch.Tensor,
                scores: torch.Tensor) -> torch.Tensor:
    """out[t] = sum_j scores[t, j] * y_sorted[inv_order[t*top_k + j]].

    The unsort of forward_gather_global_sort (qwen3_next.rs:1802-1808) fused
    with the score-weighted sum of the MoE block (qwen3_moe.rs:355-357).
    y_sorted: [n, D] (or [n, 1, D]); scores: [..., top_k]; returns
    scores.shape[:-1] + [D].
    """
    tag = "moe_combine"
    dev = _check_device(tag, y_sorted, inv_order, scores)
    top_k = scores.shape[-1]
    tokens = scores.numel() // top_k if top_k else 0
    D = y_sorted.shape[-1]
    y = y_sorted.contiguous().reshape(-1, D)
    inv = _as_u32_indices(tag, inv_order, "inv_order").reshape(-1)
    if y.shape[0] != tokens * top_k or inv.numel() != tokens * top_k:
        raise _err(f"[{tag}] y_sorted has {y.shape[0]} rows and inv_order {inv.numel()} for "
                   f"{tokens} tokens x top_k {top_k}.")
    if y.dtype not in _DT or scores.dtype not in _DT:
        raise _err(f"[{tag}] y and scores must be float arrays.")
    out = torch.empty((*scores.shape[:-1], D), dtype=y.dtype, device=dev)
    if out.numel():
        _lib.check(_lib.lib().hq_moe_combine(
            _ptr(out), _ptr(y), _ptr(inv), _ptr(scores.contiguous()), tokens, top_k, D,
            _DT[y.dtype], _DT[scores.dtype], _stream(dev)))
    return out


def _proj(t: Sequence, group_size: int, bits: int):
    """A projection argument: (w, scales, biases) uses the call's group_size
    and bits; (w, scales, biases, group_size, bits) carries its own, as each
    SwitchLinear of a mixed-precision checkpoint does."""
    if len(t) == 5:
        return tuple(t[:3]), int(t[3]), int(t[4])
    if len(t) == 3:
        return tuple(t), group_size, bits
    raise _err("[switch_glu] a projection is (w, scales, biases[, group_size, bits]).")


def _switch_sorted(x, indices, gate, up, down, group_size, bits):
    """Sort, gate/up + SwiGLU, down; returns (y_sorted [n, D], inv_order).

    Each projection uses its own (group_size, bits) (qwen3_next.rs:1764-1800
    passes gate_proj's, up_proj's and down_proj's settings to their own
    gather_qmm). Gate and up run as one fused launch when they share their
    settings; otherwise as two sorted gather_qmm calls and swiglu."""
    (g_t, g_gs, g_b) = _proj(gate, group_size, bits)
    (u_t, u_gs, u_b) = _proj(up, group_size, bits)
    (d_t, d_gs, d_b) = _proj(down, group_size, bits)
    E = g_t[0].shape[0]
    D = x.shape[-1]
    order, inv, srt, tok = moe_sort(indices, E)
    xf = x.reshape(-1, 1, D)
    if (g_gs, g_b) == (u_gs, u_b):
        h = gather_qmm_swiglu(xf, g_t, u_t, tok, srt, g_gs, g_b)        # [n, 1, I]
    else:
        gt = gather_qmm(xf, *g_t, tok, srt, True, g_gs, g_b, True)
        ut = gather_qmm(xf, *u_t, tok, srt, True, u_gs, u_b, True)
        h = swiglu(gt, ut)
    y = gather_qmm(h, *d_t, None, srt, True, d_gs, d_b, True)
    return y.reshape(-1, y.shape[-1]), inv


def forward_gather_global_sort(x: torch.Tensor, indices: torch.Tensor,
                               gate: Sequence, up: Sequence, down: Sequence,
                               group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """SwitchMlpWeights::forward_gather_global_sort (qwen3_next.rs:1731-1809).

    x: [B, L, D]; indices: [B, L, top_k]; gate/up/down: (w, scales, biases)
    of SwitchLinear weights [E, N, P], optionally followed by that
    projection's own group_size and bits. Returns [B, L, top_k, D] in the
    original (unsorted) order. The x gather rides on gather_qmm's
    lhs_indices, gate/up/SwiGLU is one launch, and the unsort is a combine
    with unit scores (an exact row copy).
    """
    B, L, D = x.shape
    top_k = indices.shape[-1]
    y, inv = _switch_sorted(x, indices, gate, up, down, group_size, bits)
    ones = torch.ones((y.shape[0], 1), dtype=y.dtype, device=y.device)
    out = moe_combine(y, inv, ones)
    return out.reshape(B, L, top_k, -1)


def forward_gather(x: torch.Tensor, indices: torch.Tensor, gate: Sequence, up: Sequence,
                   down: Sequence, group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """SwitchMlpWeights::forward_gather, the unsorted path (qwen3_next.rs:1660-1720).

    x: [B, L, D] is viewed as [B, L, 1, 1, D] and broadcast against indices
    [B, L, top_k]: gate and up are gather_qmm calls with the null-lhs
    broadcast, then swiglu, then down with the same indices; the result
    [B, L, top_k, 1, D] is squeezed to [B, L, top_k, D]. Every (token, slot)
    row reads its expert's weights on its own (no sort), which is why the
    reference moved to the global-sort path; both must agree
    (qwen3_next.rs:4431-4530).
    """
    (g_t, g_gs, g_b) = _proj(gate, group_size, bits)
    (u_t, u_gs, u_b) = _proj(up, group_size, bits)
    (d_t, d_gs, d_b) = _proj(down, group_size, bits)
    B, L, D = x.shape
    top_k = indices.shape[-1]
    xe = x.reshape(B, L, 1, 1, D)
    g = gather_qmm(xe, *g_t, None, indices, True, g_gs, g_b, False)      # [B, L, k, 1, I]
    u = gather_qmm(xe, *u_t, None, indices, True, u_gs, u_b, False)
    h = swiglu(g, u)
    y = gather_qmm(h, *d_t, None, indices, True, d_gs, d_b, False)      # [B, L, k, 1, D]
    return y.reshape(B, L, top_k, -1)


def moe_block(x: torch.Tensor, indices: torch.Tensor, scores: torch.Tensor,
              gate: Sequence, up: Sequence, down: Sequence, group_size: int = 64,
              bits: int = 4) -> torch.Tensor:
    """Experts of the MoE block after routing (qwen3_moe.rs:353-357):
    forward_gather_global_sort(x, indices) * scores, summed over top_k.

    x: [B, L, D]; indices, scores: [B, L, top_k]. Returns [B, L, D]. Four
    launches (sort, gate/up + SwiGLU, down, unsort + weighted sum) when gate
    and up share their quantization settings.
    """
    y, inv = _switch_sorted(x, indices, gate, up, down, group_size, bits)
    return moe_combine(y, inv, scores)
