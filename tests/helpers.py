"""Shared helpers for the GPU parity tests: numpy <-> device tensors and the
error metric. Relative error is max_i |y_i - r_i| / max_i |r_i| against the
oracle's fp64-accumulated result (element-wise relative error is unbounded
near zero)."""
import numpy as np
import torch

import oracle as O
from higgs_amd import gen

TORCH_DT = {O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16}
DT_OF = {v: k for k, v in TORCH_DT.items()}

# Tolerances stated by the north star: bf16/fp16 output 1e-2, fp32 output 1e-3.
TOL = {O.BF16: 1e-2, O.F16: 1e-2, O.F32: 1e-3}


def to_dev(a: np.ndarray, dt: int, dev) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if dt == O.F32:
        return torch.from_numpy(a.astype(np.float32)).to(dev)
    return torch.from_numpy(a.view(np.int16)).view(TORCH_DT[dt]).to(dev)


def words_dev(w: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(w).view(np.int32)).to(dev)


def idx_dev(i: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(i, dtype=np.uint32).view(np.int32)).to(dev)


def to_host_bits(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> numpy: float32 values, or uint16 bit patterns for 16-bit."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def to_host_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    den = np.abs(ref).max()
    return float(np.abs(y - ref).max() / (den if den > 0 else 1.0))


def quant(seed, rows, K, bits, g, dt, lead=(), bias_noise=1e-3):
    """Seeded quantized matrix with scales/biases in dtype `dt` (numpy)."""
    w, s, b = gen.np_quantized(seed, rows, K, bits, g, bias_noise=bias_noise, lead=lead)
    if dt == O.BF16:
        return w, s, b
    sf, bf = gen.bf16_bits_to_f32(s), gen.bf16_bits_to_f32(b)
    if dt == O.F32:
        return w, sf, bf
    return w, O.from_f32(sf, O.F16), O.from_f32(bf, O.F16)


def x_of(seed, shape, dt):
    xb = gen.np_x_bf16(seed, shape)
    if dt == O.BF16:
        return xb
    xf = gen.bf16_bits_to_f32(xb)
    if dt == O.F32:
        return (xf * np.float32(1.0) + np.float32(1e-3) * gen.np_normal(seed + 99, xf.size)
                .reshape(xf.shape).astype(np.float32))
    return O.from_f32(xf, O.F16)
