"""Seeded synthetic inputs with the distributions of the benchmark configs.

* packed weights: every element uniform over [0, 2^bits - 1]. Because each
  element is `bits` independent uniform bits of the row bitstream, uniform
  random u32 words are exactly uniformly distributed packed matrices for every
  bit width, including the word-straddling 3/5/6-bit layouts.
* scales = bf16(|N(0,1)| * 0.02 + 1e-3)
* biases = bf16(-2^(bits-1) * scale + N(0, bias_noise))  (bias_noise 1e-3 is
  read as a standard deviation; 0 gives the noise-free c3 form)
* x ~ N(0, 1) rounded to bf16.

Two engines: ``np_*`` uses counter-based SplitMix64 (output i of stream
`seed` = mix64(seed + (i + 1) * 0x9E3779B97F4A7C15), identical to the
sequential SplitMix64 generator) with Box-Muller normals, for CPU tests and
fixtures; ``torch_*`` uses torch's seeded device generator for GB-scale
benchmark tensors generated directly in HBM.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset..offset+n-1 of the SplitMix64 stream seeded with `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def np_uniform(seed: int, n: int) -> np.ndarray:
    """Uniform doubles in [0, 1) with 53 random bits."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def np_normal(seed: int, n: int) -> np.ndarray:
    """Standard normals by Box-Muller (cosine branch) from pairs of uniforms."""
    u = splitmix64(seed, 2 * n)
    u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / (1 << 53))  # (0, 1]
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round-to-nearest-even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_bits(q: np.ndarray, bits: int) -> np.ndarray:
    """Pack unsigned ints (last axis) LSB-first into little-endian u32 words."""
    q = np.asarray(q, dtype=np.uint32)
    cols = q.shape[-1]
    if (cols * bits) % 32:
        raise ValueError("last dim * bits must be a multiple of 32")
    bitplanes = ((q[..., None] >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.uint8)
    stream = bitplanes.reshape(*q.shape[:-1], cols * bits)
    by = np.packbits(stream, axis=-1, bitorder="little")
    return np.ascontiguousarray(by).view("<u4").reshape(*q.shape[:-1], cols * bits // 32)


def np_quantized(seed: int, rows: int, K: int, bits: int, group_size: int,
                 bias_noise: float = 1e-3, lead: tuple = ()):
    """(w u32 [*lead, rows, K*bits/32], scales bf16-bits, biases bf16-bits [*lead, rows, K/g])."""
    n_lead = int(np.prod(lead)) if lead else 1
    P = K * bits // 32
    G = K // group_size
    nw = n_lead * rows * P
    w = (splitmix64(seed, nw) >> np.uint64(32)).astype(np.uint32).reshape(*lead, rows, P)
    ns = n_lead * rows * G
    s = (np.abs(np_normal(seed + 1, ns)) * 0.02 + 1e-3).astype(np.float32)
    s_bits = f32_to_bf16_bits(s)
    s_r = bf16_bits_to_f32(s_bits)
    noise = np_normal(seed + 2, ns).astype(np.float32) * np.float32(bias_noise)
    b = (-(np.float32(2 ** (bits - 1))) * s_r + noise).astype(np.float32)
    b_bits = f32_to_bf16_bits(b)
    return w, s_bits.reshape(*lead, rows, G), b_bits.reshape(*lead, rows, G)


def np_x_bf16(seed: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    return f32_to_bf16_bits(np_normal(seed, n).astype(np.float32)).reshape(shape)


# ---------------------------------------------------------------------------
# device (torch) engine
# ---------------------------------------------------------------------------

def torch_quantized(seed: int, rows: int, K: int, bits: int, group_size: int, device,
                    bias_noise: float = 1e-3, lead: tuple = (), dtype=None):
    """Device tensors (w int32 [*lead, rows, P], scales, biases [*lead, rows, G])."""
    import torch

    dtype = dtype or torch.bfloat16
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    P = K * bits // 32
    G = K // group_size
    w = torch.randint(-(2 ** 31), 2 ** 31, (*lead, rows, P), dtype=torch.int32, device=device,
                      generator=g)
    s = (torch.randn((*lead, rows, G), device=device, generator=g).abs() * 0.02 + 1e-3).to(dtype)
    noise = torch.randn((*lead, rows, G), device=device, generator=g) * bias_noise
    b = (-(2.0 ** (bits - 1)) * s.float() + noise).to(dtype)
    return w, s, b


def torch_x(seed: int, shape, device, dtype=None):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(tuple(shape), device=device, generator=g).to(dtype or torch.bfloat16)


def topk_routing(seed: int, tokens: int, experts: int, top_k: int) -> np.ndarray:
    """Router indices: softmax(N(0,1) logits) -> top-k experts per token, as uint32
    [tokens, top_k] (ties broken by the lower expert id)."""
    logits = np_normal(seed, tokens * experts).reshape(tokens, experts)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :top_k]
    return order.astype(np.uint32)
