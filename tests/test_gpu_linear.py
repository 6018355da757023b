"""Quantized linear layers with a bias, and affine quantize, on the GPU through
the C ABI (via the torch facade), against the CPU oracle.

* hq_quantized_linear: mlx-rs QuantizedLinear::forward = quantized_matmul
  then + bias (Qwen2-style q/k/v biases, crates/higgs-models/src/
  transformer.rs:180-191). Two bars: bit-exact against the product kernel's
  own output plus the bias rounded once more (the epilogue must add exactly
  the bias of its column, after rounding the product), and max relative
  error <= 1e-2 (16-bit) / 1e-3 (fp32) against the fp64 oracle.
* hq_quantize: mlx-rs ops::quantize (qwen3_next.rs:4305-4307, 12942),
  bit-exact against the oracle's op-by-op restatement (codes, scales and
  biases), for every dtype, bit width and group size, with the special
  groups the algorithm branches on.
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import TORCH_DT, TOL, quant, rel_err, to_dev, to_host_bits, to_host_f64, words_dev, \
    x_of
from higgs_amd import gen, layers, ops

pytestmark = pytest.mark.gpu


def _bias(seed, N, dt):
    return x_of(seed, (N,), dt)


def _round_sum(y_bits, bias_bits, dt):
    """round(float(y) + float(bias)) in dt: the epilogue's arithmetic."""
    yf = O.to_f32(y_bits, dt) if dt != O.F32 else y_bits
    bf = O.to_f32(bias_bits, dt) if dt != O.F32 else bias_bits
    s = (yf.astype(np.float32) + bf.astype(np.float32)[None, :]).astype(np.float32)
    return s if dt == O.F32 else O.from_f32(s, dt)


# (M, N, K, x dtype, scale dtype): every transpose=true kernel family --
# streaming decode GEMV (K > 2048, M in 1, 2, 4, 8), persistent GEMV (K = 2048,
# M = 3), batched GEMV (K % 1024 != 0), the VALU GEMV (fp32 x), 8-row GEMV
# launches for 9-32 rows on few W rows (M = 12, 26), the general GEMM (mixed
# dtypes), the large-tile GEMM (M = 20, M >= 128).
CASES = [
    (1, 1024, 4096, O.BF16, O.BF16),
    (2, 4096, 4096, O.BF16, O.BF16),
    (4, 1024, 4096, O.BF16, O.BF16),
    (8, 4096, 4096, O.F16, O.F16),
    (3, 512, 2048, O.BF16, O.BF16),
    (1, 320, 640, O.BF16, O.BF16),
    (2, 256, 512, O.F32, O.F32),
    (20, 384, 1024, O.BF16, O.BF16),
    (12, 1024, 4096, O.BF16, O.BF16),
    (26, 512, 4096, O.F16, O.F16),
    (33, 256, 512, O.F16, O.BF16),
    (256, 640, 1024, O.BF16, O.BF16),
    (200, 512, 768, O.F16, O.F16),
]


@pytest.mark.parametrize("M,N,K,xdt,sdt", CASES)
def test_linear_bias_epilogue(dev, M, N, K, xdt, sdt):
    w, s, b = quant(300 + M, N, K, 4, 64, sdt)
    x = x_of(301 + M, (M, K), xdt)
    odt = O.result_dtype(xdt, sdt)
    lb = _bias(302 + M, N, odt)
    W = words_dev(w, dev)
    S, B = to_dev(s, sdt, dev), to_dev(b, sdt, dev)
    X, LB = to_dev(x, xdt, dev), to_dev(lb, odt, dev)
    y = ops.quantized_linear(X, W, S, B, LB, 64, 4)
    y0 = ops.quantized_matmul(X, W, S, B, True, 64, 4)
    # the bias is added to the rounded product, column by column
    np.testing.assert_array_equal(to_host_bits(y), _round_sum(to_host_bits(y0), lb, odt))
    exact = O.qmm_f64(x, xdt, w, s, b, sdt, 64, 4)
    lbf = (O.to_f32(lb, odt) if odt != O.F32 else lb).astype(np.float64)
    ref = exact + lbf[None, :]
    assert rel_err(to_host_f64(y), ref) <= TOL[odt], (M, N, K)
    # no bias: the plain product, bit for bit
    assert torch.equal(ops.quantized_linear(X, W, S, B, None, 64, 4), y0)


@pytest.mark.parametrize("M", [1, 4, 8])
def test_qwen2_style_qkv_bias_at_llama_shapes(dev, M):
    """configs[1] q [4096, 4096] and k/v [1024, 4096] (4-bit g64) as Qwen2
    builds them, with biases (transformer.rs:180-191)."""
    for j, N in enumerate((4096, 1024, 1024)):
        w, s, b = quant(310 + j, N, 4096, 4, 64, O.BF16)
        x = x_of(320 + M, (M, 4096), O.BF16)
        lb = _bias(330 + j, N, O.BF16)
        lin = layers.QLinear(words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev),
                             64, 4, bias=to_dev(lb, O.BF16, dev))
        y = lin(to_dev(x, O.BF16, dev))
        ref = O.qmm_f64(x, O.BF16, w, s, b, O.BF16, 64, 4) + \
            O.to_f32(lb, O.BF16).astype(np.float64)[None, :]
        assert rel_err(to_host_f64(y), ref) <= 1e-2, (N, M)


def _special_rows(rng, K, g):
    """Rows of random groups at several magnitudes, plus the groups the
    algorithm branches on: constant, all zero, all negative, all positive,
    |min| == |max|, an exact zero among random values, tiny and huge values."""
    rows = [rng.standard_normal(K) * 10.0 ** rng.integers(-4, 3) for _ in range(6)]
    special = []
    for kind in range(8):
        v = rng.standard_normal(g)
        if kind == 0:
            v[:] = 0.37
        elif kind == 1:
            v[:] = 0.0
        elif kind == 2:
            v = -np.abs(v) - 0.5
        elif kind == 3:
            v = np.abs(v) + 0.5
        elif kind == 4:
            v[0], v[1] = -2.0, 2.0
            v = np.clip(v, -2.0, 2.0)
        elif kind == 5:
            v[3] = 0.0
        elif kind == 6:
            v = v * 1e-6
        else:
            v = v * 3e3
        special.append(v)
    sp = np.concatenate(special)
    reps = -(-K // sp.size)
    rows.append(np.tile(sp, reps)[:K])
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("g", [32, 64, 128])
def test_quantize_bit_exact(dev, dt, bits, g):
    rng = np.random.default_rng(bits * 100 + g + dt)
    wf = _special_rows(rng, 1024, g)
    wh = wf if dt == O.F32 else O.from_f32(wf, dt)
    wq, s, b = O.quantize(wh, dt, g, bits)
    Wq, S, B = ops.quantize(to_dev(wh, dt, dev), g, bits)
    assert Wq.dtype == torch.int32 and S.dtype == TORCH_DT[dt]
    np.testing.assert_array_equal(Wq.cpu().numpy().view(np.uint32), wq)
    np.testing.assert_array_equal(to_host_bits(S), s)
    np.testing.assert_array_equal(to_host_bits(B), b)


def test_quantize_llama_gate_shape_round_trip(dev):
    """A [14336, 4096] bf16 weight (the Llama-3-8B gate) at 4-bit g64:
    bit-exact against the oracle, and quantize -> dequantize on the GPU equals
    the oracle's dequantize of the oracle's codes."""
    N, K = 14336, 4096
    wd = gen.torch_x(340, (N, K), dev)           # N(0,1) in bf16
    Wq, S, B = ops.quantize(wd, 64, 4)
    wh = to_host_bits(wd)
    wq, s, b = O.quantize(wh, O.BF16, 64, 4)
    np.testing.assert_array_equal(Wq.cpu().numpy().view(np.uint32), wq)
    np.testing.assert_array_equal(to_host_bits(S), s)
    np.testing.assert_array_equal(to_host_bits(B), b)
    rows = np.arange(0, N, 97)
    deq = to_host_bits(ops.dequantize(Wq, S, B, 64, 4))[rows]
    np.testing.assert_array_equal(deq, O.dequantize(wq[rows], s[rows], b[rows], 64, 4, O.BF16))


@pytest.mark.parametrize("M", [1, 300])
def test_qlinear_from_float(dev, M):
    """nn::quantize of a float layer (transformer.rs:954-965) then its forward:
    the result is the product with the layer's own quantized weights."""
    N, K = 512, 1024
    wf = gen.torch_x(350, (N, K), dev)
    lin = layers.QLinear.from_float(wf, 64, 4)
    x = gen.torch_x(351 + M, (M, K), dev)
    y = lin(x)
    w = lin.weight.cpu().numpy().view(np.uint32)
    ref = O.qmm_f64(to_host_bits(x), O.BF16, w, to_host_bits(lin.scales),
                    to_host_bits(lin.biases), O.BF16, 64, 4)
    assert rel_err(to_host_f64(y), ref) <= 1e-2
    # and the quantized layer is close to the float one (4-bit: within a few %)
    dense = (x.float() @ wf.float().T).cpu().numpy().astype(np.float64)
    assert rel_err(to_host_f64(y), dense) <= 0.1
