"""Parity of the HIP path (through the C ABI, via the torch facade) with the
CPU oracle on identical seeded inputs.

Bars: dequantize bit-exact (two-rounding convention, include/higgs_qmm.h);
quantized_matmul / gather_qmm max relative error (max|y-r| / max|r| against the
oracle's fp64 result) <= 1e-2 for bf16/fp16 output and <= 1e-3 for fp32 output.
Shapes: small ones the oracle finishes in seconds, plus the BASELINE configs at
full size, compared on sampled weight rows (each sampled row is an exact
sub-problem, so the check is size independent).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import (TOL, idx_dev, quant, rel_err, to_dev, to_host_bits, to_host_f64,
                     words_dev, x_of)
from higgs_amd import gen, ops

pytestmark = pytest.mark.gpu

BITS = (2, 3, 4, 5, 6, 8)
GROUPS = (32, 64, 128)


def _qmm_check(dev, M, N, K, bits, g, xdt, sdt, seed=0, transpose=True, lead_x=None):
    rows, cols = (N, K) if transpose else (K, N)
    w, s, b = quant(seed, rows, cols, bits, g, sdt)
    x = x_of(seed + 7, (M, K), xdt)
    y = ops.quantized_matmul(to_dev(x, xdt, dev), words_dev(w, dev), to_dev(s, sdt, dev),
                             to_dev(b, sdt, dev), transpose, g, bits)
    odt = O.result_dtype(xdt, sdt)
    assert y.dtype == {O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16}[odt]
    assert tuple(y.shape) == (M, N)
    ref = O.qmm_f64(x, xdt, w, s, b, sdt, g, bits, transpose=transpose)
    err = rel_err(to_host_f64(y), ref)
    assert err <= TOL[odt], (M, N, K, bits, g, xdt, sdt, err)
    return err


# --- dequantize ---------------------------------------------------------------

@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
def test_dequantize_bit_exact(dev, bits, g, dt):
    w, s, b = quant(bits * 10 + g, 37, 384, bits, g, dt)
    out = ops.dequantize(words_dev(w, dev), to_dev(s, dt, dev), to_dev(b, dt, dev), g, bits)
    ref = O.dequantize(w, s, b, g, bits, dt)
    np.testing.assert_array_equal(to_host_bits(out), ref)


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_special_values_bit_exact(dev, dt, bits):
    """Scales and biases at NaN (both signs, odd payloads), +-Inf, the largest
    finite value (products overflow), denormals, signed zeros. Every non-NaN
    output bit equals the oracle's and every NaN output is a NaN where the
    oracle's is: the sign of a NaN made by an invalid operation (Inf * 0,
    Inf - Inf) is the platform's default NaN (negative on x86, where the
    oracle runs; positive on the GPU), not a property of the algorithm."""
    if dt == O.BF16:
        special = [0x7fc0, 0xffc1, 0x7f81, 0x7f80, 0xff80, 0x7f7f, 0xff7f, 0x0001, 0x8003,
                   0x0080, 0x0000, 0x8000, 0x3f80, 0xbf80, 0x3c00, 0x0040]
    else:
        special = [0x7e00, 0xfe01, 0x7c01, 0x7c00, 0xfc00, 0x7bff, 0xfbff, 0x0001, 0x8003,
                   0x0400, 0x0000, 0x8000, 0x3c00, 0xbc00, 0x2000, 0x0200]
    rows, K, g = 16, 256, 32
    G = K // g
    rng = np.random.default_rng(bits)
    sp = np.array(special, dtype=np.uint16)
    s = sp[rng.integers(0, len(sp), (rows, G))]
    b = sp[rng.integers(0, len(sp), (rows, G))]
    s[0, :] = sp[:G]            # every special value as a scale and as a bias
    b[1, :] = sp[:G]
    s[2, :] = sp[G:2 * G] if len(sp) >= 2 * G else sp[:G]
    b[3, :] = sp[G:2 * G] if len(sp) >= 2 * G else sp[:G]
    q = rng.integers(0, 1 << bits, (rows, K), dtype=np.uint64)
    q[:, :4] = 0                # 0 * Inf
    w = gen.pack_bits(q, bits)
    out = to_host_bits(ops.dequantize(words_dev(w, dev), to_dev(s, dt, dev), to_dev(b, dt, dev),
                                      g, bits))
    ref = O.dequantize(w, s, b, g, bits, dt)
    exp_mask, man_mask = (0x7f80, 0x007f) if dt == O.BF16 else (0x7c00, 0x03ff)
    isnan = lambda u: ((u & exp_mask) == exp_mask) & ((u & man_mask) != 0)
    np.testing.assert_array_equal(isnan(out), isnan(ref))
    assert isnan(ref).any() and (~isnan(ref)).any()
    np.testing.assert_array_equal(out[~isnan(ref)], ref[~isnan(ref)])
    # NaN outputs are canonical quiet NaNs
    nan_bits = out[isnan(out)] & 0x7fff
    assert np.all(nan_bits == (0x7fc0 if dt == O.BF16 else 0x7e00))


def test_dequantize_bit_exact_c0_shape(dev):
    # [8192, 2048] 4-bit g64, bf16 scales
    w, s, b = quant(1, 8192, 2048, 4, 64, O.BF16)
    out = ops.dequantize(words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev), 64, 4)
    np.testing.assert_array_equal(to_host_bits(out), O.dequantize(w, s, b, 64, 4, O.BF16))


def test_dequantize_batched_leading_dims(dev):
    w, s, b = quant(3, 6, 256, 3, 32, O.BF16, lead=(2,))
    out = ops.dequantize(words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev), 32, 3)
    assert tuple(out.shape) == (2, 6, 256)
    ref = O.dequantize(w.reshape(12, -1), s.reshape(12, -1), b.reshape(12, -1), 32, 3, O.BF16)
    np.testing.assert_array_equal(to_host_bits(out).reshape(12, -1), ref)


def test_embedding_gather_then_dequantize_equivalence(dev):
    # qwen3_next.rs:12374-12412: take-then-dequantize == dequantize-then-take
    w, s, b = quant(5, 256, 128, 4, 64, O.BF16)
    W, S, B = words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev)
    idx = np.array([[0, 5, 42], [255, 5, 7]], np.uint32)
    emb = ops.embedding(idx_dev(idx, dev), W, S, B, 64, 4)
    assert tuple(emb.shape) == (2, 3, 128)
    full = ops.dequantize(W, S, B, 64, 4)
    np.testing.assert_array_equal(to_host_bits(emb), to_host_bits(full[idx_dev(idx, dev).long()]))
    bad = ops.embedding(idx_dev(np.array([256, 1], np.uint32), dev), W, S, B, 64, 4)
    assert torch.isnan(bad[0]).all() and not torch.isnan(bad[1]).any()


# --- quantized_matmul: decode GEMV --------------------------------------------

@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("g", GROUPS)
def test_qmv_bf16_all_bits_groups(dev, bits, g):
    for M in (1, 3, 8):
        _qmm_check(dev, M, 200, 512, bits, g, O.BF16, O.BF16, seed=bits + g)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("xdt,sdt", [(O.F32, O.F32), (O.F16, O.F16), (O.BF16, O.F16),
                                     (O.F32, O.BF16), (O.F16, O.BF16), (O.BF16, O.F32)])
def test_qmv_dtypes(dev, M, xdt, sdt):
    _qmm_check(dev, M, 96, 384, 4, 64, xdt, sdt, seed=M)


# --- quantized_matmul: prefill GEMM -------------------------------------------

@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("g", [32, 128])
def test_qmm_bf16_all_bits(dev, bits, g):
    _qmm_check(dev, 70, 160, 384, bits, g, O.BF16, O.BF16, seed=bits)


@pytest.mark.parametrize("M,N,K", [(9, 64, 64), (128, 128, 128), (200, 300, 96), (513, 257, 320)])
@pytest.mark.parametrize("xdt,sdt", [(O.BF16, O.BF16), (O.F16, O.F16), (O.F32, O.F32),
                                     (O.BF16, O.F16)])
def test_qmm_shapes_dtypes(dev, M, N, K, xdt, sdt):
    _qmm_check(dev, M, N, K, 4, 32, xdt, sdt, seed=M + N)


def test_qmm_leading_dims_flatten(dev):
    w, s, b = quant(2, 64, 128, 4, 64, O.BF16)
    x = x_of(3, (2, 5, 128), O.BF16)
    y = ops.quantized_matmul(to_dev(x, O.BF16, dev), words_dev(w, dev), to_dev(s, O.BF16, dev),
                             to_dev(b, O.BF16, dev), True, 64, 4)
    assert tuple(y.shape) == (2, 5, 64)
    ref = O.qmm_f64(x.reshape(10, 128), O.BF16, w, s, b, O.BF16, 64, 4)
    assert rel_err(to_host_f64(y).reshape(10, 64), ref) <= 1e-2


@pytest.mark.parametrize("M", [1, 4, 33])
@pytest.mark.parametrize("bits", [3, 4, 8])
def test_no_transpose(dev, M, bits):
    _qmm_check(dev, M, 128, 100, bits, 64, O.BF16, O.BF16, seed=M, transpose=False)


def test_empty_and_minimal(dev):
    w, s, b = quant(4, 16, 32, 4, 32, O.BF16)
    W, S, B = words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev)
    y = ops.quantized_matmul(torch.zeros(0, 32, dtype=torch.bfloat16, device=dev), W, S, B, True,
                             32, 4)
    assert tuple(y.shape) == (0, 16)
    _qmm_check(dev, 1, 1, 32, 4, 32, O.BF16, O.BF16)
    _qmm_check(dev, 17, 1, 32, 4, 32, O.BF16, O.BF16)


def test_fused_gate_up_equals_separate(dev):
    # qwen3_next.rs:13132-13169: one qmv over concat(gate, up) == two qmvs
    wg, sg, bg = quant(11, 96, 64, 4, 32, O.F16)
    wu, su, bu = quant(12, 96, 64, 4, 32, O.F16)
    x = to_dev(x_of(13, (1, 64), O.F16), O.F16, dev)
    d = lambda a, dt=O.F16: to_dev(a, dt, dev)
    fused = ops.quantized_matmul(x, words_dev(np.concatenate([wg, wu]), dev),
                                 d(np.concatenate([sg, su])), d(np.concatenate([bg, bu])), True,
                                 32, 4)
    g_ = ops.quantized_matmul(x, words_dev(wg, dev), d(sg), d(bg), True, 32, 4)
    u_ = ops.quantized_matmul(x, words_dev(wu, dev), d(su), d(bu), True, 32, 4)
    assert torch.equal(fused, torch.cat([g_, u_], dim=-1))


def test_qmv_equals_qmm_rows(dev):
    # qwen3_next.rs:12929-13006 (custom qgemv vs quantized_matmul): the GEMV path
    # (M <= 8) and the GEMM path (M > 8) agree row by row within tolerance.
    w, s, b = quant(14, 256, 1024, 4, 64, O.BF16)
    W, S, B = words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev)
    x = to_dev(x_of(15, (16, 1024), O.BF16), O.BF16, dev)
    big = ops.quantized_matmul(x, W, S, B, True, 64, 4).float()
    for r in (0, 7, 15):
        one = ops.quantized_matmul(x[r:r + 1], W, S, B, True, 64, 4).float()
        assert (one - big[r:r + 1]).abs().max() <= 1e-2 * big.abs().max()


# --- gather_qmm ---------------------------------------------------------------

def _experts(seed, E, N, K, bits, g, dt=O.BF16):
    return quant(seed, N, K, bits, g, dt, lead=(E,))


def test_gather_matches_per_expert(dev):
    # qwen3_next.rs:4344-4398
    w, s, b = _experts(20, 4, 64, 64, 4, 64)
    W, S, B = words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev)
    x = to_dev(x_of(21, (1, 64), O.BF16), O.BF16, dev)
    old = ops.quantized_matmul(x, W[2], S[2], B[2], True, 64, 4)
    new = ops.gather_qmm(x.unsqueeze(-2), W, S, B, None, idx_dev(np.array([[2]]), dev), True, 64,
                         4, False)
    assert tuple(new.shape) == (1, 1, 1, 64)
    assert torch.equal(old.reshape(-1), new.reshape(-1))


def test_gather_shapes_like_reference(dev):
    # qwen3_next.rs:4310-4341, 4626-4708: output shape contracts
    w, s, b = _experts(22, 8, 64, 64, 4, 64)
    W, S, B = words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev)
    x = to_dev(x_of(23, (1, 9, 1, 1, 64), O.BF16), O.BF16, dev)
    idx = np.array([0, 1, 2, 3, 4, 5, 6, 7, 0, 1, 2, 3, 4, 5, 6, 7, 0, 7], np.uint32).reshape(1, 9, 2)
    y = ops.gather_qmm(x, W, S, B, None, idx_dev(idx, dev), True, 64, 4, False)
    assert tuple(y.shape) == (1, 9, 2, 1, 64)
    ref = O.gather_qmm_f64(x_of(23, (9, 1, 64), O.BF16), O.BF16, w, s, b, O.BF16, None,
                           idx.reshape(-1), 1, 64, 64, 64, 4)
    assert rel_err(to_host_f64(y).reshape(18, 1, 64), ref) <= 1e-2


@pytest.mark.parametrize("M", [1, 3, 12])
@pytest.mark.parametrize("bits", [3, 4, 8])
def test_gather_vs_oracle(dev, M, bits):
    E, N, K, g = 6, 96, 256, 64
    w, s, b = _experts(30 + M, E, N, K, bits, g)
    x = x_of(31, (5, M, K), O.BF16)
    rng = np.random.default_rng(M)
    lhs = rng.integers(0, 5, 11).astype(np.uint32)
    rhs = rng.integers(0, E, 11).astype(np.uint32)
    y = ops.gather_qmm(to_dev(x, O.BF16, dev), words_dev(w, dev), to_dev(s, O.BF16, dev),
                       to_dev(b, O.BF16, dev), idx_dev(lhs, dev), idx_dev(rhs, dev), True, g, bits)
    ref = O.gather_qmm_f64(x, O.BF16, w, s, b, O.BF16, lhs, rhs, M, N, K, g, bits)
    assert rel_err(to_host_f64(y), ref) <= 1e-2


def test_gather_out_of_range_gives_nan(dev):
    w, s, b = _experts(40, 3, 64, 128, 4, 64)
    x = x_of(41, (2, 1, 128), O.BF16)
    y = ops.gather_qmm(to_dev(x, O.BF16, dev), words_dev(w, dev), to_dev(s, O.BF16, dev),
                       to_dev(b, O.BF16, dev), idx_dev(np.array([0, 1, 7]), dev),
                       idx_dev(np.array([3, 1, 0]), dev), True, 64, 4)
    assert torch.isnan(y[0]).all() and torch.isnan(y[2]).all()
    assert not torch.isnan(y[1]).any()


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_sorted_equals_unsorted_and_global_sort_roundtrip(dev, dt):
    # qwen3_next.rs:4431-4530 (global sort == baseline), 1731-1809 (sort/unsort).
    # The reference asserts max |diff| < 1e-5 in float32; in bfloat16 the two
    # paths run different kernels and may differ by an output rounding.
    E, D, I, L, k = 8, 64, 64, 16, 3
    wg, sg, bg = _experts(50, E, I, D, 4, 64, dt)
    x = x_of(51, (1, L, D), dt)
    idx = (np.arange(L * k) % E).astype(np.uint32).reshape(1, L, k)
    Wd, Sd, Bd = words_dev(wg, dev), to_dev(sg, dt, dev), to_dev(bg, dt, dev)
    xd = to_dev(x, dt, dev)
    base = ops.gather_qmm(xd.reshape(1, L, 1, 1, D), Wd, Sd, Bd, None, idx_dev(idx, dev), True,
                          64, 4, False).reshape(L * k, I)
    order, inv, srt, tok = O.gather_sort(idx, k)
    xs = xd.reshape(L, 1, D)[torch.from_numpy(tok.astype(np.int64)).to(dev)]
    ys = ops.gather_qmm(xs, Wd, Sd, Bd, None, idx_dev(srt, dev), True, 64, 4, True).reshape(-1, I)
    unsorted = ys[torch.from_numpy(inv.astype(np.int64)).to(dev)]
    diff = (unsorted.float() - base.float()).abs().max().item()
    if dt == O.F32:
        assert diff < 1e-5
    else:
        assert diff <= 1e-2 * base.float().abs().max().item()


@pytest.mark.parametrize("xdt,sdt", [(O.F32, O.F32), (O.F16, O.F16), (O.BF16, O.F16)])
def test_gather_dtypes(dev, xdt, sdt):
    w, s, b = _experts(60, 4, 64, 128, 4, 32, sdt)
    x = x_of(61, (6, 2, 128), xdt)
    rhs = np.array([3, 0, 0, 1, 2, 3], np.uint32)
    y = ops.gather_qmm(to_dev(x, xdt, dev), words_dev(w, dev), to_dev(s, sdt, dev),
                       to_dev(b, sdt, dev), None, idx_dev(rhs, dev), True, 32, 4)
    ref = O.gather_qmm_f64(x, xdt, w, s, b, sdt, None, rhs, 2, 64, 128, 32, 4)
    assert rel_err(to_host_f64(y), ref) <= TOL[O.result_dtype(xdt, sdt)]


# --- BASELINE configs at full size (sampled rows) -----------------------------

def _sampled_rows_check(dev, M, N, K, bits, g, seed, n_rows=384, bias_noise=1e-3):
    W, S, B = gen.torch_quantized(seed, N, K, bits, g, dev, bias_noise=bias_noise)
    X = gen.torch_x(seed + 1, (M, K), dev)
    Y = ops.quantized_matmul(X, W, S, B, True, g, bits)
    torch.cuda.synchronize()
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, N - 1], rng.integers(0, N, n_rows)]))
    rt = torch.from_numpy(rows).to(dev)
    w = W[rt].cpu().numpy().view(np.uint32)
    s = S[rt].cpu().view(torch.int16).numpy().view(np.uint16)
    b = B[rt].cpu().view(torch.int16).numpy().view(np.uint16)
    x = X.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = O.qmm_f64(x, O.BF16, w, s, b, O.BF16, g, bits)
    err = rel_err(to_host_f64(Y[:, rt]), ref)
    assert err <= 1e-2, (M, N, K, bits, g, err)


@pytest.mark.parametrize("B", [1, 4, 8])
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336),
                                 (128256, 4096)])
def test_c1_llama3_8b_decode_shapes(dev, B, N, K):
    _sampled_rows_check(dev, B, N, K, 4, 64, seed=N + K + B)


def test_c0_llama32_1b_up(dev):
    _sampled_rows_check(dev, 1, 8192, 2048, 4, 64, seed=0)


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_c2_prefill_2048(dev, N, K):
    _sampled_rows_check(dev, 2048, N, K, 4, 64, seed=N, n_rows=64)


@pytest.mark.parametrize("bits,g", [(2, 64), (3, 64), (8, 64), (4, 32), (4, 128)])
@pytest.mark.parametrize("M", [1, 512])
def test_c3_qwen3_bit_group_sweep(dev, bits, g, M):
    for N, K in ((6144, 2048), (2048, 6144)):
        _sampled_rows_check(dev, M, N, K, bits, g, seed=bits * 100 + g + M, n_rows=128,
                            bias_noise=0.0)


# --- vocabulary-sized single-row products (the streaming decode kernel) ------

@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("bits,g", [(4, 64), (4, 32), (4, 128), (2, 64), (3, 64), (8, 64)])
@pytest.mark.parametrize("K", [2048, 8192])
def test_wide_single_row(dev, dt, bits, g, K):
    """M = 1 with >= 2048 row tiles (N = 32771: the last tile is partial) takes
    the one-block-per-tile streaming kernel; sampled rows against the oracle."""
    tdt, odt = (torch.bfloat16, O.BF16) if dt == "bf16" else (torch.float16, O.F16)
    N = 32771
    seed = 7000 + K + 10 * bits + g
    W, S, B = gen.torch_quantized(seed, N, K, bits, g, dev, dtype=tdt)
    X = gen.torch_x(seed + 1, (1, K), dev, dtype=tdt)
    Y = ops.quantized_matmul(X, W, S, B, True, g, bits)
    torch.cuda.synchronize()
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, N - 16, N - 1], rng.integers(0, N, 256)]))
    rt = torch.from_numpy(rows).to(dev)
    w = W[rt].cpu().numpy().view(np.uint32)
    s = S[rt].cpu().view(torch.int16).numpy().view(np.uint16)
    b = B[rt].cpu().view(torch.int16).numpy().view(np.uint16)
    x = X.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = O.qmm_f64(x, odt, w, s, b, odt, g, bits)
    err = rel_err(to_host_f64(Y[:, rt]), ref)
    assert err <= TOL[odt], (N, K, bits, g, dt, err)


# --- two to eight rows of x at K >= 3072 (the streaming decode kernel) ---------

@pytest.mark.parametrize("M", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("bits,g", [(4, 64), (4, 32), (4, 128), (2, 64), (3, 64), (8, 64)])
@pytest.mark.parametrize("N,K", [(301, 3072), (130, 4096), (77, 14336), (4099, 8192)])
def test_few_rows_streaming(dev, M, dt, bits, g, N, K):
    """M = 2..8 with K a multiple of 1024 above 2048 (the streaming kernel:
    512-element K ranges at K <= 4096, 1024 above, two per wave above 8192;
    the persistent kernel where it is not used); N not a multiple of the
    16-row tile."""
    _qmm_check(dev, M, N, K, bits, g, dt, dt, seed=N + K + bits * 7 + g + M)


# --- 9..127 rows (batched decode of many requests, short prefill chunks) ----

@pytest.mark.parametrize("M", [9, 16, 33, 100, 127])
@pytest.mark.parametrize("bits,g", [(4, 64), (3, 32), (8, 128), (2, 64)])
def test_qmm_mid_rows_on_the_gemm(dev, M, bits, g):
    """Between the GEMV kernels' 8 rows and a full 128-row tile the product
    runs on the large-tile GEMM (ragged rows, split K); sampled rows vs the
    oracle."""
    _sampled_rows_check(dev, M, 1000, 2048, bits, g, seed=M * 13 + bits + g, n_rows=64)


@pytest.mark.parametrize("N,K", [(8200, 2048), (9000, 4096), (40008, 2048)])
@pytest.mark.parametrize("dt,g", [(O.BF16, 64), (O.F16, 128)])
def test_qmv_eight_rows_streaming_form(dev, N, K, dt, g):
    """8 rows of 4-bit weights with many output tiles run on the streaming
    kernel's batched form (x for the whole K in LDS, two waves per tile);
    ragged N (the last tile clamped), both 16-bit dtypes, groups 64 and 128;
    N = 40008 gives a block more tile groups than its waves hold at once (2,501
    tiles over at most one block per CU: a tile count per block that is not a
    multiple of 4, and blocks past the last tile); every output row of 96
    sampled weight rows vs the oracle."""
    w, s, b = quant(N + K, N, K, 4, g, dt)
    x = x_of(N + 1, (8, K), dt)
    y = ops.quantized_matmul(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                             to_dev(b, dt, dev), True, g, 4)
    rows = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(N).integers(0, N, 96)]))
    ref = O.qmm_f64(x, dt, w[rows], s[rows], b[rows], dt, g, 4)
    got = to_host_f64(y)[:, rows]
    assert rel_err(got, ref) <= 1e-2


@pytest.mark.parametrize("bits,g", [(4, 64), (3, 32), (8, 128), (2, 64)])
def test_qgemm_224_row_tiles(dev, bits, g):
    """A product the tile cost model gives 224 x 256 tiles (the last 32
    threads' W rows unused): N not a multiple of 224 and M not of 256 (ragged
    tiles both ways); sampled rows vs the oracle."""
    _sampled_rows_check(dev, 544, 13321, 1024, bits, g, seed=224 + bits + g, n_rows=96)


@pytest.mark.parametrize("M,N,K", [(137, 10990, 1024), (512, 6144, 2048)])
@pytest.mark.parametrize("bits,g", [(4, 64), (3, 32), (8, 128), (2, 64)])
def test_qgemm_96_row_tiles(dev, M, N, K, bits, g):
    """Products the tile cost model gives 96 x 128 split-K tiles (the last 32
    threads' W rows unused): ragged N and M, and the configs[3] gate/up
    shape; sampled rows vs the oracle."""
    _sampled_rows_check(dev, M, N, K, bits, g, seed=96 + M + bits + g, n_rows=96)


@pytest.mark.parametrize("M", [65, 100, 128])
@pytest.mark.parametrize("bits,g", [(4, 64), (3, 32), (8, 128)])
def test_qgemm_64x128_tiles(dev, M, bits, g):
    """65-128 rows against many W rows run on 64 x 128 tiles with K split
    over 2 wave groups (half the threads without a W row): ragged N and M;
    sampled rows vs the oracle."""
    _sampled_rows_check(dev, M, 14000, 1024, bits, g, seed=192 + M + bits + g, n_rows=96)


@pytest.mark.parametrize("M", [4, 5])
def test_qmv_few_rows_vocabulary_dense_form(dev, M):
    """4-7 rows against a vocabulary-sized N run on the streaming kernel's
    dense form (16 row slots, only M of them staged); 66,000 rows give 17
    tiles per block; sampled weight rows vs the oracle."""
    N, K, dt, g = 66000, 2048, O.BF16, 64
    w, s, b = quant(N + M, N, K, 4, g, dt)
    x = x_of(M, (M, K), dt)
    y = ops.quantized_matmul(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                             to_dev(b, dt, dev), True, g, 4)
    rows = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(N + M).integers(0, N, 96)]))
    ref = O.qmm_f64(x, dt, w[rows], s[rows], b[rows], dt, g, 4)
    assert rel_err(to_host_f64(y)[:, rows], ref) <= 1e-2


@pytest.mark.parametrize("M,K,g", [(9, 4096, 64), (12, 2048, 128), (16, 4096, 64)])
def test_qmm_nine_to_sixteen_rows_dense_form(dev, M, K, g):
    """9-16 rows of 4-bit weights with a ragged N of 14,003 rows run the
    streaming kernel's dense form in place of the GEMM's 64 x 64 tiles;
    sampled weight rows vs the oracle."""
    N, dt = 14003, O.BF16
    w, s, b = quant(N + M + K, N, K, 4, g, dt)
    x = x_of(M + K, (M, K), dt)
    y = ops.quantized_matmul(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                             to_dev(b, dt, dev), True, g, 4)
    rows = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(N + M).integers(0, N, 96)]))
    ref = O.qmm_f64(x, dt, w[rows], s[rows], b[rows], dt, g, 4)
    assert rel_err(to_host_f64(y)[:, rows], ref) <= 1e-2


def test_qmm_nine_to_sixteen_rows_dense_form_f16(dev):
    """14 rows, fp16 x and scales, 8,200 W rows (the smallest N the dense
    form takes, ragged), K = 4096 group 128; sampled rows vs the oracle."""
    M, N, K, g, dt = 14, 8200, 4096, 128, O.F16
    w, s, b = quant(M + N, N, K, 4, g, dt)
    x = x_of(M + 3, (M, K), dt)
    y = ops.quantized_matmul(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                             to_dev(b, dt, dev), True, g, 4)
    assert y.dtype == torch.float16
    rows = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(N).integers(0, N, 96)]))
    ref = O.qmm_f64(x, dt, w[rows], s[rows], b[rows], dt, g, 4)
    assert rel_err(to_host_f64(y)[:, rows], ref) <= 1e-2


@pytest.mark.parametrize("M,N,K,bits,g", [(20, 1000, 4096, 4, 64), (31, 1000, 4096, 4, 64),
                                         (12, 2000, 4096, 8, 128), (9, 4100, 4096, 2, 32),
                                         (17, 6000, 4096, 3, 64)])
def test_qmm_few_output_tiles_gemv_launches(dev, M, N, K, bits, g):
    """9-32 rows against few W rows run as ceil(M / 8) GEMV launches (the
    last one ragged: 4, 7, 1 and 1 rows here); sampled rows vs the oracle."""
    _sampled_rows_check(dev, M, N, K, bits, g, seed=M + N + bits, n_rows=96)


def test_qmm_few_output_tiles_gemv_launches_f16(dev):
    _qmm_check(dev, 12, 300, 4096, 4, 64, O.F16, O.F16, seed=12)


@pytest.mark.parametrize("M,N,K,bits,g", [
    (M, N, K, bits, g)
    for (M, N, K) in [(803, 14653, 1024), (285, 10990, 1024), (803, 9325, 1024),
                      (137, 12322, 1024), (137, 8326, 1024), (100, 1000, 1088)]
    for (bits, g) in [(4, 64), (3, 32), (8, 128)] if K % g == 0])
def test_qgemm_every_tile_form(dev, M, N, K, bits, g):
    """The tile cost model's other forms, each on a shape that picks it with
    ragged N and M (on 256 CUs): 256 x 256, 256 x 128, 128 x 128 without and
    with split-K, 64 x 64 with K split over 2 groups, and 64 x 64 without
    split-K (K / 64 odd, so no group of 128); sampled rows vs the oracle."""
    _sampled_rows_check(dev, M, N, K, bits, g, seed=M + N + K + 7 * bits, n_rows=96)


@pytest.mark.parametrize("M", [4, 8])
@pytest.mark.parametrize("N", [1003, 520])
def test_qmv_few_w_rows_eight_row_tiles(dev, M, N):
    """4 and 8 x rows against at most 1024 W rows run the streaming GEMV on
    8-row tiles (the MFMA's other 8 columns repeat them, unstored): ragged
    last tile; every row vs the oracle."""
    _sampled_rows_check(dev, M, N, 4096, 4, 64, seed=N + 8 * M, n_rows=N)


# --- prefill GEMM with K split inside the block (few output tiles) -----------

@pytest.mark.parametrize("M,N,K", [(300, 1000, 2048), (129, 4000, 1536), (512, 8000, 1024),
                                   (256, 2048, 6144), (128, 128, 128)])
@pytest.mark.parametrize("bits,g", [(4, 64), (3, 32), (8, 128)])
def test_qgemm_split_k(dev, M, N, K, bits, g):
    """Products with fewer 128-row tiles than CUs split K over 2 or 4 wave
    groups of a block (ragged M and N included); sampled rows vs the oracle."""
    _sampled_rows_check(dev, M, N, K, bits, g, seed=M + N + K + bits, n_rows=96)
