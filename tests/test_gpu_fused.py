"""Fused SwiGLU entry points and the on-device MoE block, through the C ABI
(via the torch facade), against the CPU oracle.

References in higgs:
* dense_hidden_fused (crates/higgs-models/src/qwen3_next.rs:2539-2585): one
  quantized_matmul over gate||up, split, silu_mul; the in-tree check
  qwen3_next.rs:13132-13169 asserts fused == separate.
* forward_gather_global_sort (qwen3_next.rs:1731-1809) and the MoE combine
  (qwen3_moe.rs:353-357); qwen3_next.rs:4431-4530 asserts the global-sort
  path equals the plain gather path.

Bars: integer index outputs bit-exact; bf16/fp16 outputs within max relative
error 1e-2 of the oracle (gate and up rounded to the output dtype, swiglu in
fp64, rounded once).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import TORCH_DT, idx_dev, quant, rel_err, to_dev, to_host_bits, to_host_f64, \
    words_dev, x_of
from higgs_amd import _lib, gen, ops

pytestmark = pytest.mark.gpu


def _round(v64, dt):
    return O.from_f32(v64.astype(np.float32), dt) if dt != O.F32 else v64.astype(np.float32)


def _swiglu_ref(x, xdt, wg, sg, bg, wu, su, bu, g, bits):
    """fp64 gate/up, each rounded to the output dtype, oracle swiglu (one rounding)."""
    gate = _round(O.qmm_f64(x, xdt, wg, sg, bg, xdt, g, bits), xdt)
    up = _round(O.qmm_f64(x, xdt, wu, su, bu, xdt, g, bits), xdt)
    h = O.swiglu(gate, up, xdt)
    return O.to_f32(h, xdt).astype(np.float64)


def _dense_case(seed, M, N, K, bits, g, dt):
    w, s, b = quant(seed, 2 * N, K, bits, g, dt)
    x = x_of(seed + 5, (M, K), dt)
    return x, w, s, b


@pytest.mark.parametrize("M", [1, 2, 5, 8, 11, 12, 20, 33, 127, 256])
@pytest.mark.parametrize("bits,g", [(4, 64), (3, 32), (8, 128)])
def test_dense_hidden_fused_matches_oracle(dev, M, bits, g):
    N, K, dt = 200, 1024, O.BF16
    x, w, s, b = _dense_case(M * 10 + bits, M, N, K, bits, g, dt)
    h = ops.dense_hidden_fused(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                               to_dev(b, dt, dev), N, g, bits)
    assert tuple(h.shape) == (M, N) and h.dtype == torch.bfloat16
    ref = _swiglu_ref(x, dt, w[:N], s[:N], b[:N], w[N:], s[N:], b[N:], g, bits)
    assert rel_err(to_host_f64(h), ref) <= 1e-2


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("K", [3072, 4096, 12288])
@pytest.mark.parametrize("bits,g", [(4, 64), (4, 32), (8, 128)])
def test_dense_hidden_fused_streaming(dev, M, K, bits, g):
    # K a multiple of 1024 above 2048: the streaming kernel with the gate and
    # up halves in one block (M = 1, 2; M = 4, 8 at K <= 4096), the persistent
    # kernel otherwise; N = 200 leaves a partial 16-row tile.
    N, dt = 200, O.BF16
    x, w, s, b = _dense_case(K + M * 10 + bits, M, N, K, bits, g, dt)
    h = ops.dense_hidden_fused(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                               to_dev(b, dt, dev), N, g, bits)
    assert tuple(h.shape) == (M, N) and h.dtype == torch.bfloat16
    ref = _swiglu_ref(x, dt, w[:N], s[:N], b[:N], w[N:], s[N:], b[N:], g, bits)
    assert rel_err(to_host_f64(h), ref) <= 1e-2


@pytest.mark.parametrize("M", [1, 8, 300])
def test_dense_hidden_fused_f16(dev, M):
    N, K, dt, bits, g = 136, 2048, O.F16, 4, 64
    x, w, s, b = _dense_case(77 + M, M, N, K, bits, g, dt)
    h = ops.dense_hidden_fused(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                               to_dev(b, dt, dev), N, g, bits)
    assert h.dtype == torch.float16
    ref = _swiglu_ref(x, dt, w[:N], s[:N], b[:N], w[N:], s[N:], b[N:], g, bits)
    assert rel_err(to_host_f64(h), ref) <= 1e-2


def test_fused_swiglu_on_64x128_tiles(dev):
    """100 rows against 6000 gate/up columns: the fused GEMM on 64 x 128
    tiles with split-K (32 output columns per tile, ragged N and M)."""
    M, N, K, dt, bits, g = 100, 6000, 1024, O.BF16, 4, 64
    x, w, s, b = _dense_case(640 + M, M, N, K, bits, g, dt)
    h = ops.dense_hidden_fused(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                               to_dev(b, dt, dev), N, g, bits)
    ref = _swiglu_ref(x, dt, w[:N], s[:N], b[:N], w[N:], s[N:], b[N:], g, bits)
    assert rel_err(to_host_f64(h), ref) <= 1e-2


@pytest.mark.parametrize("M", [64, 256, 512])
def test_fused_swiglu_gemm_tile_forms(dev, M):
    """The fused GEMM's tile forms at 14000 gate/up columns (ragged): 64 x 64
    with split-K (M = 64), 256 x 128 (M = 256) and 256 x 256 (M = 512), as
    the tile cost model picks them on 256 CUs; 96 sampled output columns vs
    the oracle."""
    N, K, dt, bits, g = 14000, 1024, O.BF16, 4, 64
    x, w, s, b = _dense_case(900 + M, M, N, K, bits, g, dt)
    h = ops.dense_hidden_fused(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                               to_dev(b, dt, dev), N, g, bits)
    cols = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(M).integers(0, N, 96)]))
    ref = _swiglu_ref(x, dt, w[cols], s[cols], b[cols], w[N + cols], s[N + cols], b[N + cols], g, bits)
    assert rel_err(to_host_f64(h)[:, cols], ref) <= 1e-2


@pytest.mark.parametrize("M", [8, 9, 12, 16])
@pytest.mark.parametrize("K,g", [(4096, 64), (2048, 128)])
def test_fused_swiglu_dense_streaming_form(dev, M, K, g):
    """8-16 rows against 14,003 gate/up columns (ragged) of 4-bit weights:
    the streaming kernel's dense form with both projections per tile (group
    sums strided for its 16 rows); 96 sampled output columns vs the oracle."""
    N, dt, bits = 14003, O.BF16, 4
    x, w, s, b = _dense_case(1700 + M + K, M, N, K, bits, g, dt)
    h = ops.dense_hidden_fused(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                               to_dev(b, dt, dev), N, g, bits)
    cols = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(M + K).integers(0, N, 96)]))
    ref = _swiglu_ref(x, dt, w[cols], s[cols], b[cols], w[N + cols], s[N + cols], b[N + cols], g, bits)
    assert rel_err(to_host_f64(h)[:, cols], ref) <= 1e-2


@pytest.mark.parametrize("M", [8, 13])
def test_fused_swiglu_dense_streaming_form_f16(dev, M):
    """The same dense form with fp16 x and scales (K = 2048, group 64)."""
    N, K, dt, bits, g = 9000, 2048, O.F16, 4, 64
    x, w, s, b = _dense_case(1800 + M, M, N, K, bits, g, dt)
    h = ops.dense_hidden_fused(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                               to_dev(b, dt, dev), N, g, bits)
    assert h.dtype == torch.float16
    cols = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(M).integers(0, N, 96)]))
    ref = _swiglu_ref(x, dt, w[cols], s[cols], b[cols], w[N + cols], s[N + cols], b[N + cols], g, bits)
    assert rel_err(to_host_f64(h)[:, cols], ref) <= 1e-2


def _host_rows(W, S, B, cols, dev):
    ct = torch.from_numpy(cols).to(dev)
    return (W[ct].cpu().numpy().view(np.uint32), S[ct].cpu().view(torch.int16).numpy().view(np.uint16),
            B[ct].cpu().view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("M", [4, 7])
def test_fused_swiglu_dense_form_vocabulary_n(dev, M):
    """4-7 rows against 65,600 gate/up columns (K = 2048) take the dense form
    with both projections per tile; weights made on the device, 96 sampled
    output columns vs the oracle."""
    N, K, g, bits = 65600, 2048, 64, 4
    G = gen.torch_quantized(2000 + M, N, K, bits, g, dev)
    U = gen.torch_quantized(3000 + M, N, K, bits, g, dev)
    X = gen.torch_x(4000 + M, (M, K), dev)
    h = ops.swiglu_pair(X, G, U, g, bits)
    torch.cuda.synchronize()
    cols = np.unique(np.concatenate([[0, N - 1], np.random.default_rng(M).integers(0, N, 96)]))
    x = X.cpu().view(torch.int16).numpy().view(np.uint16)
    wg, sg, bg = _host_rows(*G, cols, dev)
    wu, su, bu = _host_rows(*U, cols, dev)
    ref = _swiglu_ref(x, O.BF16, wg, sg, bg, wu, su, bu, g, bits)
    assert rel_err(to_host_f64(h)[:, cols], ref) <= 1e-2


@pytest.mark.parametrize("M", [1, 2, 4, 256])
def test_fused_equals_separate(dev, M):
    # qwen3_next.rs:13132-13169: fused gate||up == separate projections
    N, K, dt, bits, g = 512, 4096, O.BF16, 4, 64
    x, w, s, b = _dense_case(300 + M, M, N, K, bits, g, dt)
    xd, wd, sd, bd = to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev), to_dev(b, dt, dev)
    h = ops.dense_hidden_fused(xd, wd, sd, bd, N, g, bits)
    gate = ops.quantized_matmul(xd, wd[:N], sd[:N], bd[:N], True, g, bits)
    up = ops.quantized_matmul(xd, wd[N:], sd[N:], bd[N:], True, g, bits)
    sep = ops.swiglu(gate, up)
    a, r = h.float(), sep.float()
    assert (a - r).abs().max().item() <= 1e-2 * r.abs().max().item()


def test_unsupported_shape_runs_unfused(dev):
    # K = 768 is not a multiple of 1024: the C entry declines, the facade runs
    # two quantized_matmul calls and swiglu, with the same result contract.
    N, K, dt, bits, g, M = 96, 768, O.BF16, 4, 64, 3
    x, w, s, b = _dense_case(901, M, N, K, bits, g, dt)
    xd, wd, sd, bd = to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev), to_dev(b, dt, dev)
    rc = _lib.lib().hq_quantized_matmul_swiglu(
        0x1000, xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), wd[N:].data_ptr(),
        sd[N:].data_ptr(), bd[N:].data_ptr(), M, N, K, g, bits, dt, dt, None)
    assert rc == _lib.HQ_ERR_UNSUPPORTED and "K=768" in _lib.last_error()
    h = ops.dense_hidden_fused(xd, wd, sd, bd, N, g, bits)
    ref = _swiglu_ref(x, dt, w[:N], s[:N], b[:N], w[N:], s[N:], b[N:], g, bits)
    assert rel_err(to_host_f64(h), ref) <= 1e-2


def test_swiglu_elementwise_matches_oracle(dev):
    for dt in (O.BF16, O.F16, O.F32):
        gt = x_of(5, (3000,), dt)
        ut = x_of(6, (3000,), dt)
        out = ops.swiglu(to_dev(gt, dt, dev), to_dev(ut, dt, dev))
        ref = O.to_f32(O.swiglu(gt, ut, dt), dt) if dt != O.F32 else O.swiglu(gt, ut, dt)
        got = out.float().cpu().numpy()
        # float32 evaluation, one rounding: at most one ulp of the output dtype
        ulp = {O.BF16: 2 ** -7, O.F16: 2 ** -10, O.F32: 2 ** -19}[dt]
        assert np.all(np.abs(got - ref) <= ulp * np.maximum(np.abs(ref), 1e-30) + 1e-30)


# --- MoE -----------------------------------------------------------------------

@pytest.mark.parametrize("n,E", [(1, 1), (7, 4), (1000, 8), (1024, 128), (1025, 128),
                                 (3000, 2), (4096, 128), (16384, 64), (16385, 64),
                                 (33000, 512), (5000, 2048)])
def test_moe_sort_is_the_stable_argsort(dev, n, E):
    rng = np.random.default_rng(n + E)
    k = 8 if n % 8 == 0 else 1
    idx = rng.integers(0, E, n).astype(np.uint32)
    order, inv, srt, tok = ops.moe_sort(idx_dev(idx, dev).reshape(-1, k), E)
    o_order, o_inv, o_srt, o_tok = O.gather_sort(idx, k)
    for got, ref in ((order, o_order), (inv, o_inv), (srt, o_srt), (tok, o_tok)):
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref)


def test_moe_sort_out_of_range_indices_go_last_in_order(dev):
    idx = np.array([3, 200, 1, 7, 150, 0, 3, 9, 200, 2], np.uint32)
    E = 8
    order, inv, srt, tok = ops.moe_sort(idx_dev(idx, dev).reshape(-1, 2), E)
    clamped = np.minimum(idx, E)
    o_order, o_inv, _, o_tok = O.gather_sort(clamped, 2)
    np.testing.assert_array_equal(order.cpu().numpy().view(np.uint32), o_order)
    np.testing.assert_array_equal(inv.cpu().numpy().view(np.uint32), o_inv)
    np.testing.assert_array_equal(srt.cpu().numpy().view(np.uint32), idx[o_order])
    np.testing.assert_array_equal(tok.cpu().numpy().view(np.uint32), o_tok)


def test_moe_combine_matches_oracle(dev):
    tokens, k, E, D = 300, 8, 64, 200
    idx = gen.topk_routing(4, tokens, E, k)
    order, inv, srt, tok = O.gather_sort(idx, k)
    y = gen.np_x_bf16(8, (tokens * k, D))
    sc = gen.np_x_bf16(9, (tokens, k))
    out = ops.moe_combine(to_dev(y, O.BF16, dev), idx_dev(inv, dev), to_dev(sc, O.BF16, dev))
    ref = O.moe_combine(y, O.BF16, inv, sc, O.BF16)
    got = to_host_bits(out)
    # fp32 vs fp64 sum of the rounded products: equal, or one bf16 ulp apart
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99
    # unit scores, top_k = 1: an exact row permutation (the unsort)
    ones = torch.ones((tokens * k, 1), dtype=torch.bfloat16, device=dev)
    back = ops.moe_combine(to_dev(y, O.BF16, dev), idx_dev(inv, dev), ones)
    np.testing.assert_array_equal(to_host_bits(back), y[inv])


def _moe_weights(seed, E, D, I, bits, g, dev):
    gw, gs, gb = gen.torch_quantized(seed, I, D, bits, g, dev, lead=(E,))
    uw, us, ub = gen.torch_quantized(seed + 1, I, D, bits, g, dev, lead=(E,))
    dw, ds, db = gen.torch_quantized(seed + 2, D, I, bits, g, dev, lead=(E,))
    return (gw, gs, gb), (uw, us, ub), (dw, ds, db)


def test_gather_qmm_swiglu_equals_separate(dev):
    tokens, k, E, D, I, bits, g = 96, 4, 16, 512, 320, 4, 64
    gate, up, _ = _moe_weights(60, E, D, I, bits, g, dev)
    idx = gen.topk_routing(61, tokens, E, k)
    order, inv, srt, tok = O.gather_sort(idx, k)
    x = gen.torch_x(62, (tokens, 1, D), dev)
    h = ops.gather_qmm_swiglu(x, gate, up, idx_dev(tok, dev), idx_dev(srt, dev), g, bits)
    xs = x[torch.from_numpy(tok.astype(np.int64)).to(dev)]
    gg = ops.gather_qmm(xs, *gate, None, idx_dev(srt, dev), True, g, bits, True)
    uu = ops.gather_qmm(xs, *up, None, idx_dev(srt, dev), True, g, bits, True)
    sep = ops.swiglu(gg, uu)
    a, r = h.float(), sep.float()
    assert tuple(h.shape) == (tokens * k, 1, I)
    assert (a - r).abs().max().item() <= 1e-2 * r.abs().max().item()


def test_moe_block_c4_matches_oracle_on_sampled_tokens(dev):
    # 512 tokens, top-8 of 128 experts, D 2048, I 768, 4-bit g64
    tokens, k, E, D, I, bits, g = 512, 8, 128, 2048, 768, 4, 64
    gate, up, down = _moe_weights(70, E, D, I, bits, g, dev)
    idx = gen.topk_routing(71, tokens, E, k)
    x = gen.torch_x(72, (1, tokens, D), dev)
    sc = torch.softmax(gen.torch_x(73, (1, tokens, k), dev).float(), -1).to(torch.bfloat16)
    out = ops.moe_block(x, idx_dev(idx, dev).reshape(1, tokens, k), sc, gate, up, down, g, bits)
    assert tuple(out.shape) == (1, tokens, D)
    xs, scs = to_host_bits(x).reshape(tokens, D), to_host_bits(sc).reshape(tokens, k)
    W = [(w.cpu().numpy().view(np.uint32), to_host_bits(s), to_host_bits(b))
         for (w, s, b) in (gate, up, down)]
    got = to_host_f64(out).reshape(tokens, D)
    for t in (0, 1, 77, 255, 256, 400, 511):
        ys = []
        for j in range(k):
            e = int(idx[t, j])
            h = O.from_f32(_swiglu_ref(xs[t:t + 1], O.BF16, W[0][0][e], W[0][1][e], W[0][2][e],
                                       W[1][0][e], W[1][1][e], W[1][2][e], g, bits)
                           .astype(np.float32), O.BF16)
            ys.append(_round(O.qmm_f64(h, O.BF16, W[2][0][e], W[2][1][e], W[2][2][e], O.BF16,
                                       g, bits), O.BF16)[0])
        y = np.stack(ys)                                          # [k, D] sorted-free
        ref = O.moe_combine(y, O.BF16, np.arange(k, dtype=np.uint32), scs[t:t + 1], O.BF16)
        assert rel_err(got[t], O.to_f32(ref, O.BF16)[0].astype(np.float64)) <= 1e-2, t


def test_global_sort_block_equals_plain_gather_path(dev):
    # qwen3_next.rs:4431-4530: forward_gather_global_sort == forward_gather
    B, L, k, E, D, I, bits, g = 2, 40, 4, 16, 256, 192, 4, 64
    gate, up, down = _moe_weights(80, E, D, I, bits, g, dev)
    idx = gen.topk_routing(81, B * L, E, k).reshape(B, L, k)
    x = gen.torch_x(82, (B, L, D), dev)
    fast = ops.forward_gather_global_sort(x, idx_dev(idx, dev), gate, up, down, g, bits)
    assert tuple(fast.shape) == (B, L, k, D)
    # forward_gather (qwen3_next.rs:1660-1720): x [B,L,1,1,D] against idx [B,L,k]
    xi = x.reshape(B, L, 1, 1, D)
    ii = idx_dev(idx, dev)
    gg = ops.gather_qmm(xi, *gate, None, ii, True, g, bits, False)
    uu = ops.gather_qmm(xi, *up, None, ii, True, g, bits, False)
    dd = ops.gather_qmm(ops.swiglu(gg, uu), *down, None, ii, True, g, bits, False)
    plain = dd.reshape(B, L, k, D)
    a, r = fast.float(), plain.float()
    assert (a - r).abs().max().item() <= 1e-2 * r.abs().max().item()
