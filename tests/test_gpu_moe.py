"""gather_qmm on the MoE global-sort path (Qwen3-30B-A3B
style, 128 experts, top-8 of 512 tokens, hidden 2048, expert intermediate 768,
4-bit g64), through the C ABI via the torch facade, against the CPU oracle.

The reference's own checks are relational (crates/higgs-models/src/
qwen3_next.rs:4344-4398 gather == per-expert quantized_matmul;
4431-4530 global-sort == unsorted path); these tests assert the same
relations plus absolute parity with the fp64 oracle on sampled rows
(max|y-r| / max|r| <= 1e-2 for bf16 output).
"""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import idx_dev, rel_err, to_host_bits
from higgs_amd import gen, ops

pytestmark = pytest.mark.gpu

TOKENS, TOPK, E, HID, INTER, G, BITS = 512, 8, 128, 2048, 768, 64, 4


def _host(t):
    return to_host_bits(t)


def _routing(seed=3):
    idx = gen.topk_routing(seed, TOKENS, E, TOPK)           # [512, 8]
    order, inv, srt, tok = O.gather_sort(idx, TOPK)          # qwen3_next.rs:1748-1761
    return idx, order, inv, srt, tok


def _oracle_rows(xs, W, S, B, idx_rows, rows, N, K):
    """fp64 reference for the sampled rows: y[i] = x_sorted[i] . deq(W[idx[i]])^T."""
    w = W.cpu().numpy().view(np.uint32)
    s = S.cpu().view(torch.int16).numpy().view(np.uint16)
    b = B.cpu().view(torch.int16).numpy().view(np.uint16)
    x = xs.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1, K)
    out = np.empty((len(rows), N))
    for j, r in enumerate(rows):
        e = int(idx_rows[r])
        out[j] = O.qmm_f64(x[r:r + 1], O.BF16, w[e], s[e], b[e], O.BF16, G, BITS)[0]
    return out


@pytest.mark.parametrize("which", ["gate", "down"])
def test_c4_sorted_gather_matches_oracle(dev, which):
    N, K = (INTER, HID) if which == "gate" else (HID, INTER)
    idx, order, inv, srt, tok = _routing()
    W, S, B = gen.torch_quantized(40, N, K, BITS, G, dev, lead=(E,))
    x = gen.torch_x(41, (TOKENS, K), dev)
    xs = x[torch.from_numpy(tok.astype(np.int64)).to(dev)].reshape(-1, 1, K)
    y = ops.gather_qmm(xs, W, S, B, None, idx_dev(srt, dev), True, G, BITS, True)
    assert tuple(y.shape) == (TOKENS * TOPK, 1, N)
    rng = np.random.default_rng(5)
    # every expert's first and last row plus random rows
    firsts = np.searchsorted(srt, np.arange(E))
    lasts = np.searchsorted(srt, np.arange(E), side="right") - 1
    rows = np.unique(np.concatenate([firsts[firsts < len(srt)], lasts[lasts >= 0],
                                     rng.integers(0, len(srt), 64)]))
    ref = _oracle_rows(xs, W, S, B, srt, rows, N, K)
    got = y.float().cpu().numpy().reshape(-1, N)[rows].astype(np.float64)
    assert rel_err(got, ref) <= 1e-2


def test_c4_sorted_equals_unsorted_and_unsort_roundtrip(dev):
    # qwen3_next.rs:4431-4530: the global-sort path equals the plain path.
    idx, order, inv, srt, tok = _routing(7)
    W, S, B = gen.torch_quantized(42, INTER, HID, BITS, G, dev, lead=(E,))
    x = gen.torch_x(43, (TOKENS, HID), dev)
    # plain path (forward_gather, qwen3_next.rs:1660-1720): x [L,1,1,D] vs idx [L,k]
    base = ops.gather_qmm(x.reshape(TOKENS, 1, 1, HID), W, S, B, None,
                          idx_dev(idx, dev), True, G, BITS, False)      # [512, 8, 1, 768]
    xs = x[torch.from_numpy(tok.astype(np.int64)).to(dev)].reshape(-1, 1, HID)
    ys = ops.gather_qmm(xs, W, S, B, None, idx_dev(srt, dev), True, G, BITS, True)
    unsorted = ys.reshape(-1, INTER)[torch.from_numpy(inv.astype(np.int64)).to(dev)]
    a = unsorted.float()
    b = base.reshape(-1, INTER).float()
    assert (a - b).abs().max().item() <= 1e-2 * b.abs().max().item()


def test_sorted_gather_via_lhs_indices_equals_materialized(dev):
    # Fusing the token gather into gather_qmm (lhs_indices = token of each
    # sorted row) gives exactly the materialized x_sorted result.
    idx, order, inv, srt, tok = _routing(9)
    W, S, B = gen.torch_quantized(44, INTER, HID, BITS, G, dev, lead=(E,))
    x = gen.torch_x(45, (TOKENS, HID), dev)
    xs = x[torch.from_numpy(tok.astype(np.int64)).to(dev)].reshape(-1, 1, HID)
    y1 = ops.gather_qmm(xs, W, S, B, None, idx_dev(srt, dev), True, G, BITS, True)
    y2 = ops.gather_qmm(x.reshape(TOKENS, 1, HID), W, S, B, idx_dev(tok, dev),
                        idx_dev(srt, dev), True, G, BITS, True)
    assert torch.equal(y1, y2)


def test_sorted_gather_out_of_range_rows_are_nan(dev):
    N, K, Ex = 128, 256, 4
    W, S, B = gen.torch_quantized(46, N, K, BITS, G, dev, lead=(Ex,))
    x = gen.torch_x(47, (10, 1, K), dev)
    rhs = np.array([0, 0, 1, 2, 2, 2, 3, 9, 9, 11], np.uint32)   # last 3 out of range
    y = ops.gather_qmm(x, W, S, B, None, idx_dev(rhs, dev), True, G, BITS, True)
    assert torch.isnan(y[7:]).all() and not torch.isnan(y[:7]).any()
    ref = O.gather_qmm_f64(_host(x), O.BF16, W.cpu().numpy().view(np.uint32),
                           _host(S), _host(B), O.BF16, np.arange(7, dtype=np.uint32), rhs[:7],
                           1, N, K, G, BITS, x_batch=10)
    assert rel_err(y[:7].float().cpu().numpy().astype(np.float64), ref) <= 1e-2
    lhs = np.array([0, 1, 2, 3, 4, 5, 77, 7, 8, 9], np.uint32)    # x index 77 out of range
    y2 = ops.gather_qmm(x, W, S, B, idx_dev(lhs, dev), idx_dev(rhs, dev), True, G, BITS, True)
    assert torch.isnan(y2[6]).all() and not torch.isnan(y2[:6]).any()


@pytest.mark.parametrize("M", [1, 3])
def test_sorted_gather_small_matches_per_expert(dev, M):
    # qwen3_next.rs:4344-4398 on the sorted path, with M rows per element
    N, K, Ex = 192, 512, 6
    W, S, B = gen.torch_quantized(48, N, K, BITS, G, dev, lead=(Ex,))
    rhs = np.array([0, 1, 1, 1, 4, 4, 5], np.uint32)
    x = gen.torch_x(49, (len(rhs), M, K), dev)
    y = ops.gather_qmm(x, W, S, B, None, idx_dev(rhs, dev), True, G, BITS, True)
    for i, e in enumerate(rhs):
        one = ops.quantized_matmul(x[i], W[e], S[e], B[e], True, G, BITS)
        assert (y[i].float() - one.float()).abs().max().item() <= 1e-2 * one.float().abs().max().item()


def _block_oracle(x_bits, idx, scs, projs, tokens_to_check):
    """fp64 expert block for a few tokens with per-projection (group, bits):
    gate/up rounded to bf16, swiglu, down rounded, then the oracle combine."""
    (gw, gs, gb, gg, gbits), (uw, us, ub, ug, ubits), (dw, ds, db, dg, dbits) = projs
    out = {}
    k = idx.shape[1]
    for t in tokens_to_check:
        ys = []
        for j in range(k):
            e = int(idx[t, j])
            g = O.from_f32(O.qmm_f64(x_bits[t:t + 1], O.BF16, gw[e], gs[e], gb[e], O.BF16, gg,
                                     gbits).astype(np.float32), O.BF16)
            u = O.from_f32(O.qmm_f64(x_bits[t:t + 1], O.BF16, uw[e], us[e], ub[e], O.BF16, ug,
                                     ubits).astype(np.float32), O.BF16)
            h = O.swiglu(g, u, O.BF16)
            ys.append(O.from_f32(O.qmm_f64(h, O.BF16, dw[e], ds[e], db[e], O.BF16, dg, dbits)
                                 .astype(np.float32), O.BF16)[0])
        ref = O.moe_combine(np.stack(ys), O.BF16, np.arange(k, dtype=np.uint32), scs[t:t + 1],
                            O.BF16)
        out[t] = O.to_f32(ref, O.BF16)[0].astype(np.float64)
    return out


@pytest.mark.parametrize("down_bits,down_g", [(8, 64), (4, 32)])
def test_moe_block_mixed_projection_widths(dev, down_bits, down_g):
    """A mixed-precision checkpoint quantizes switch_mlp.down_proj with other
    settings than gate/up; each gather_qmm uses its own projection's
    (qwen3_next.rs:1764-1800). SwitchGLU carries them per projection."""
    from higgs_amd import layers

    tokens, k, Ex, D, I = 64, 4, 16, 512, 256
    gate = gen.torch_quantized(90, I, D, 4, 64, dev, lead=(Ex,))
    up = gen.torch_quantized(91, I, D, 4, 64, dev, lead=(Ex,))
    down = gen.torch_quantized(92, D, I, down_bits, down_g, dev, lead=(Ex,))
    sw = layers.SwitchGLU(layers.QLinear(*gate, 64, 4), layers.QLinear(*up, 64, 4),
                          layers.QLinear(*down, down_g, down_bits))
    idx = gen.topk_routing(93, tokens, Ex, k)
    x = gen.torch_x(94, (1, tokens, D), dev)
    sc = torch.softmax(gen.torch_x(95, (1, tokens, k), dev).float(), -1).to(torch.bfloat16)
    out = sw.moe(x, idx_dev(idx, dev).reshape(1, tokens, k), sc)
    host = lambda t: (t[0].cpu().numpy().view(np.uint32), _host(t[1]), _host(t[2]))
    projs = (host(gate) + (64, 4), host(up) + (64, 4), host(down) + (down_g, down_bits))
    ref = _block_oracle(_host(x).reshape(tokens, D), idx, _host(sc).reshape(tokens, k), projs,
                        (0, 9, 33, 63))
    got = out.float().cpu().numpy().reshape(tokens, D).astype(np.float64)
    for t, r in ref.items():
        assert rel_err(got[t], r) <= 1e-2, t
    # mixed gate/up settings take the unfused gate/up path: same result
    sw2 = layers.SwitchGLU(layers.QLinear(*gate, 64, 4), layers.QLinear(*up, 64, 4),
                           layers.QLinear(*down, down_g, down_bits))
    y_sorted = sw2.forward_gather_global_sort(x.reshape(1, tokens, D),
                                              idx_dev(idx, dev).reshape(1, tokens, k))
    assert tuple(y_sorted.shape) == (1, tokens, k, D)


def test_switch_forward_gather_equals_global_sort(dev):
    """SwitchGLU.forward_gather (the unsorted path, qwen3_next.rs:1660-1720)
    equals forward_gather_global_sort (qwen3_next.rs:4431-4530 asserts it)."""
    from higgs_amd import layers

    B, L, k, Ex, D, I = 2, 24, 4, 8, 256, 192
    qs = [gen.torch_quantized(96 + j, *nk, 4, 64, dev, lead=(Ex,))
          for j, nk in enumerate(((I, D), (I, D), (D, I)))]
    sw = layers.SwitchGLU(*(layers.QLinear(*t, 64, 4) for t in qs))
    idx = idx_dev(gen.topk_routing(99, B * L, Ex, k).reshape(B, L, k), dev)
    x = gen.torch_x(100, (B, L, D), dev)
    a = sw.forward_gather(x, idx).float()
    b = sw.forward_gather_global_sort(x, idx).float()
    assert a.shape == b.shape == (B, L, k, D)
    assert (a - b).abs().max().item() <= 1e-2 * b.abs().max().item()


def test_gather_qmm_swiglu_float32_activations_fall_back(dev):
    """fp32 activations are outside the fused grouped kernel: the facade runs
    the reference's own form (two sorted gather_qmm calls and swiglu)."""
    tokens, k, Ex, D, I = 32, 2, 4, 256, 128
    gate = gen.torch_quantized(101, I, D, 4, 64, dev, lead=(Ex,), dtype=torch.float32)
    up = gen.torch_quantized(102, I, D, 4, 64, dev, lead=(Ex,), dtype=torch.float32)
    idx = gen.topk_routing(103, tokens, Ex, k)
    order, inv, srt, tok = O.gather_sort(idx, k)
    x = gen.torch_x(104, (tokens, 1, D), dev, dtype=torch.float32)
    h = ops.gather_qmm_swiglu(x, gate, up, idx_dev(tok, dev), idx_dev(srt, dev), 64, 4)
    assert h.dtype == torch.float32 and tuple(h.shape) == (tokens * k, 1, I)
    xs = x.cpu().numpy().reshape(tokens, D)
    hw = lambda t: (t[0].cpu().numpy().view(np.uint32), t[1].cpu().numpy(), t[2].cpu().numpy())
    (gw, gs, gb), (uw, us, ub) = hw(gate), hw(up)
    got = h.cpu().numpy().reshape(-1, I).astype(np.float64)
    for r in (0, 5, 17, tokens * k - 1):
        e, t = int(srt[r]), int(tok[r])
        gg = O.qmm_f64(xs[t:t + 1], O.F32, gw[e], gs[e], gb[e], O.F32, 64, 4)
        uu = O.qmm_f64(xs[t:t + 1], O.F32, uw[e], us[e], ub[e], O.F32, 64, 4)
        ref = gg / (1 + np.exp(-gg)) * uu
        assert rel_err(got[r:r + 1], ref) <= 1e-3, r


@pytest.mark.parametrize("K", [512, 768, 1024, 2048])
@pytest.mark.parametrize("dt,g", [(O.BF16, 64), (O.F16, 64), (O.BF16, 128), (O.F16, 128)])
def test_grouped_kernel_skewed_routing(dev, dt, g, K):
    """4-bit sorted gather at groups 64 and 128 with skewed expert loads --
    one expert with 150 rows (several row tiles over its weights), experts
    with none, a 1-row expert, an out-of-range tail -- with x gathered
    through lhs_indices, against the oracle on every row; and the fused
    gate/up SwiGLU form over the same routing."""
    from helpers import TORCH_DT, quant, to_dev, words_dev, x_of

    Ex, N = 6, 192
    counts = [0, 150, 1, 0, 37, 19]
    rhs = np.concatenate([np.full(c, e, np.uint32) for e, c in enumerate(counts)] +
                         [np.array([Ex, Ex + 3], np.uint32)])
    rows = len(rhs)
    x = x_of(110 + g, (64, 1, K), dt)
    lhs = np.random.default_rng(g).integers(0, 64, rows).astype(np.uint32)
    lhs[5] = 999                                  # out-of-range x index -> NaN row
    w, s, b = quant(111, Ex * N, K, 4, g, dt)
    w, s, b = w.reshape(Ex, N, -1), s.reshape(Ex, N, -1), b.reshape(Ex, N, -1)
    X = to_dev(x, dt, dev)
    W, S, B = words_dev(w, dev), to_dev(s, dt, dev), to_dev(b, dt, dev)
    y = ops.gather_qmm(X, W, S, B, idx_dev(lhs, dev), idx_dev(rhs, dev), True, g, 4, True)
    got = y.float().cpu().numpy().reshape(rows, N).astype(np.float64)
    ref = O.gather_qmm_f64(x, dt, w, s, b, dt, lhs, rhs, 1, N, K, g, 4, x_batch=64)
    ref = ref.reshape(rows, N)
    nan_rows = np.isnan(ref).any(axis=1)
    assert nan_rows.sum() == 3 and np.array_equal(np.isnan(got).all(axis=1), nan_rows)
    assert rel_err(got[~nan_rows], ref[~nan_rows]) <= 1e-2
    # fused gate/up + SwiGLU over the same routing (the up weights: another seed)
    wu, su, bu = quant(112, Ex * N, K, 4, g, dt)
    wu, su, bu = wu.reshape(Ex, N, -1), su.reshape(Ex, N, -1), bu.reshape(Ex, N, -1)
    h = ops.gather_qmm_swiglu(X, (W, S, B), (words_dev(wu, dev), to_dev(su, dt, dev),
                                              to_dev(bu, dt, dev)),
                              idx_dev(lhs, dev), idx_dev(rhs, dev), g, 4)
    gh = h.float().cpu().numpy().reshape(rows, N).astype(np.float64)
    ru = O.gather_qmm_f64(x, dt, wu, su, bu, dt, lhs, rhs, 1, N, K, g, 4, x_batch=64)
    ru = ru.reshape(rows, N)
    rg = O.to_f32(O.from_f32(ref.astype(np.float32), dt), dt).astype(np.float64)
    ru = O.to_f32(O.from_f32(ru.astype(np.float32), dt), dt).astype(np.float64)
    sw = rg / (1 + np.exp(-rg)) * ru
    assert np.array_equal(np.isnan(gh).all(axis=1), nan_rows)
    assert rel_err(gh[~nan_rows], sw[~nan_rows]) <= 1e-2
