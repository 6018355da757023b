"""Pins the CPU oracle (oracle/hq_oracle.c) before it is trusted as the checker.

The reference ships no golden vectors for this path (its hot-path tests are
relational, MLX-vs-MLX on unkeyed random inputs), so each oracle function is
pinned by something independent of its own code: a library routine (torch's
bf16/fp16 rounding and elementwise ops, numpy float64 matmul and stable
argsort), a closed form or special case, an independent construction (Python
big integers for the bitstream), or the reference's relational invariants
(crates/higgs-models/src/qwen3_next.rs:4344-4398, 4431-4530, 12374-12412).
Each check is chosen so that a plausible slip -- nibble order reversed, a
dropped bias, a wrong group index, transposed operands, an unstable sort --
fails it.
"""
import numpy as np
import pytest
import torch

import oracle as O
from higgs_amd import gen

BITS = (2, 3, 4, 5, 6, 8)
GROUPS = (32, 64, 128)
TORCH16 = {O.BF16: torch.bfloat16, O.F16: torch.float16}


def _special_floats():
    v = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 5.96e-8, 2.98e-8,
         6.1035156e-05, 6.09e-05, 3.0e38, -3.0e38, np.inf, -np.inf, 1.0 + 2 ** -8,
         1.0 + 2 ** -9, 1.0 + 3 * 2 ** -9, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 2 ** -126,
         2 ** -149, 2 ** -25, 2 ** -24, 1.5 * 2 ** -25, 3 * 2 ** -26]
    rng = np.random.default_rng(1)
    r = np.concatenate([rng.standard_normal(20000) * s for s in (1e-6, 1e-3, 1, 1e3, 1e5)])
    # exact halfway points between neighbouring bf16 / fp16 values
    base = rng.standard_normal(4000).astype(np.float32)
    bh = (base.view(np.uint32) & 0xFFFF0000) | 0x8000
    fh = (base.view(np.uint32) & 0xFFFFE000) | 0x1000
    return np.concatenate([np.array(v, np.float32), r.astype(np.float32),
                           bh.view(np.float32), fh.view(np.float32)])


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
def test_rounding_matches_torch(orc, dt):
    v = _special_floats()
    got = orc.from_f32(v, dt)
    ref = torch.from_numpy(v).to(TORCH16[dt]).view(torch.int16).numpy().view(np.uint16)
    finite = np.isfinite(v)
    np.testing.assert_array_equal(got[finite], ref[finite])
    # widening is exact: round trip through the oracle's own to_f32
    back = orc.to_f32(got, dt)
    np.testing.assert_array_equal(back[finite],
                                  torch.from_numpy(ref.view(np.int16)).view(TORCH16[dt])
                                  .float().numpy()[finite])


def test_nan_is_canonical(orc):
    v = np.array([np.nan, -np.nan], np.float32)
    assert list(orc.from_f32(v, O.BF16)) == [0x7FC0, 0x7FC0]
    assert all(x & 0x7FFF == 0x7E00 for x in orc.from_f32(v, O.F16))


# --- packing ----------------------------------------------------------------

def test_unpack_nibble_order_kat(orc):
    # qwen3_next.rs:978-986: (packed >> 4*i) & 0xF is element 8*j + i of word j
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    assert orc.unpack(w, 4).tolist() == [list(range(16))]
    assert orc.unpack(np.array([[0x04030201]], np.uint32), 8).tolist() == [[1, 2, 3, 4]]
    w2 = np.array([[0b11100100 | (0b00011011 << 8)] + [0] * 1], np.uint32)
    assert orc.unpack(w2, 2)[0, :8].tolist() == [0, 1, 2, 3, 3, 2, 1, 0]


@pytest.mark.parametrize("bits", BITS)
def test_pack_matches_bigint_bitstream(orc, bits):
    rng = np.random.default_rng(bits)
    rows, cols = 5, 128
    q = rng.integers(0, 2 ** bits, size=(rows, cols), dtype=np.uint32)
    w = orc.pack(q, bits)
    for r in range(rows):
        acc = 0
        for i, v in enumerate(q[r].tolist()):
            acc |= v << (bits * i)
        raw = acc.to_bytes(cols * bits // 8, "little")
        np.testing.assert_array_equal(w[r], np.frombuffer(raw, "<u4"))
    np.testing.assert_array_equal(orc.unpack(w, bits), q)
    # the product-side packer (higgs_amd.gen) agrees with the oracle
    np.testing.assert_array_equal(gen.pack_bits(q, bits), w)


def test_three_bit_straddles_words(orc):
    q = np.zeros((1, 32), np.uint32)
    q[0, 10] = 0b101  # bits 30,31 of word 0 and bit 0 of word 1
    w = orc.pack(q, 3)
    assert w[0, 0] == (0b01 << 30) and w[0, 1] == 0b1


# --- dequantize -------------------------------------------------------------

def _quant(seed, rows, K, bits, g, dt):
    w, s, b = gen.np_quantized(seed, rows, K, bits, g)
    if dt == O.F32:
        s = gen.bf16_bits_to_f32(s) * np.float32(1.37)
        b = gen.bf16_bits_to_f32(b) * np.float32(0.71)
    elif dt == O.F16:
        s = torch.from_numpy(gen.bf16_bits_to_f32(s)).half().view(torch.int16).numpy().view(np.uint16)
        b = torch.from_numpy(gen.bf16_bits_to_f32(b)).half().view(torch.int16).numpy().view(np.uint16)
    return w, s, b


def _t16(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(TORCH16[dt])


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
def test_dequantize_identity_scales(orc, bits, dt):
    rng = np.random.default_rng(7)
    q = rng.integers(0, 2 ** bits, size=(3, 128), dtype=np.uint32)
    w = orc.pack(q, bits)
    one = orc.from_f32(np.ones((3, 2), np.float32), dt)
    zero = orc.from_f32(np.zeros((3, 2), np.float32), dt)
    out = orc.to_f32(orc.dequantize(w, one, zero, 64, bits, dt), dt)
    np.testing.assert_array_equal(out, q.astype(np.float32))


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("dt", [O.F16, O.BF16])
def test_dequantize_two_rounding_matches_torch_ops(orc, bits, g, dt):
    w, s, b = _quant(100 + bits, 16, 256, bits, g, dt)
    got = orc.dequantize(w, s, b, g, bits, dt)
    q = torch.from_numpy(orc.unpack(w, bits).astype(np.float32)).to(TORCH16[dt])
    st = _t16(s, dt).repeat_interleave(g, dim=1)
    bt = _t16(b, dt).repeat_interleave(g, dim=1)
    ref = (q * st) + bt  # torch rounds the product and the sum to the 16-bit type
    np.testing.assert_array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("bits", (3, 4, 8))
def test_dequantize_f32_no_fma(orc, bits):
    w, s, b = _quant(5, 8, 128, bits, 32, O.F32)
    got = orc.dequantize(w, s, b, 32, bits, O.F32)
    q = orc.unpack(w, bits).astype(np.float32)
    ref = (q * np.repeat(s, 32, axis=1)) + np.repeat(b, 32, axis=1)  # numpy: two roundings
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("dt", [O.F16, O.BF16])
def test_dequantize_fused_single_rounding(orc, dt):
    w, s, b = _quant(11, 16, 256, 4, 64, dt)
    got = orc.dequantize(w, s, b, 64, 4, dt, fused=True)
    q = orc.unpack(w, 4).astype(np.float64)
    s64 = np.repeat(orc.to_f32(s, dt).astype(np.float64), 64, axis=1)
    b64 = np.repeat(orc.to_f32(b, dt).astype(np.float64), 64, axis=1)
    exact = q * s64 + b64
    assert np.array_equal(exact.astype(np.float32).astype(np.float64), exact)  # float holds it
    ref = torch.from_numpy(exact.astype(np.float32)).to(TORCH16[dt])
    np.testing.assert_array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))
    # the two conventions do differ on these inputs, so the switch is meaningful
    assert not np.array_equal(got, orc.dequantize(w, s, b, 64, 4, dt))


# --- quantized matmul -------------------------------------------------------

def _deq64(orc, w, s, b, g, bits, dt):
    q = orc.unpack(w, bits).astype(np.float64)
    sf = np.repeat(orc.to_f32(s, dt).astype(np.float64), g, axis=-1)
    bf = np.repeat(orc.to_f32(b, dt).astype(np.float64), g, axis=-1)
    return sf * q + bf


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_qmm_f64_matches_numpy(orc, bits, dt):
    M, N, K, g = 5, 48, 256, 64
    w, s, b = _quant(21, N, K, bits, g, dt)
    x = gen.np_x_bf16(3, (M, K))
    y = orc.qmm_f64(x, O.BF16, w, s, b, dt, g, bits)
    ref = gen.bf16_bits_to_f32(x).astype(np.float64) @ _deq64(orc, w, s, b, g, bits, dt).T
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("bits", (3, 4))
def test_qmm_f64_no_transpose_matches_numpy(orc, bits):
    M, N, K, g = 3, 128, 40, 32
    w, s, b = _quant(22, K, N, bits, g, O.BF16)  # W stored [K, N], groups along N
    x = gen.np_x_bf16(4, (M, K))
    y = orc.qmm_f64(x, O.BF16, w, s, b, O.BF16, g, bits, transpose=False)
    ref = gen.bf16_bits_to_f32(x).astype(np.float64) @ _deq64(orc, w, s, b, g, bits, O.BF16)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_qmm_one_hot_reads_one_column(orc):
    N, K, g, bits = 32, 128, 64, 4
    w, s, b = _quant(23, N, K, bits, g, O.BF16)
    deq = _deq64(orc, w, s, b, g, bits, O.BF16)
    for k in (0, 7, 8, 63, 64, 127):
        x = np.zeros((1, K), np.float32)
        x[0, k] = 1.0
        y = orc.qmm_f64(x, O.F32, w, s, b, O.BF16, g, bits)
        np.testing.assert_array_equal(y[0], deq[:, k])


def test_qmm_mlx_exact_on_integers_and_close_otherwise(orc):
    N, K, g, bits = 16, 128, 32, 4
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint32)
    w = orc.pack(q, bits)
    one = orc.from_f32(np.ones((N, K // g), np.float32), O.BF16)
    zero = orc.from_f32(np.zeros((N, K // g), np.float32), O.BF16)
    x = orc.from_f32(rng.integers(-1, 2, size=(2, K)).astype(np.float32), O.BF16)
    exact = orc.qmm_f64(x, O.BF16, w, one, zero, O.BF16, g, bits)
    for b_ in (4, 3):  # the float-lane path and the bf16-accumulation path
        wq = orc.pack(q % (2 ** b_), b_)
        ex = orc.qmm_f64(x, O.BF16, wq, one, zero, O.BF16, g, b_)
        got = orc.to_f32(orc.qmm_mlx(x, O.BF16, wq, one, zero, O.BF16, g, b_), O.BF16)
        assert np.abs(ex).max() < 256  # every partial sum is a bf16 integer
        np.testing.assert_array_equal(got, ex.astype(np.float32))
    assert exact.shape == (2, N)
    w, s, b = _quant(24, 64, 1024, 4, 64, O.BF16)
    x = gen.np_x_bf16(5, (4, 1024))
    ref = orc.qmm_f64(x, O.BF16, w, s, b, O.BF16, 64, 4)
    got = orc.to_f32(orc.qmm_mlx(x, O.BF16, w, s, b, O.BF16, 64, 4), O.BF16)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-2


# --- gather_qmm and the global sort ----------------------------------------

def test_gather_matches_per_expert(orc):
    # qwen3_next.rs:4344-4398: gather_qmm(x, W, [e]) == quantized_matmul(x, W[e])
    E, N, K, g, bits = 4, 64, 64, 64, 4
    w, s, b = _quant(30, N, K, bits, g, O.BF16)
    w = np.stack([_quant(30 + e, N, K, bits, g, O.BF16)[0] for e in range(E)])
    s = np.stack([_quant(30 + e, N, K, bits, g, O.BF16)[1] for e in range(E)])
    b = np.stack([_quant(30 + e, N, K, bits, g, O.BF16)[2] for e in range(E)])
    x = gen.np_x_bf16(6, (3, 1, K))
    rhs = np.array([2, 0, 3], np.uint32)
    y = orc.gather_qmm_f64(x, O.BF16, w, s, b, O.BF16, None, rhs, 1, N, K, g, bits)
    for i, e in enumerate(rhs):
        ref = orc.qmm_f64(x[i], O.BF16, w[e], s[e], b[e], O.BF16, g, bits)
        np.testing.assert_array_equal(y[i], ref)
    # null lhs with x batch 3 repeated: batch 6 -> x element i // 2
    rhs6 = np.array([0, 1, 2, 3, 1, 0], np.uint32)
    y6 = orc.gather_qmm_f64(x, O.BF16, w, s, b, O.BF16, None, rhs6, 1, N, K, g, bits)
    lhs6 = np.array([0, 0, 1, 1, 2, 2], np.uint32)
    y6e = orc.gather_qmm_f64(x, O.BF16, w, s, b, O.BF16, lhs6, rhs6, 1, N, K, g, bits)
    np.testing.assert_array_equal(y6, y6e)
    # out-of-range indices give NaN rows, in-range rows are untouched
    bad = orc.gather_qmm_f64(x, O.BF16, w, s, b, O.BF16, np.array([0, 5], np.uint32),
                             np.array([9, 1], np.uint32), 1, N, K, g, bits)
    assert np.isnan(bad).all()
    ok = orc.gather_qmm_f64(x, O.BF16, w, s, b, O.BF16, np.array([1], np.uint32),
                            np.array([1], np.uint32), 1, N, K, g, bits)
    np.testing.assert_array_equal(ok[0], orc.qmm_f64(x[1], O.BF16, w[1], s[1], b[1], O.BF16,
                                                     g, bits))


def test_gather_sort_is_stable_argsort(orc):
    idx = gen.topk_routing(9, 64, 16, 4)
    order, inv, srt, tok = orc.gather_sort(idx, 4)
    flat = idx.reshape(-1)
    np.testing.assert_array_equal(order, np.argsort(flat, kind="stable"))
    np.testing.assert_array_equal(srt, flat[order])
    assert np.all(np.diff(srt.astype(np.int64)) >= 0)
    np.testing.assert_array_equal(inv[order], np.arange(flat.size))
    np.testing.assert_array_equal(tok, order // 4)


def test_topk_routing_rows_are_distinct_experts():
    idx = gen.topk_routing(1, 512, 128, 8)
    assert idx.shape == (512, 8) and idx.max() < 128
    assert all(len(set(r)) == 8 for r in idx.tolist())


def test_swiglu_matches_torch_silu(orc):
    g = gen.np_x_bf16(1, (4096,))
    u = gen.np_x_bf16(2, (4096,))
    got = orc.swiglu(g, u, O.BF16)
    gt = torch.from_numpy(gen.bf16_bits_to_f32(g).astype(np.float64))
    ut = torch.from_numpy(gen.bf16_bits_to_f32(u).astype(np.float64))
    ref64 = (torch.nn.functional.silu(gt) * ut).numpy()
    ref = orc.from_f32(ref64.astype(np.float32), O.BF16)
    # rounding double -> bf16 directly vs via float can differ only at exact ties
    assert (got != ref).sum() <= 2
    zero = orc.swiglu(np.zeros(4, np.uint16), u[:4], O.BF16)
    assert gen.bf16_bits_to_f32(zero).tolist() == [0.0] * 4  # +-0: sign follows u


def test_splitmix64_published_vector():
    # SplitMix64 reference output for seed 1234567 (Vigna's splitmix64.c)
    assert [int(v) for v in gen.splitmix64(1234567, 5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]
    assert [int(v) for v in gen.splitmix64(1234567, 2, offset=3)] == [
        4593380528125082431, 16408922859458223821]


def _combine_case(seed, tokens, k, E, D):
    idx = gen.topk_routing(seed, tokens, E, k)
    order, inv, srt, tok = O.gather_sort(idx, k)
    y = gen.np_x_bf16(seed + 1, (tokens * k, D))
    return idx, order, inv, y


def test_moe_combine_unit_scores_is_the_unsort(orc):
    # top_k = 1 view with unit scores: out[i] = y_sorted[inv[i]] bit for bit, and
    # with y_sorted = rows in sorted order this restores the original order.
    idx, order, inv, y = _combine_case(3, 40, 4, 16, 24)
    n = y.shape[0]
    ones = np.full((n, 1), 0x3F80, np.uint16)              # bf16 1.0
    out = orc.moe_combine(y, O.BF16, inv, ones, O.BF16)
    np.testing.assert_array_equal(out, y[inv])
    # sorted rows of an identity table come back as the row numbers
    rows = orc.from_f32(np.repeat(np.arange(n, dtype=np.float32)[:, None], 2, 1), O.F32)
    srt_rows = rows[order]
    back = orc.moe_combine(srt_rows, O.F32, inv, np.ones((n, 1), np.float32), O.F32)
    np.testing.assert_array_equal(back[:, 0], np.arange(n, dtype=np.float32))


def test_moe_combine_one_hot_scores_pick_a_slot(orc):
    idx, order, inv, y = _combine_case(5, 32, 4, 8, 16)
    tokens, k = 32, 4
    for j in range(k):
        sc = np.zeros((tokens, k), np.float32)
        sc[:, j] = 1.0
        out = orc.moe_combine(y, O.BF16, inv, orc.from_f32(sc, O.BF16), O.BF16)
        np.testing.assert_array_equal(out, y[inv.reshape(tokens, k)[:, j]])


def test_moe_combine_weighted_sum_matches_float64(orc):
    tokens, k, D = 64, 8, 48
    idx, order, inv, y = _combine_case(11, tokens, k, 32, D)
    sc = gen.np_x_bf16(12, (tokens, k))
    out = gen.bf16_bits_to_f32(orc.moe_combine(y, O.BF16, inv, sc, O.BF16)).astype(np.float64)
    yf = gen.bf16_bits_to_f32(y).astype(np.float64)
    sf = gen.bf16_bits_to_f32(sc).astype(np.float64)
    ref = (yf[inv].reshape(tokens, k, D) * sf[:, :, None]).sum(axis=1)
    # products and the sum each round to bf16: within a few bf16 ulps of exact
    assert np.abs(out - ref).max() <= 2 ** -6 * np.abs(yf).max() * np.abs(sf).max() * k


def test_moe_combine_out_of_range_inv_gives_nan(orc):
    y = gen.np_x_bf16(1, (8, 4))
    inv = np.arange(8, dtype=np.uint32)
    inv[5] = 99
    sc = np.full((4, 2), 0x3F80, np.uint16)
    out = gen.bf16_bits_to_f32(orc.moe_combine(y, O.BF16, inv, sc, O.BF16))
    assert np.isnan(out[2]).all() and not np.isnan(np.delete(out, 2, 0)).any()


# --- quantize (mlx-rs ops::quantize, qwen3_next.rs:4305-4307, 12942) --------
# MLX's exact scale selection cannot be checked offline (MLX is absent); the
# oracle's quantize is pinned by what the algorithm's mathematics fixes:
# exact recovery of inputs on a grid whose zero is a code, the negation and
# power-of-two symmetries, the error bound, the code range and constant
# groups. Each fails for a plausible slip (wrong n_bins, wrong edge or sign,
# bias not the edge, a missing clip).

def _qdeq64(wq, s, b, g, bits, dt):
    q = O.unpack(wq, bits).astype(np.float64)
    sf = (s if dt == O.F32 else O.to_f32(s, dt)).astype(np.float64)
    bf = (b if dt == O.F32 else O.to_f32(b, dt)).astype(np.float64)
    return q * np.repeat(sf, g, axis=-1) + np.repeat(bf, g, axis=-1)


def _grid_rows(rng, rows, K, bits, g, zero_point=True):
    """Rows of groups w = s0 * (q - z) with q spanning 0..n_bins in every group,
    s0 a power of two and z an integer zero point (so 0 is a grid value)."""
    nb = (1 << bits) - 1
    q = rng.integers(0, nb + 1, (rows, K))
    q[:, ::g] = 0
    q[:, 1::g] = nb                              # both ends present in every group
    z = rng.integers(0, nb + 1, (rows, K // g))
    s0 = 2.0 ** rng.integers(-9, -2, (rows, K // g))
    if not zero_point:
        z = z + 0.5
    return ((q - np.repeat(z, g, axis=1)) * np.repeat(s0, g, axis=1)).astype(np.float32)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("g", GROUPS)
def test_quantize_recovers_grid_inputs_exactly(orc, bits, g):
    rng = np.random.default_rng(bits * 1000 + g)
    w = _grid_rows(rng, 6, 2 * 128, bits, g)
    for dt in (O.F32, O.BF16, O.F16):
        if dt == O.BF16 and bits == 8:
            continue  # integers up to 255 times a power of two need 8 significant bits
        wd = w if dt == O.F32 else O.from_f32(w, dt)
        assert np.array_equal(O.to_f32(wd, dt) if dt != O.F32 else wd, w)
        wq, s, b = O.quantize(wd, dt, g, bits)
        assert np.array_equal(_qdeq64(wq, s, b, g, bits, dt), w.astype(np.float64)), (bits, g, dt)


@pytest.mark.parametrize("bits", BITS)
def test_quantize_error_bound_and_code_range(orc, bits):
    rng = np.random.default_rng(7 + bits)
    g = 64
    w = (rng.standard_normal((8, 512)) * np.exp(rng.uniform(-6, 3, (8, 1)))).astype(np.float32)
    w[0, :64] += 5.0                              # an all-positive group
    w[1, :64] = -np.abs(w[1, :64]) - 1.0          # an all-negative group
    wq, s, b = O.quantize(w, O.F32, g, bits)
    q = O.unpack(wq, bits)
    assert q.max() <= (1 << bits) - 1
    err = np.abs(_qdeq64(wq, s, b, g, bits, O.F32) - w)
    srep = np.abs(np.repeat(s.astype(np.float64), g, axis=1))
    # every element within one step; elements that need no clip within half a
    # step (+ float32 slack); the edge maps to an exact code
    assert (err <= srep * (1 + 1e-5) + 1e-6 * np.abs(w)).all()
    t = (w.astype(np.float64) - np.repeat(b, g, axis=1)) / np.repeat(s, g, axis=1)
    inside = t <= (1 << bits) - 1 + 0.5 - 1e-3
    assert (err[inside] <= 0.5 * srep[inside] * (1 + 1e-4) + 1e-6 * np.abs(w[inside])).all()
    # a dropped clip or a wrong n_bins pushes far more than a few elements over
    assert (~inside).sum() <= 2 * w.size // g


def test_quantize_negation_and_power_of_two_symmetry(orc):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((16, 256)).astype(np.float32)
    for bits in (3, 4, 8):
        wq, s, b = O.quantize(w, O.F32, 64, bits)
        # negation: same codes, negated scales and biases (no |min| == |max| ties here)
        wq2, s2, b2 = O.quantize(-w, O.F32, 64, bits)
        assert np.array_equal(wq, wq2) and np.array_equal(s2, -s) and np.array_equal(b2, -b)
        # power-of-two scaling is exact in every operation
        wq3, s3, b3 = O.quantize(w * np.float32(8.0), O.F32, 64, bits)
        assert np.array_equal(wq, wq3) and np.array_equal(s3, 8 * s) and np.array_equal(b3, 8 * b)


def test_quantize_picks_the_larger_magnitude_edge(orc):
    """The bias is the min or max of larger magnitude and the scale's sign
    follows: a mostly-negative group keeps a positive scale and its minimum as
    bias; a mostly-positive one a negative scale and its maximum."""
    w = np.zeros((1, 64), np.float32)
    w[0, :] = np.linspace(-3.0, 1.0, 64, dtype=np.float32)
    wq, s, b = O.quantize(w, O.F32, 64, 4)
    assert s[0, 0] > 0 and b[0, 0] == np.float32(-3.0)
    wq, s, b = O.quantize(-w, O.F32, 64, 4)
    assert s[0, 0] < 0 and b[0, 0] == np.float32(3.0)
    assert O.unpack(wq, 4)[0, 0] == 0  # the edge itself is code 0


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
def test_quantize_constant_and_zero_groups(orc, dt):
    vals = np.array([0.0, 1.0, -2.5, 0.0078125, 1000.0, -0.001], np.float32)
    w = np.repeat(vals, 64)[None, :]
    wd = w if dt == O.F32 else O.from_f32(w, dt)
    wq, s, b = O.quantize(wd, dt, 64, 4)
    assert (O.unpack(wq, 4) == 0).all()
    deq = _qdeq64(wq, s, b, 64, 4, dt)
    ref = O.to_f32(wd, dt) if dt != O.F32 else wd
    assert np.array_equal(deq, ref.astype(np.float64))


def test_quantize_bf16_stays_within_its_rounding(orc):
    """bf16 weights: scales and biases round to bf16, so the bound widens by
    the rounding of the stored scale and bias (relative 2^-8 each)."""
    rng = np.random.default_rng(11)
    w = O.from_f32(rng.standard_normal((8, 256)).astype(np.float32), O.BF16)
    wq, s, b = O.quantize(w, O.BF16, 64, 4)
    wf = O.to_f32(w, O.BF16).astype(np.float64)
    err = np.abs(_qdeq64(wq, s, b, 64, 4, O.BF16) - wf)
    sr = np.abs(np.repeat(O.to_f32(s, O.BF16).astype(np.float64), 64, axis=1))
    br = np.abs(np.repeat(O.to_f32(b, O.BF16).astype(np.float64), 64, axis=1))
    assert (err <= sr * (1 + 15 * 2 ** -8) + br * 2 ** -8 + 1e-6).all()


@pytest.mark.parametrize("bits", BITS)
def test_quantize_represents_zero(orc, bits):
    """The larger-magnitude edge is an exact multiple of the scale (scale =
    edge / round(edge / scale)), so a 0 in a group maps to an integer code and
    dequantizes to 0 up to float32 rounding (~n_bins * 2^-23 of a step);
    keeping range / n_bins as the scale would miss 0 by up to half a step."""
    rng = np.random.default_rng(19 + bits)
    w = (rng.standard_normal((32, 256)) + rng.uniform(-2, 2, (32, 1))).astype(np.float32)
    zeros = rng.integers(0, 64, (32, 4)) + np.arange(4) * 64
    for r in range(32):
        w[r, zeros[r]] = 0.0
    wq, s, b = O.quantize(w, O.F32, 64, bits)
    deq = _qdeq64(wq, s, b, 64, bits, O.F32)
    srep = np.abs(np.repeat(s.astype(np.float64), 64, axis=1))
    at0 = w == 0.0
    assert (np.abs(deq[at0]) <= 1e-4 * srep[at0]).all()
