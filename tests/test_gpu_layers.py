"""The quantized layer types over an MLX-format checkpoint loaded onto the
GPU (higgs_amd.loader + higgs_amd.layers), against the CPU oracle:
QLinear.forward (qwen3_next.rs:255-264), QEmbedding.forward (take ->
dequantize, 308-318, bit-exact), QEmbedding.as_linear (the tied lm_head,
320-333), DenseSwiGLU (dense_hidden_fused, 2539-2585) and SwitchGLU."""
import numpy as np
import pytest
import torch

import oracle as O
from ckpt_util import write_checkpoint
from helpers import idx_dev, rel_err, to_host_bits, to_host_f64
from higgs_amd import gen, layers, loader, ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory, dev):
    d = str(tmp_path_factory.mktemp("mlx_ckpt"))
    written = write_checkpoint(d, seed=21)
    return loader.Checkpoint(d, dev), written


@pytest.mark.parametrize("M", [1, 3, 200])
def test_linear_from_checkpoint_matches_oracle(ckpt, dev, M):
    ck, written = ckpt
    for name in ("model.layers.0.self_attn.q_proj", "model.layers.0.mlp.gate"):
        w, s, b, bits, g = written[name]
        lin = ck.linear(name)
        x = gen.np_x_bf16(M + 3, (M, 256))
        xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev)
        y = lin(xd)
        ref = O.qmm_f64(x, O.BF16, w, s, b, O.BF16, g, bits)
        assert rel_err(to_host_f64(y), ref) <= 1e-2, (name, M)


def test_embedding_forward_is_take_then_dequantize(ckpt, dev):
    ck, written = ckpt
    w, s, b, bits, g = written["model.embed_tokens"]
    emb = ck.embedding("model.embed_tokens")
    ids = np.array([[0, 5, 95], [17, 17, 3]], np.uint32)
    out = emb(idx_dev(ids, dev).reshape(2, 3))
    assert tuple(out.shape) == (2, 3, 256)
    flat = ids.reshape(-1)
    ref = O.dequantize(w[flat], s[flat], b[flat], g, bits, O.BF16)
    np.testing.assert_array_equal(to_host_bits(out).reshape(-1, 256), ref)


@pytest.mark.parametrize("M", [1, 7])
def test_embedding_as_linear_is_the_tied_lm_head(ckpt, dev, M):
    ck, written = ckpt
    w, s, b, bits, g = written["model.embed_tokens"]
    emb = ck.embedding("model.embed_tokens")
    x = gen.np_x_bf16(40 + M, (1, M, 256))
    xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev)
    logits = emb.as_linear(xd)
    assert tuple(logits.shape) == (1, M, w.shape[0])
    ref = O.qmm_f64(x.reshape(M, 256), O.BF16, w, s, b, O.BF16, g, bits)
    assert rel_err(to_host_f64(logits).reshape(M, -1), ref) <= 1e-2
    # the head is the embedding's own table: row t of deq(table) . x = logit t
    one_hot_row = to_host_bits(emb(idx_dev(np.array([11], np.uint32), dev)))[0]
    xr = gen.bf16_bits_to_f32(x.reshape(M, 256)[0]).astype(np.float64)
    tab = gen.bf16_bits_to_f32(one_hot_row).astype(np.float64)
    assert abs(float(logits.float()[0, 0, 11]) - tab @ xr) <= 1e-2 * np.abs(ref[0]).max()


@pytest.mark.parametrize("M", [1, 300])
def test_dense_swiglu_from_checkpoint(ckpt, dev, M):
    ck, written = ckpt
    gate, up = ck.linear("model.layers.0.mlp.gate_proj"), ck.linear("model.layers.0.mlp.up_proj")
    mlp = layers.DenseSwiGLU(gate, up)
    x = gen.np_x_bf16(50 + M, (M, 256))
    xd = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev)
    h = mlp(xd)
    gw, gs, gb, bits, g = written["model.layers.0.mlp.gate_proj"]
    uw, us, ub, _, _ = written["model.layers.0.mlp.up_proj"]
    gr = O.from_f32(O.qmm_f64(x, O.BF16, gw, gs, gb, O.BF16, g, bits).astype(np.float32), O.BF16)
    ur = O.from_f32(O.qmm_f64(x, O.BF16, uw, us, ub, O.BF16, g, bits).astype(np.float32), O.BF16)
    ref = O.to_f32(O.swiglu(gr, ur, O.BF16), O.BF16).astype(np.float64)
    assert rel_err(to_host_f64(h), ref) <= 1e-2


def test_switch_glu_moe_matches_block(dev):
    E, D, I, k, T = 8, 256, 128, 2, 24
    q = [layers.QLinear(*gen.torch_quantized(90 + j, n, kk, 4, 64, dev, lead=(E,)), 64, 4)
         for j, (n, kk) in enumerate(((I, D), (I, D), (D, I)))]
    sw = layers.SwitchGLU(*q)
    idx = idx_dev(gen.topk_routing(91, T, E, k), dev).reshape(1, T, k)
    x = gen.torch_x(92, (1, T, D), dev)
    sc = torch.softmax(gen.torch_x(93, (1, T, k), dev).float(), -1).to(torch.bfloat16)
    out = sw.moe(x, idx, sc)
    per = sw.forward_gather_global_sort(x, idx)                    # [1, T, k, D]
    ref = (per.float() * sc.float()[..., None]).sum(-2)
    assert (out.float() - ref).abs().max().item() <= 1e-2 * ref.abs().max().item()


@pytest.mark.parametrize("M", [1, 200])
def test_linear_with_bias_from_checkpoint(tmp_path, dev, M):
    """A Qwen2-style q_proj with its bias (transformer.rs:180-191) loaded from
    an MLX checkpoint, forward against the oracle."""
    d = str(tmp_path)
    q = "model.layers.0.self_attn.q_proj"
    written = write_checkpoint(d, seed=31, bias_layers=(q,))
    lin = loader.Checkpoint(d, dev).linear(q)
    w, s, b, bits, g = written[q]
    x = gen.np_x_bf16(60 + M, (M, 256))
    y = lin(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev))
    ref = O.qmm_f64(x, O.BF16, w, s, b, O.BF16, g, bits) + \
        gen.bf16_bits_to_f32(written[q + ".bias"]).astype(np.float64)[None, :]
    assert rel_err(to_host_f64(y), ref) <= 1e-2
