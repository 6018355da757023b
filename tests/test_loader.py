"""MLX-format checkpoint loading (higgs_amd.loader) without a GPU: key remap
(golden cases of crates/higgs-models/src/lib.rs:1057-1100), shard discovery
(lib.rs:965-990), the safetensors container parser against the safetensors
package, per-layer quantization overrides, and shape validation."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file
from safetensors.torch import save_file as save_torch

from ckpt_util import LAYERS, write_checkpoint
from higgs_amd import loader


@pytest.mark.parametrize("key,want", [
    ("model.layers.0.self_attn.q_proj.weight", "model.layers.0.self_attn.q_proj.inner.weight"),
    ("model.layers.0.self_attn.q_proj.bias", "model.layers.0.self_attn.q_proj.inner.bias"),
    ("model.layers.0.self_attn.q_proj.biases", "model.layers.0.self_attn.q_proj.inner.biases"),
    ("model.layers.0.self_attn.q_proj.scales", "model.layers.0.self_attn.q_proj.inner.scales"),
    ("model.embed_tokens.weight", "model.embed_tokens.inner.weight"),
    ("model.norm.weight", "model.norm.inner.weight"),
    ("model.layers.0.self_attn.rotary.inv_freq", None),
])
def test_remap_quantized_key_reference_cases(key, want):
    assert loader.remap_quantized_key(key) == want


def test_collect_files_index_single_and_missing(tmp_path):
    d = str(tmp_path)
    with pytest.raises(loader.CheckpointError, match="No safetensors files found"):
        loader.collect_safetensors_files(d)
    write_checkpoint(d, sharded=True)
    files = loader.collect_safetensors_files(d)
    assert [os.path.basename(f) for f in files] == ["model-00001-of-00002.safetensors",
                                                      "model-00002-of-00002.safetensors"]
    d2 = str(tmp_path / "single")
    write_checkpoint(d2, sharded=False)
    assert [os.path.basename(f) for f in loader.collect_safetensors_files(d2)] == \
        ["model.safetensors"]


def test_parser_matches_safetensors_package(tmp_path):
    rng = np.random.default_rng(0)
    arrs = {"w": rng.integers(0, 2 ** 32, (7, 3), dtype=np.uint32),
            "h": rng.standard_normal((4, 5)).astype(np.float16),
            "f": rng.standard_normal((2, 2, 3)).astype(np.float32),
            "i": np.arange(5, dtype=np.int32), "scalar": np.array(3.0, np.float32)}
    p = str(tmp_path / "a.safetensors")
    save_file(arrs, p, metadata={"format": "mlx"})
    got = {n: (a, t) for n, a, t in loader.iter_safetensors(p)}
    assert set(got) == set(arrs)
    for n, a in arrs.items():
        g, tag = got[n]
        assert g.shape == a.shape
        np.testing.assert_array_equal(g.view(a.dtype) if a.dtype == np.float16 else g, a)
    b = torch.randn(3, 4).to(torch.bfloat16)
    p2 = str(tmp_path / "b.safetensors")
    save_torch({"b": b}, p2)
    (name, arr, tag), = list(loader.iter_safetensors(p2))
    assert tag == "BF16" and np.array_equal(arr, b.view(torch.int16).numpy().view(np.uint16))
    t = loader.to_device(arr, tag, "cpu")
    assert t.dtype == torch.bfloat16 and torch.equal(t, b)


def test_parser_rejects_bad_files(tmp_path):
    p = str(tmp_path / "bad.safetensors")
    with open(p, "wb") as f:
        f.write(b"\x05\x00")
    with pytest.raises(loader.CheckpointError, match="truncated"):
        list(loader.iter_safetensors(p))
    hdr = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 8]}}).encode()
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", len(hdr)) + hdr + b"\x00" * 8)
    with pytest.raises(loader.CheckpointError, match="do not match"):
        list(loader.iter_safetensors(p))
    hdr = json.dumps({"x": {"dtype": "C64", "shape": [1], "data_offsets": [0, 8]}}).encode()
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", len(hdr)) + hdr + b"\x00" * 8)
    with pytest.raises(loader.CheckpointError, match="unsupported dtype"):
        list(loader.iter_safetensors(p))


def test_quantization_overrides():
    cfg = {"quantization": {"group_size": 64, "bits": 4,
                            "model.layers.0.mlp.gate": {"group_size": 64, "bits": 8},
                            "lm_head": False}}
    assert loader.quantization_for(cfg, "model.layers.0.mlp.up_proj") == (64, 4)
    assert loader.quantization_for(cfg, "model.layers.0.mlp.gate") == (64, 8)
    assert loader.quantization_for(cfg, "lm_head") is None
    assert loader.quantization_for({}, "x") is None


@pytest.mark.parametrize("inner", [False, True])
def test_checkpoint_builds_layers_on_cpu(tmp_path, inner):
    d = str(tmp_path)
    written = write_checkpoint(d, inner=inner)
    ck = loader.Checkpoint(d, "cpu")
    for name, (w, s, b, bits, g) in written.items():
        lin = ck.linear(name)
        assert (lin.group_size, lin.bits) == (g, bits)
        np.testing.assert_array_equal(lin.weight.numpy().view(np.uint32), w)
        np.testing.assert_array_equal(lin.scales.view(torch.int16).numpy().view(np.uint16), s)
        assert lin.scales.dtype == torch.bfloat16
    emb = ck.embedding("model.embed_tokens")
    assert emb.weight.shape == (LAYERS["model.embed_tokens"][0], 256 * 4 // 32)
    assert ck.get("model.norm.weight").shape == (256,)
    with pytest.raises(loader.CheckpointError, match="no quantized weight"):
        ck.linear("model.layers.9.mlp.up_proj")


def test_checkpoint_rejects_mismatched_bits(tmp_path):
    d = str(tmp_path)
    write_checkpoint(d)
    cfg = json.load(open(os.path.join(d, "config.json")))
    cfg["quantization"]["model.layers.0.mlp.gate"] = {"group_size": 64, "bits": 4}
    json.dump(cfg, open(os.path.join(d, "config.json"), "w"))
    ck = loader.Checkpoint(d, "cpu")
    with pytest.raises(loader.CheckpointError, match="disagree"):
        ck.linear("model.layers.0.mlp.gate")


@pytest.mark.parametrize("inner", [False, True])
def test_checkpoint_loads_linear_bias(tmp_path, inner):
    """Qwen2-style q/k/v biases (transformer.rs:180-191) load as QLinear.bias
    from <layer>.bias or, after the remap, <layer>.inner.bias (lib.rs:1002-1005);
    layers without one keep bias None."""
    d = str(tmp_path)
    q = "model.layers.0.self_attn.q_proj"
    written = write_checkpoint(d, inner=inner, bias_layers=(q,))
    ck = loader.Checkpoint(d, "cpu")
    lin = ck.linear(q)
    assert lin.bias is not None and lin.bias.dtype == torch.bfloat16
    np.testing.assert_array_equal(lin.bias.view(torch.int16).numpy().view(np.uint16),
                                  written[q + ".bias"])
    assert ck.linear("model.layers.0.mlp.up_proj").bias is None


def test_checkpoint_rejects_bias_of_wrong_length(tmp_path):
    d = str(tmp_path)
    q = "model.layers.0.self_attn.q_proj"
    write_checkpoint(d, bias_layers=(q,))
    ck = loader.Checkpoint(d, "cpu")
    ck.tensors[q + ".bias"] = ck.tensors[q + ".bias"][:5]
    with pytest.raises(loader.CheckpointError, match="is not"):
        ck.linear(q)


def test_prefixed_checkpoint_reads_override_under_the_full_key(tmp_path):
    """With a prefix (a multimodal checkpoint's language model), the per-layer
    override is keyed by the full tensor path (qwen3_next.rs:3431-3437 reads
    'language_model.model.layers.0.mlp.gate'): the 8-bit router gate must get
    its 8 bits, not the 4-bit default."""
    d = str(tmp_path)
    pre = "language_model."
    written = write_checkpoint(d, prefix=pre)
    ck = loader.Checkpoint(d, "cpu", prefix=pre)
    gate = ck.linear("model.layers.0.mlp.gate")
    assert (gate.group_size, gate.bits) == (64, 8)
    np.testing.assert_array_equal(gate.weight.numpy().view(np.uint32),
                                  written["model.layers.0.mlp.gate"][0])
    assert ck.linear("model.layers.0.mlp.up_proj").bits == 4
