"""Writes small MLX-format quantized checkpoints for the loader tests, with
the safetensors package (an independent writer of the container format)."""
import json
import os

import numpy as np
import torch
from safetensors.torch import save_file

from higgs_amd import gen

# layer path -> (rows, cols, bits, group_size); the router gate carries a
# per-layer override in config.json, as Qwen3-Next checkpoints do
LAYERS = {
    "model.embed_tokens": (96, 256, 4, 64),
    "model.layers.0.self_attn.q_proj": (128, 256, 4, 64),
    "model.layers.0.mlp.gate_proj": (160, 256, 4, 64),
    "model.layers.0.mlp.up_proj": (160, 256, 4, 64),
    "model.layers.0.mlp.down_proj": (256, 256, 4, 64),
    "model.layers.0.mlp.gate": (16, 256, 8, 64),
}


def write_checkpoint(path: str, seed: int = 5, sharded: bool = True, inner: bool = False,
                     prefix: str = "", bias_layers=()):
    """Returns {layer: (w, s, b, bits, group_size)} of what was written; with
    ``bias_layers`` also {layer + ".bias": bf16 bits [rows]} (a Qwen2-style
    additive linear bias, stored as ``<layer>.bias``). ``prefix`` is put in
    front of every tensor name and of the per-layer override key, as
    multimodal checkpoints nest the language model."""
    os.makedirs(path, exist_ok=True)
    written, tensors = {}, {}
    for i, (name, (rows, cols, bits, g)) in enumerate(LAYERS.items()):
        w, s, b = gen.np_quantized(seed + i, rows, cols, bits, g)
        key = prefix + name + (".inner" if inner else "")
        if name in bias_layers:
            lb = gen.np_x_bf16(seed + 100 + i, (rows,))
            tensors[key + ".bias"] = torch.from_numpy(lb.view(np.int16)).view(torch.bfloat16)
            written[name + ".bias"] = lb
        tensors[key + ".weight"] = torch.from_numpy(w.astype(np.uint32)).view(torch.uint32)
        # scales / biases as bfloat16 (MLX stores them as float16 or bfloat16)
        tensors[key + ".scales"] = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
        tensors[key + ".biases"] = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
        written[name] = (w, s, b, bits, g)
    tensors[prefix + "model.norm.weight"] = torch.ones(256, dtype=torch.float32)
    names = sorted(tensors)
    shards = [names[: len(names) // 2], names[len(names) // 2:]] if sharded else [names]
    weight_map = {}
    for j, part in enumerate(shards):
        fname = f"model-{j + 1:05d}-of-{len(shards):05d}.safetensors" if sharded \
            else "model.safetensors"
        save_file({k: tensors[k] for k in part}, os.path.join(path, fname),
                  metadata={"format": "mlx"})
        for k in part:
            weight_map[k] = fname
    if sharded:
        with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": weight_map}, f)
    cfg = {"model_type": "llama",
           "quantization": {"group_size": 64, "bits": 4,
                            prefix + "model.layers.0.mlp.gate": {"group_size": 64, "bits": 8}}}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    return written
