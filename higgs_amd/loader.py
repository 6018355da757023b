"""MLX-format quantized checkpoint loading (safetensors) onto the GPU.

Follows higgs' loader (crates/higgs-models/src/lib.rs:843-1008) and the
on-disk MLX layout (docs/mlx_rs_capabilities.md:38-52):

* ``<layer>.weight`` -- packed uint32 [rows, cols*bits/32] (LSB-first),
  ``<layer>.scales`` / ``<layer>.biases`` -- float16 or bfloat16
  [rows, cols/group_size];
* shards listed by ``model.safetensors.index.json`` (its weight_map values,
  sorted), else a single ``model.safetensors`` (``collect_safetensors_files``,
  lib.rs:965-990);
* ``remap_quantized_key`` (lib.rs:994-1008): flat MLX names retried with
  ``.inner.`` inserted, for mlx-rs' nested MaybeQuantized parameters;
* ``config.json`` ``quantization`` = {group_size, bits} (transformer.rs:57-62),
  with per-layer overrides keyed by the layer path (qwen3_next.rs:3431-3437
  reads one for the MoE router gate, under the full tensor-name path);
* a linear layer's optional additive ``<layer>.bias`` (``.inner.bias`` after
  the remap, lib.rs:1002-1005), present on Qwen2-style q/k/v projections
  (qkv_bias, transformer.rs:180-191).

The safetensors container is parsed here directly (8-byte little-endian
header length, JSON header of {name: {dtype, shape, data_offsets}}, then
the raw little-endian data), memory-mapped, and each tensor copied once to
the device. Loading is host-side I/O: no arithmetic on weights happens here.
"""
from __future__ import annotations

import json
import os
import struct
from typing import Dict, Iterator, List, Optional, Tuple

import numpy as np

# safetensors dtype tag -> (numpy storage dtype, torch dtype name)
_ST_DTYPES = {
    "U32": (np.uint32, "int32"),      # packed quantized words: same bits as int32
    "I32": (np.int32, "int32"),
    "F32": (np.float32, "float32"),
    "F16": (np.uint16, "float16"),
    "BF16": (np.uint16, "bfloat16"),
    "U8": (np.uint8, "uint8"),
    "I64": (np.int64, "int64"),
}


class CheckpointError(RuntimeError):
    """A checkpoint is missing, malformed or inconsistent with its config."""


def collect_safetensors_files(model_path: str) -> List[str]:
    """Shard files of a model directory (lib.rs:965-990)."""
    index = os.path.join(model_path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            weight_map = json.load(f)["weight_map"]
        return sorted({os.path.join(model_path, v) for v in weight_map.values()})
    single = os.path.join(model_path, "model.safetensors")
    if os.path.exists(single):
        return [single]
    raise CheckpointError("No safetensors files found")


def remap_quantized_key(key: str) -> Optional[str]:
    """``x.weight`` -> ``x.inner.weight`` (also .scales, .biases, .bias);
    None for other keys (lib.rs:994-1008)."""
    for suffix in (".weight", ".scales", ".biases", ".bias"):
        if key.endswith(suffix):
            return key[: -len(suffix)] + ".inner" + suffix
    return None


def read_safetensors_header(path: str) -> Tuple[dict, int]:
    """(header dict, byte offset of the data section)."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise CheckpointError(f"{path}: truncated safetensors header")
        (n,) = struct.unpack("<Q", raw)
        if n > (1 << 30):
            raise CheckpointError(f"{path}: implausible header length {n}")
        hdr = f.read(n)
        if len(hdr) != n:
            raise CheckpointError(f"{path}: truncated safetensors header")
    try:
        return json.loads(hdr), 8 + n
    except ValueError as e:
        raise CheckpointError(f"{path}: bad safetensors header: {e}") from None


def iter_safetensors(path: str) -> Iterator[Tuple[str, np.ndarray, str]]:
    """(name, read-only memory-mapped array, safetensors dtype tag) per tensor."""
    header, base = read_safetensors_header(path)
    size = os.path.getsize(path)
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    for name, info in header.items():
        if name == "__metadata__":
            continue
        tag = info["dtype"]
        if tag not in _ST_DTYPES:
            raise CheckpointError(f"{path}: tensor {name} has unsupported dtype {tag}")
        npdt = np.dtype(_ST_DTYPES[tag][0])
        begin, end = info["data_offsets"]
        shape = tuple(int(d) for d in info["shape"])
        count = int(np.prod(shape)) if shape else 1
        if end - begin != count * npdt.itemsize or base + end > size or begin > end:
            raise CheckpointError(f"{path}: tensor {name} data_offsets {begin}..{end} do not "
                                  f"match shape {shape} of {tag}")
        arr = mm[base + begin: base + end].view(npdt).reshape(shape)
        yield name, arr, tag


def to_device(arr: np.ndarray, tag: str, device):
    """Copy one memory-mapped array to the device with its torch dtype."""
    import torch

    storage, tname = _ST_DTYPES[tag]
    a = np.array(arr, copy=True)  # a writable host copy of the mapped bytes
    if tag == "U32":
        t = torch.from_numpy(a.view(np.int32))
    elif tag in ("F16", "BF16"):
        t = torch.from_numpy(a.view(np.int16)).view(getattr(torch, tname))
    else:
        t = torch.from_numpy(a)
    return t.to(device)


def load_config(model_path: str) -> dict:
    p = os.path.join(model_path, "config.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f)


def quantization_for(config: dict, layer: str) -> Optional[Tuple[int, int]]:
    """(group_size, bits) for a layer path: a per-layer entry of the
    ``quantization`` table if present, else its top-level defaults; None if
    the checkpoint is not quantized."""
    q = config.get("quantization") or config.get("quantization_config")
    if not q:
        return None
    over = q.get(layer)
    if isinstance(over, dict) and "bits" in over:
        return int(over.get("group_size", q.get("group_size", 64))), int(over["bits"])
    if over is False:  # an explicit "not quantized" entry
        return None
    if "bits" not in q:
        return None
    return int(q.get("group_size", 64)), int(q["bits"])


class Checkpoint:
    """Every tensor of an MLX-format checkpoint on one device, keyed by name.

    ``linear(path)`` / ``embedding(path)`` / ``switch_linear(path)`` build the
    quantized layer types of ``higgs_amd.layers`` from ``<path>.weight``,
    ``.scales`` and ``.biases`` (or their ``.inner.`` variants), with the
    layer's group size and bits from config.json, checked against the shapes.
    """

    def __init__(self, model_path: str, device, prefix: str = ""):
        self.path = model_path
        self.prefix = prefix
        self.config = load_config(model_path)
        self.tensors: Dict[str, object] = {}
        for f in collect_safetensors_files(model_path):
            for name, arr, tag in iter_safetensors(f):
                if prefix:
                    if not name.startswith(prefix):
                        continue
                    name = name[len(prefix):]
                self.tensors[name] = to_device(arr, tag, device)

    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def get(self, name: str):
        if name in self.tensors:
            return self.tensors[name]
        raise CheckpointError(f"missing tensor {name}")

    def _triple(self, path: str):
        for base in (path, path + ".inner"):
            if base + ".weight" in self.tensors and base + ".scales" in self.tensors:
                if base + ".biases" not in self.tensors:
                    raise CheckpointError(f"{base}.biases missing (MLX affine quantization "
                                          "stores scales and biases)")
                return (self.tensors[base + ".weight"], self.tensors[base + ".scales"],
                        self.tensors[base + ".biases"])
        raise CheckpointError(f"no quantized weight for {path}")

    def _bias(self, path: str, out_features: int):
        """The layer's additive bias (``.bias`` or ``.inner.bias``), or None."""
        for key in (path + ".bias", path + ".inner.bias"):
            if key in self.tensors:
                b = self.tensors[key]
                if tuple(b.shape) != (out_features,):
                    raise CheckpointError(f"{key}: shape {tuple(b.shape)} is not "
                                          f"({out_features},)")
                return b
        return None

    def _params(self, path: str, w, s):
        # per-layer overrides are keyed by the full tensor path (the prefix
        # included); then the bare path; then the top-level defaults
        gb = None
        if self.prefix:
            q = self.config.get("quantization") or self.config.get("quantization_config") or {}
            if (self.prefix + path) in q:
                gb = quantization_for(self.config, self.prefix + path)
        if gb is None:
            gb = quantization_for(self.config, path)
        if gb is None:
            raise CheckpointError(f"{path}: config.json has no quantization for this layer")
        g, bits = gb
        cols = w.shape[-1] * 32 // bits
        if w.shape[-1] * 32 % bits or s.shape[-1] * g != cols or s.shape[:-1] != w.shape[:-1]:
            raise CheckpointError(f"{path}: weight {tuple(w.shape)} and scales "
                                  f"{tuple(s.shape)} disagree with group_size={g}, bits={bits}")
        return g, bits

    def linear(self, path: str):
        from .layers import QLinear

        w, s, b = self._triple(path)
        g, bits = self._params(path, w, s)
        return QLinear(w, s, b, g, bits, bias=self._bias(path, w.shape[-2]))

    def embedding(self, path: str):
        from .layers import QEmbedding

        w, s, b = self._triple(path)
        g, bits = self._params(path, w, s)
        return QEmbedding(w, s, b, g, bits)

    def switch_linear(self, path: str):
        from .layers import QLinear

        w, s, b = self._triple(path)
        if w.dim() != 3:
            raise CheckpointError(f"{path}: SwitchLinear weights are [experts, N, P] "
                                  f"(got {tuple(w.shape)})")
        g, bits = self._params(path, w, s)
        return QLinear(w, s, b, g, bits)
