"""Quantized layer types of the path, over the ops facade.

* ``QLinear`` -- crates/higgs-models/src/qwen3_next.rs:232-280 (raw weight /
  scales / biases + group_size / bits; ``forward`` = quantized_matmul with
  transpose=true, quantized_forward at 218-227; ``forward_decode_fast`` is
  the same kernel here, the decode GEMV is the default path), plus the
  optional bias of mlx-rs QuantizedLinear (transformer.rs:148-157, 180-191).
* ``QEmbedding`` -- qwen3_next.rs:284-333: ``forward`` = take rows then
  dequantize (fused: only the selected rows are read); ``as_linear`` = the
  tied lm_head, quantized_matmul against the embedding table
  (transformer.rs:842-848 for mlx-rs' QuantizedEmbedding::as_linear).
* ``DenseSwiGLU`` -- FfnBlock::dense_hidden_fused (qwen3_next.rs:2539-2585):
  gate and up concatenated once, one fused launch per call.
* ``SwitchGLU`` -- SwitchMlpWeights (qwen3_next.rs:1660-1809) with stacked
  [experts, N, P] weights: ``forward_gather`` (unsorted),
  ``forward_gather_global_sort`` and the score-weighted ``moe`` of
  qwen3_moe.rs:353-357; each projection keeps its own group size and bits.
"""
from __future__ import annotations

import torch

from . import ops


class QLinear:
    """``bias`` (optional, [out_features]) is the layer's additive bias, as on
    mlx-rs QuantizedLinear for Qwen2-style q/k/v projections
    (transformer.rs:180-191); it is added in the kernel's epilogue."""

    def __init__(self, weight, scales, biases, group_size: int = 64, bits: int = 4, bias=None):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits = group_size, bits
        self.bias = bias

    @classmethod
    def from_float(cls, weight: torch.Tensor, group_size: int = 64, bits: int = 4, bias=None):
        """Quantize a float [out, in] weight on the GPU (mlx_rs::nn::quantize of
        an nn::Linear, transformer.rs:954-965)."""
        wq, s, b = ops.quantize(weight, group_size, bits)
        return cls(wq, s, b, group_size, bits, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.bias is not None:
            return ops.quantized_linear(x, self.weight, self.scales, self.biases, self.bias,
                                        self.group_size, self.bits)
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                    self.group_size, self.bits)

    __call__ = forward
    forward_decode_fast = forward

    @property
    def out_features(self) -> int:
        return self.weight.shape[-2]

    @property
    def in_features(self) -> int:
        return self.weight.shape[-1] * 32 // self.bits


class QEmbedding:
    def __init__(self, weight, scales, biases, group_size: int = 64, bits: int = 4):
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits = group_size, bits

    def forward(self, indices: torch.Tensor) -> torch.Tensor:
        return ops.embedding(indices, self.weight, self.scales, self.biases, self.group_size,
                             self.bits)

    __call__ = forward

    def as_linear(self, x: torch.Tensor) -> torch.Tensor:
        """Logits against the tied embedding table: x @ deq(table).T."""
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                    self.group_size, self.bits)


class DenseSwiGLU:
    """gate/up projection pair with SwiGLU, concatenated once at construction
    (the reference caches the concatenation on first use)."""

    def __init__(self, gate: QLinear, up: QLinear):
        if (gate.group_size, gate.bits) != (up.group_size, up.bits) or \
                gate.weight.shape != up.weight.shape:
            raise ValueError("gate_proj and up_proj must share shape, group_size and bits")
        self.intermediate = gate.out_features
        self.group_size, self.bits = gate.group_size, gate.bits
        self.weight = torch.cat([gate.weight, up.weight], 0).contiguous()
        self.scales = torch.cat([gate.scales, up.scales], 0).contiguous()
        self.biases = torch.cat([gate.biases, up.biases], 0).contiguous()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.dense_hidden_fused(x, self.weight, self.scales, self.biases,
                                      self.intermediate, self.group_size, self.bits)

    __call__ = forward


class SwitchGLU:
    """Experts with stacked weights: gate_proj / up_proj [E, I, P],
    down_proj [E, D, P']."""

    def __init__(self, gate: QLinear, up: QLinear, down: QLinear):
        self.gate, self.up, self.down = gate, up, down
        self.num_experts = gate.weight.shape[0]

    def _t(self, l: QLinear):
        # each projection carries its own quantization settings
        return (l.weight, l.scales, l.biases, l.group_size, l.bits)

    def forward_gather(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """The unsorted path (qwen3_next.rs:1660-1720): x [B, L, D], indices
        [B, L, top_k] -> [B, L, top_k, D]."""
        return ops.forward_gather(x, indices, self._t(self.gate), self._t(self.up),
                                  self._t(self.down))

    def forward_gather_global_sort(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """x [B, L, D], indices [B, L, top_k] -> [B, L, top_k, D]."""
        return ops.forward_gather_global_sort(x, indices, self._t(self.gate), self._t(self.up),
                                              self._t(self.down))

    def moe(self, x: torch.Tensor, indices: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
        """sum over top_k of scores * expert outputs: [B, L, D]."""
        return ops.moe_block(x, indices, scores, self._t(self.gate), self._t(self.up),
                             self._t(self.down))
