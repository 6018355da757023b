#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Headline workload: one Llama-3-8B decode step at
batch B (default 1) = 32 layers x (q, k, v, o, gate, up, down) + lm_head, i.e.
225 4-bit group-64 quantized GEMVs over 4.2 GB of distinct weights resident in
HBM (16x the 256 MB Infinity Cache, so every step streams from HBM). The step
is captured once as a HIP graph and replayed; inputs are already in HBM when
the timed region starts.

Printed JSON line (one, on stdout):
  value         whole-step throughput: algorithmic bytes / step time (GB/s)
  roofline      the decode GEMV kernel (qmvs_kernel: every launch of the step
                is one): algorithmic bytes per launch / mean launch duration,
                the duration taken from HIP events recorded on the replay
                stream around the timed replays; peak = MI355X HBM3E 8 TB/s. `traffic` is the measured
                HBM bytes per launch from the committed rocprofv3 FETCH_SIZE /
                WRITE_SIZE summary (profiles/), or null if absent.
  qmv_shapes    per-projection mean launch time and GB/s (one graph over
                >= 1 GiB of distinct copies of that projection)
  qmv_batch     the decode step at B = 1, 4, 8
  mid_rows      16 / 32 / 64 / 127 rows at the gate/up shape (plain product
                and fused gate/up + SwiGLU), GB/s and fraction of HBM peak
  qmm           configs[2]: M = 2048 prefill GEMMs, TFLOP/s and fraction of
                the 2.5 PFLOP/s dense bf16 MFMA peak
  prefill_chunks  the Llama-3-8B q/o, k/v, gate/up and down products at
                M = 512 and 1024 rows (chunked prefill), TFLOP/s
  moe           configs[4]: sorted gather_qmm (gate, down) at the MoE shapes,
                and the whole expert block on device (sort, fused gate/up +
                SwiGLU, down, unsort + score-weighted combine)
  configs       configs[0] (Llama-3.2-1B up-proj qmv at B=1) and configs[3]
                (Qwen3-1.7B gate/up and down at bits 2/3/8 g64 and 4-bit
                g32/g128, B=1 GB/s and M=512 TFLOP/s)
  dequant       dequantize of whole 4-bit g64 tensors (configs[0] shape and
                the Llama-3-8B gate), GB/s of bytes read + written, and the
                quantized embedding (take + dequantize) of 512 token rows
  decode_fused  the same decode step with the launches fused: q|k|v
                concatenated (one launch), gate/up + SwiGLU in one launch
                (hq_quantized_matmul_swiglu, the reference's
                dense_hidden_fused), o, down, lm_head: 129 launches;
                at --batch rows and at B = 1, 4, 8 ("batches")
  cpu_baseline  the CPU oracle's MLX-style quantized_matmul on every host
                CPU the job may run on (and on 1 thread), on a bounded sample
                of the same workload (layer 0's seven projections at B), with
                the CPU model and counts

Every timed graph cycles through >= 1 GiB of distinct weights (4x the 256 MB
Infinity Cache), so weights stream from HBM in every section.

Other modes (for profiling runs):
  --mode copy   a plain device copy of --copy-mb MB (calibrates rocprofv3
                FETCH_SIZE / WRITE_SIZE against known bytes)
  --mode launch the per-launch floor: a graph of 225 launches of the
                library's smallest kernel
  --only S,...  run only the named extra sections (no headline, no CPU leg)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "4-bit qmv GB/s (% HBM peak) + qmm TFLOPS (% MFMA peak), Llama-3-8B shapes"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
BITS, GROUP = 4, 64
HIDDEN, INTER, VOCAB, LAYERS = 4096, 14336, 128256, 32
LAYER_SHAPES = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qmv_decode_llama3_8b_traffic.txt")


def qmv_bytes(M, N, K, bits=BITS, g=GROUP):
    """Algorithmic HBM bytes of one quantized product: packed W + bf16 scales and
    biases + bf16 x + bf16 y, each touched once."""
    return N * K * bits // 8 + 2 * N * (K // g) * 2 + 2 * M * K + 2 * M * N


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Model:
    """Llama-3-8B quantized projection weights, all resident in HBM."""

    def __init__(self, dev, seed=1234):
        import torch

        from higgs_amd import gen

        self.layers = []
        for l in range(LAYERS):
            ws = {}
            for j, (name, N, K) in enumerate(LAYER_SHAPES):
                ws[name] = gen.torch_quantized(seed + 16 * l + j, N, K, BITS, GROUP, dev)
            self.layers.append(ws)
        self.lm_head = gen.torch_quantized(seed + 9999, VOCAB, HIDDEN, BITS, GROUP, dev)
        torch.cuda.synchronize()

    def calls(self, only=None):
        for ws in self.layers:
            for name, N, K in LAYER_SHAPES:
                if only is None or only == name:
                    yield name, ws[name], N, K
        if only is None or only == "lm_head":
            yield "lm_head", self.lm_head, VOCAB, HIDDEN


class Plan:
    """Pre-bound C ABI calls (no allocation, no Python work per launch beyond
    the call itself) for a list of projections at batch B."""

    def __init__(self, calls, B, dev):
        import torch

        from higgs_amd import _lib, gen

        self.lib = _lib.lib()
        self.xh = gen.torch_x(1, (B, HIDDEN), dev)
        self.xi = gen.torch_x(2, (B, INTER), dev)
        self.ys = {}
        self.plan = []
        self.bytes = 0
        for name, (w, s, b), N, K in calls:
            x = self.xi if K == INTER else self.xh
            if name not in self.ys:
                self.ys[name] = torch.empty((B, N), dtype=torch.bfloat16, device=dev)
            self.plan.append((self.ys[name].data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(),
                              b.data_ptr(), B, N, K))
            self.bytes += qmv_bytes(B, N, K)

    def run(self, stream_ptr):
        f = self.lib.hq_quantized_matmul
        for (y, x, w, s, b, M, N, K) in self.plan:
            rc = f(y, x, w, s, b, M, N, K, 1, GROUP, BITS, 2, 2, stream_ptr)
            if rc:
                from higgs_amd import _lib
                raise _lib.HiggsQmmError(rc, _lib.last_error())


def time_graph(run, steps, warmup, dev):
    """Capture run(stream) once as a HIP graph; time `steps` replays with HIP
    events recorded on the replay stream, synchronized on both sides.
    Returns ms per replay."""
    import torch

    stream = torch.cuda.Stream(dev)
    with torch.cuda.stream(stream):
        for _ in range(2):
            run(stream.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            run(stream.cuda_stream)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(steps):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def read_traffic():
    """HBM bytes per qmv launch measured by rocprofv3 (committed summary)."""
    try:
        txt = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", txt, re.M)
    return float(m.group(1)) if m else None


ROTATE_BYTES = 1 << 30  # distinct weight bytes a timed graph cycles through (4x the MALL)


def rotation(N, K, bits=BITS, g=GROUP, have=0, lead=1):
    """Copies of a [lead, N, K] quantized matrix needed for >= ROTATE_BYTES of
    distinct weights (packed words + scales + biases); `have` copies exist."""
    wb = lead * (N * K * bits // 8 + 2 * N * (K // g) * 2)
    return max(have, -(-ROTATE_BYTES // wb))


def bench_shapes(model, B, dev, steps):
    """Per projection: one graph over >= 1 GiB of distinct copies of that
    projection (the model's 32 layer copies plus extra ones), so the 256 MB
    Infinity Cache cannot serve the weights."""
    import torch

    from higgs_amd import gen

    out = {}
    for name, N, K in LAYER_SHAPES + [("lm_head", VOCAB, HIDDEN)]:
        calls = list(model.calls(only=name))
        for c in range(rotation(N, K, have=len(calls)) - len(calls)):
            calls.append((name, gen.torch_quantized(20000 + 64 * c + len(name), N, K, BITS, GROUP,
                                                    dev), N, K))
        p = Plan(calls, B, dev)
        ms = time_graph(p.run, steps, 2, dev)
        n = len(p.plan)
        out[name] = {"N": N, "K": K, "us_per_launch": round(ms * 1e3 / n, 3),
                     "GB/s": round(p.bytes / (ms * 1e-3) / 1e9, 1), "copies": n,
                     "distinct_MB": round(n * (N * K // 2 + 2 * N * (K // GROUP) * 2) / 1e6)}
        del calls, p
        torch.cuda.empty_cache()
    return out


def bench_qmm(model, dev, steps):
    """M=2048 prefill GEMMs over the 32 layers' gate and down weights."""
    import torch

    from higgs_amd import _lib, gen

    lib = _lib.lib()
    out = {}
    for name, N, K in (("gate_up", INTER, HIDDEN), ("down", HIDDEN, INTER)):
        # all 32 layer copies: 1.06 GB of distinct weights per replay
        ws = [model.layers[l]["gate" if name == "gate_up" else "down"] for l in range(LAYERS)]
        x = gen.torch_x(3, (2048, K), dev)
        y = torch.empty((2048, N), dtype=torch.bfloat16, device=dev)

        def run(stream, ws=ws, x=x, y=y, N=N, K=K):
            for (w, s, b) in ws:
                _lib.check(lib.hq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(),
                                                   s.data_ptr(), b.data_ptr(), 2048, N, K, 1,
                                                   GROUP, BITS, 2, 2, stream))
        ms = time_graph(run, steps, 1, dev) / len(ws)
        tflops = 2.0 * 2048 * N * K / (ms * 1e-3) / 1e12
        out[name] = {"M": 2048, "N": N, "K": K, "us": round(ms * 1e3, 2),
                     "tflops": round(tflops, 1), "frac": round(tflops / BF16_PEAK_TFLOPS, 4)}
    return out


def bench_prefill_chunks(dev, steps):
    """Chunked prefill (higgs prefills in chunks of at most 512 tokens, and a
    batch engine can exceed that): the Llama-3-8B projections at M = 512 and
    1024 rows, each over >= 1 GiB of distinct weight copies; TFLOP/s and the
    fraction of the 2.5 PFLOP/s bf16 peak."""
    import torch

    from higgs_amd import _lib, gen

    lib = _lib.lib()
    out = {}
    for name, N, K in (("q_o", HIDDEN, HIDDEN), ("k_v", 1024, HIDDEN), ("gate_up", INTER, HIDDEN),
                       ("down", HIDDEN, INTER)):
        ws = [gen.torch_quantized(700 + c, N, K, BITS, GROUP, dev) for c in range(rotation(N, K))]
        for M in (512, 1024):
            x = gen.torch_x(701, (M, K), dev)
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

            def run(stream, ws=ws, x=x, y=y, M=M, N=N, K=K):
                for (w, s, b) in ws:
                    _lib.check(lib.hq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(),
                                                       s.data_ptr(), b.data_ptr(), M, N, K, 1,
                                                       GROUP, BITS, 2, 2, stream))
            ms = time_graph(run, steps, 1, dev) / len(ws)
            tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
            out[f"{name}_M{M}"] = {"M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
                                   "tflops": round(tflops, 1),
                                   "frac": round(tflops / BF16_PEAK_TFLOPS, 4)}
        del ws
        torch.cuda.empty_cache()
    return out


class FusedPlan:
    """The decode step with fused launches: per layer q|k|v concatenated
    along N, o, gate/up with the SwiGLU epilogue, down; then lm_head.
    Weights are concatenated copies of the Model's (same bytes). Buffers
    hold B rows; use(b) sets the calls and bytes of a step of b <= B rows."""

    def __init__(self, model, B, dev):
        import torch

        from higgs_amd import _lib, gen

        self.lib = _lib.lib()
        self.x = gen.torch_x(1, (B, HIDDEN), dev)
        self.h = gen.torch_x(2, (B, INTER), dev)
        self.yq = torch.empty((B, 6144), dtype=torch.bfloat16, device=dev)
        self.yo = torch.empty((B, HIDDEN), dtype=torch.bfloat16, device=dev)
        self.yh = torch.empty((B, INTER), dtype=torch.bfloat16, device=dev)
        self.yl = torch.empty((B, VOCAB), dtype=torch.bfloat16, device=dev)
        self.keep = []
        self.plan = []
        for ws in model.layers:
            qkv = [torch.cat([ws[n][i] for n in ("q", "k", "v")]) for i in range(3)]
            gu = [torch.cat([ws[n][i] for n in ("gate", "up")]) for i in range(3)]
            self.keep += [qkv, gu]
            self.plan.append(("mm", self.yq, self.x, qkv, 6144, HIDDEN))
            self.plan.append(("mm", self.yo, self.x, ws["o"], HIDDEN, HIDDEN))
            self.plan.append(("swiglu", self.yh, self.x, gu, INTER, HIDDEN))
            self.plan.append(("mm", self.yo, self.h, ws["down"], HIDDEN, INTER))
        self.plan.append(("mm", self.yl, self.x, model.lm_head, VOCAB, HIDDEN))
        self.Bmax = B
        self.use(B)
        torch.cuda.synchronize()

    def use(self, B):
        assert 1 <= B <= self.Bmax
        layers = (len(self.plan) - 1) // 4
        self.bytes = layers * (qmv_bytes(B, 6144, HIDDEN) + qmv_bytes(B, HIDDEN, HIDDEN) +
                               qmv_bytes(B, 2 * INTER, HIDDEN) - 2 * B * INTER +
                               qmv_bytes(B, HIDDEN, INTER)) + qmv_bytes(B, VOCAB, HIDDEN)
        self.B = B
        rows = lambda t, n: t.data_ptr() + n * t.stride(0) * t.element_size()
        self.calls = []
        for kind, y, x, (w, s, b), N, K in self.plan:
            if kind == "mm":
                self.calls.append((0, (y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(),
                                       b.data_ptr(), B, N, K, 1, GROUP, BITS, 2, 2)))
            else:
                self.calls.append((1, (y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(),
                                       b.data_ptr(), rows(w, N), rows(s, N), rows(b, N), B, N, K,
                                       GROUP, BITS, 2, 2)))

    def run(self, stream_ptr):
        fm, fs = self.lib.hq_quantized_matmul, self.lib.hq_quantized_matmul_swiglu
        for kind, a in self.calls:
            rc = (fm if kind == 0 else fs)(*a, stream_ptr)
            if rc:
                from higgs_amd import _lib
                raise _lib.HiggsQmmError(rc, _lib.last_error())


def bench_moe(dev, steps):
    """512 tokens, top-8 of 128 experts, hidden 2048, expert
    intermediate 768, 4-bit g64; rows globally sorted by expert, sorted gather_qmm."""
    import numpy as np
    import torch

    from higgs_amd import gen, ops

    T, TK, E, H, I = 512, 8, 128, 2048, 768
    idx = gen.topk_routing(3, T, E, TK).reshape(-1)
    order = np.argsort(idx, kind="stable")
    srt = torch.from_numpy(idx[order].astype(np.int32)).to(dev)
    tok = torch.from_numpy((order // TK).astype(np.int64)).to(dev)
    used = len(np.unique(idx))
    out = {}
    for name, N, K in (("gate", I, H), ("down", H, I)):
        # >= 1 GiB of distinct expert weights per replay (10 copies of 113 MB)
        ws = [gen.torch_quantized(70 + c, N, K, BITS, GROUP, dev, lead=(E,))
              for c in range(rotation(N, K, lead=E))]
        xs = gen.torch_x(71, (T, K), dev)[tok].reshape(-1, 1, K).contiguous()

        def run(stream, ws=ws, xs=xs):
            for (w, s, b) in ws:
                ops.gather_qmm(xs, w, s, b, None, srt, True, GROUP, BITS, True)
        ms = time_graph(run, steps, 1, dev) / len(ws)
        byts = used * (N * K // 2 + 2 * N * (K // GROUP) * 2) + 2 * T * TK * (K + N)
        gbs = byts / (ms * 1e-3) / 1e9
        # HBM-bound at configs[4] (arithmetic intensity ~94 FLOP/B < ridge
        # ~312): achieved = ideal time (bytes / 8 TB/s) / measured time
        out[name] = {"rows": T * TK, "experts": E, "N": N, "K": K, "us": round(ms * 1e3, 2),
                     "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        del ws
    # the whole expert block (qwen3_moe.rs:353-357 around forward_gather_global_sort)
    # 4 copies of the block's gate, up and down experts: 1.36 GB distinct
    blocks = [tuple(gen.torch_quantized(80 + 3 * c + j, *nk, BITS, GROUP, dev, lead=(E,))
                    for j, nk in enumerate(((I, H), (I, H), (H, I)))) for c in range(4)]
    x = gen.torch_x(72, (1, T, H), dev)
    idx_d = torch.from_numpy(idx.astype(np.int32)).to(dev).reshape(1, T, TK)
    sc = torch.softmax(gen.torch_x(73, (1, T, TK), dev).float(), -1).to(torch.bfloat16)

    def run_block(stream, blocks=blocks):
        for (g, u, d) in blocks:
            ops.moe_block(x, idx_d, sc, g, u, d, GROUP, BITS)
    ms = time_graph(run_block, steps, 1, dev) / len(blocks)
    byts = used * (3 * (I * H // 2 + 2 * I * (H // GROUP) * 2)) + 2 * T * H * 2 + \
        T * TK * 2 * (H + I + I + H)
    out["block"] = {"tokens": T, "top_k": TK, "experts": E, "hidden": H, "intermediate": I,
                    "launches": 4, "us": round(ms * 1e3, 2),
                    "GB/s": round(byts / (ms * 1e-3) / 1e9, 1),
                    "frac": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del blocks
    torch.cuda.empty_cache()
    return out


def bench_configs(dev, steps):
    """per-launch time over distinct weight copies
    (about 2 GB of distinct copies: 8x the 256 MB Infinity Cache)."""
    import torch

    from higgs_amd import _lib, gen

    lib = _lib.lib()
    out = {}

    def one(M, N, K, bits, g, tag):
        wb = N * K * bits // 8 + 2 * N * (K // g) * 2
        copies = max(2, min(256, (1 << 31) // wb + 1))
        ws = [gen.torch_quantized(500 + c, N, K, bits, g, dev,
                                  bias_noise=(1e-3 if tag == "c0" else 0.0)) for c in range(copies)]
        x = gen.torch_x(501, (M, K), dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

        def run(stream, ws=ws):
            for (w, s, b) in ws:
                _lib.check(lib.hq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(),
                                                   s.data_ptr(), b.data_ptr(), M, N, K, 1, g,
                                                   bits, 2, 2, stream))
        ms = time_graph(run, steps, 1, dev) / len(ws)
        r = {"M": M, "N": N, "K": K, "bits": bits, "group_size": g, "us": round(ms * 1e3, 3)}
        if M <= 8:
            r["GB/s"] = round(qmv_bytes(M, N, K, bits, g) / (ms * 1e-3) / 1e9, 1)
        else:
            r["tflops"] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)
        del ws
        return r

    out["c0_llama32_1b_up"] = one(1, 8192, 2048, 4, 64, "c0")
    for bits, g in ((2, 64), (3, 64), (8, 64), (4, 32), (4, 128)):
        for M in (1, 512):
            for name, N, K in (("gate_up", 6144, 2048), ("down", 2048, 6144)):
                out[f"c3_{bits}b_g{g}_M{M}_{name}"] = one(M, N, K, bits, g, "c3")
    torch.cuda.empty_cache()
    return out


def bench_dequant(dev, steps):
    """dequantize (a6): whole tensors at the configs[0] and Llama-3-8B gate
    shapes over distinct copies (more than the 256 MB Infinity Cache), bytes =
    packed W + scales/biases read + bf16 out written; and the quantized
    embedding (take then dequantize) of 512 token rows of a Llama-3-8B
    vocabulary table."""
    import numpy as np
    import torch

    from higgs_amd import _lib, gen

    lib = _lib.lib()
    out = {}

    def whole(tag, N, K, copies):
        ws = [gen.torch_quantized(700 + c, N, K, BITS, GROUP, dev) for c in range(copies)]
        y = torch.empty((N, K), dtype=torch.bfloat16, device=dev)

        def run(stream, ws=ws):
            for (w, s, b) in ws:
                _lib.check(lib.hq_dequantize(y.data_ptr(), w.data_ptr(), s.data_ptr(),
                                             b.data_ptr(), N, K, GROUP, BITS, 2, stream))
        ms = time_graph(run, steps, 1, dev) / len(ws)
        nbytes = N * K * BITS // 8 + 2 * N * (K // GROUP) * 2 + N * K * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[tag] = {"rows": N, "K": K, "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4)}
        del ws

    # >= 1 GiB of distinct packed weights + scales/biases per replay
    whole("c0_8192x2048", 8192, 2048, rotation(8192, 2048))
    whole("gate_14336x4096", 14336, 4096, rotation(14336, 4096))
    # embedding: 32 batches of 512 token ids into a [128256, 4096] table (one
    # graph of 32 launches: a single small launch per replay would time the
    # host's graph launch instead)
    w, s, b = gen.torch_quantized(777, VOCAB, HIDDEN, BITS, GROUP, dev)
    nb = 32
    ids = torch.from_numpy(np.random.default_rng(5).integers(0, VOCAB, (nb, 512))
                           .astype(np.uint32).view(np.int32)).to(dev)
    e = torch.empty((512, HIDDEN), dtype=torch.bfloat16, device=dev)

    def run_e(stream):
        for i in range(nb):
            _lib.check(lib.hq_embedding_dequantize(e.data_ptr(), w.data_ptr(), s.data_ptr(),
                                                   b.data_ptr(), ids[i].data_ptr(), 512, VOCAB,
                                                   HIDDEN, GROUP, BITS, 2, stream))
    ms = time_graph(run_e, steps, 1, dev) / nb
    nbytes = 512 * (HIDDEN * BITS // 8 + 2 * (HIDDEN // GROUP) * 2 + 4 + HIDDEN * 2)
    out["embedding_512_of_128256x4096"] = {"tokens": 512, "us": round(ms * 1e3, 3),
                                           "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    del w, s, b
    torch.cuda.empty_cache()
    return out


def host_cpus():
    """(threads to use, description) for the CPU baseline: every CPU this process
    may run on -- its affinity mask, capped by a cgroup CPU quota when one is
    set -- plus the host's CPU model and counts."""
    import re as _re

    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    quota = None
    for path in ("/sys/fs/cgroup/cpu.max", "/sys/fs/cgroup/cpu/cpu.cfs_quota_us"):
        try:
            txt = open(path).read().split()
        except OSError:
            continue
        try:
            if path.endswith("cpu.max") and txt[0] != "max":
                quota = int(txt[0]) / int(txt[1])
            elif not path.endswith("cpu.max") and int(txt[0]) > 0:
                period = int(open("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read())
                quota = int(txt[0]) / period
        except (OSError, ValueError, IndexError):
            quota = None
        break
    threads = affinity if quota is None else max(1, min(affinity, int(quota)))
    try:
        models = _re.findall(r"^model name\s*:\s*(.*)$", open("/proc/cpuinfo").read(), _re.M)
    except OSError:
        models = []
    info = {"cpu_model": models[0].strip() if models else "unknown",
            "nproc": os.cpu_count(), "affinity_cpus": affinity,
            "cgroup_cpu_quota": None if quota is None else round(quota, 2),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}
    return threads, info


def cpu_baseline(model, B, target_s):
    """Oracle quantized_matmul (MLX-CPU-style restatement, oracle/hq_oracle.c
    hqo_qmm_mlx) on the host, over layer 0's seven projections at batch B:
    on every CPU the job may use, and on one thread."""
    import numpy as np
    import torch

    import oracle as O
    from higgs_amd import gen

    sample = []
    nbytes = 0
    for name, N, K in LAYER_SHAPES:
        w, s, b = model.layers[0][name]
        sample.append((w.cpu().numpy().view(np.uint32),
                       s.cpu().view(torch.int16).numpy().view(np.uint16),
                       b.cpu().view(torch.int16).numpy().view(np.uint16),
                       gen.np_x_bf16(5, (B, K)), N, K))
        nbytes += qmv_bytes(B, N, K)

    def one_pass(threads):
        for w, s, b, x, N, K in sample:
            O.qmm_mlx(x, O.BF16, w, s, b, O.BF16, GROUP, BITS, threads=threads)

    res = {}
    threads_all, info = host_cpus()
    for threads in (1, threads_all):
        t0 = time.perf_counter()
        one_pass(threads)
        dt = time.perf_counter() - t0
        reps = max(1, int(target_s / max(dt, 1e-3)) - 1)
        t0 = time.perf_counter()
        for _ in range(reps):
            one_pass(threads)
        dt = (time.perf_counter() - t0) / reps
        res[threads] = (nbytes / dt / 1e9, reps)
    gbs_all, reps_all = res[threads_all]
    out = {"value": round(gbs_all, 3), "unit": "GB/s", "cores": threads_all, "kind": "port",
           "value_1thread": round(res[1][0], 3),
           "sample": f"Llama-3-8B layer 0 q,k,v,o,gate,up,down at B={B} "
                     f"({nbytes / 1e6:.1f} MB algorithmic), {reps_all} passes on "
                     f"{threads_all} threads (every CPU the job may use) and {res[1][1]} on "
                     f"1 thread, oracle hqo_qmm_mlx (float lanes, MLX CPU loop order)"}
    out.update(info)
    return out


def mode_copy(dev, mb, steps):
    import torch

    n = mb * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        b.copy_(a)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"mode": "copy", "bytes_read": 4 * n, "bytes_written": 4 * n,
                      "ms": round(dt * 1e3, 4), "GB/s": round(8 * n / dt / 1e9, 1)}), flush=True)


def bench_batch(model, args, step, dev):
    qb = {}
    for B in (1, 4, 8):
        st = step if (step is not None and B == args.batch) else Plan(model.calls(), B, dev)
        m = time_graph(st.run, max(5, args.steps // 2), 2, dev)
        qb[str(B)] = {"ms_per_step": round(m, 4), "GB/s": round(st.bytes / (m * 1e-3) / 1e9, 1),
                      "frac": round(st.bytes / (m * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return qb


def bench_mid_rows(model, dev, steps):
    """16 to 127 rows of x (a batch engine with that many active requests, or
    a short prefill chunk) at the Llama-3-8B gate/up shape: the plain product
    and the fused gate/up + SwiGLU, over the 32 layers' weights (>= 1 GiB of
    distinct gate + up weights per replay). Bytes are the algorithmic minimum
    (weights once); the fraction is of the 8 TB/s HBM peak."""
    import torch

    from higgs_amd import _lib, gen

    lib = _lib.lib()
    out = {}
    N, K = INTER, HIDDEN
    gates = [model.layers[l]["gate"] for l in range(LAYERS)]
    ups = [model.layers[l]["up"] for l in range(LAYERS)]
    for M in (16, 32, 64, 127):
        x = gen.torch_x(7, (M, K), dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

        def run(stream, x=x, y=y, M=M):
            for (w, s, b) in gates + ups:
                _lib.check(lib.hq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(),
                                                   s.data_ptr(), b.data_ptr(), M, N, K, 1,
                                                   GROUP, BITS, 2, 2, stream))

        def run_swi(stream, x=x, y=y, M=M):
            for (g, u) in zip(gates, ups):
                _lib.check(lib.hq_quantized_matmul_swiglu(
                    y.data_ptr(), x.data_ptr(), g[0].data_ptr(), g[1].data_ptr(),
                    g[2].data_ptr(), u[0].data_ptr(), u[1].data_ptr(), u[2].data_ptr(), M, N,
                    K, GROUP, BITS, 2, 2, stream))
        ms = time_graph(run, steps, 1, dev) / (2 * LAYERS)
        ms2 = time_graph(run_swi, steps, 1, dev) / LAYERS
        one = qmv_bytes(M, N, K)
        swi = 2 * qmv_bytes(M, N, K) - 2 * M * N
        out[str(M)] = {"us": round(ms * 1e3, 2), "GB/s": round(one / (ms * 1e-3) / 1e9, 1),
                       "frac": round(one / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                       "swiglu_us": round(ms2 * 1e3, 2),
                       "swiglu_frac": round(swi / (ms2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def bench_fused(model, args, dev):
    import torch

    fp = FusedPlan(model, max(8, args.batch), dev)
    res = {}
    for B in sorted({args.batch, 1, 4, 8}):
        fp.use(B)
        mf = time_graph(fp.run, args.steps if B == args.batch else max(5, args.steps // 2), 2, dev)
        res[B] = {"ms_per_step": round(mf, 4), "GB/s": round(fp.bytes / (mf * 1e-3) / 1e9, 1),
                  "frac": round(fp.bytes / (mf * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "tokens_per_s": round(B * 1e3 / mf, 1)}
    r = {"batch": args.batch, "launches": len(fp.calls), **res[args.batch],
         "batches": {str(B): v for B, v in res.items() if B != args.batch}}
    del fp
    torch.cuda.empty_cache()
    return r


SECTIONS = ("qmv_shapes", "qmv_batch", "mid_rows", "qmm", "prefill_chunks", "moe", "configs",
            "dequant", "decode_fused")


def sections(model, args, step, dev):
    """(name, thunk) of the extra sections, in output order (all, or --only's)."""
    sub = max(3, args.steps // 4)
    table = {
        "qmv_shapes": lambda: bench_shapes(model, args.batch, dev, sub),
        "qmv_batch": lambda: bench_batch(model, args, step, dev),
        "mid_rows": lambda: bench_mid_rows(model, dev, sub),
        "qmm": lambda: bench_qmm(model, dev, sub),
        "prefill_chunks": lambda: bench_prefill_chunks(dev, sub),
        "moe": lambda: bench_moe(dev, sub),
        "configs": lambda: bench_configs(dev, sub),
        "dequant": lambda: bench_dequant(dev, sub),
        "decode_fused": lambda: bench_fused(model, args, dev),
    }
    names = SECTIONS if not args.only else args.only.split(",")
    return [(n, table[n]) for n in names]


def mode_launch(dev, steps, launches=225):
    """Per-launch floor: a graph of `launches` launches of this library's
    smallest kernel (hq_swiglu over 64 elements, one block), timed like the
    decode step. It is the cost every launch of the step pays before any
    weight byte moves."""
    import torch

    from higgs_amd import _lib

    lib = _lib.lib()
    g = torch.zeros(64, dtype=torch.bfloat16, device=dev)
    o = torch.empty_like(g)

    def run(stream):
        for _ in range(launches):
            _lib.check(lib.hq_swiglu(o.data_ptr(), g.data_ptr(), g.data_ptr(), 64, 2, stream))
    ms = time_graph(run, steps, 3, dev)
    print(json.dumps({"mode": "launch", "launches": launches, "ms_per_graph": round(ms, 4),
                      "us_per_launch": round(ms * 1e3 / launches, 3)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=6.0,
                    help="target seconds per CPU thread-count leg")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip shapes, batch, qmm, moe")
    ap.add_argument("--mode", default="decode", choices=("decode", "copy", "launch"))
    ap.add_argument("--copy-mb", type=int, default=512)
    ap.add_argument("--only", default="",
                    help="comma-separated extra sections to run alone, without the headline step "
                         "or the CPU baseline (profiling runs); prints one JSON object of them: "
                         + ", ".join(SECTIONS))
    args = ap.parse_args()
    for n in filter(None, args.only.split(",")):
        if n not in SECTIONS:
            ap.error(f"--only: unknown section {n!r} (choose from {', '.join(SECTIONS)})")
    if args.gpus != 1:
        print(f"bench.py measures one GPU (got --gpus {args.gpus}): this build's path is the "
              "single-GPU quantized-linear kernel set; multi-GPU sharding is design-only",
              file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.mode == "copy":
        mode_copy(dev, args.copy_mb, args.steps)
        return
    if args.mode == "launch":
        mode_launch(dev, args.steps)
        return

    from higgs_amd import _lib

    log(f"[bench] {_lib.version()} on {torch.cuda.get_device_name(0)}")
    if args.only:
        needs_model = {"qmv_shapes", "qmv_batch", "mid_rows", "qmm", "decode_fused"}
        model = Model(dev) if needs_model & set(args.only.split(",")) else None
        out = {}
        for name, fn in sections(model, args, None, dev):
            out[name] = fn()
            log(f"[bench] {name}: {out[name]}")
        print(json.dumps({"only": out}), flush=True)
        return
    model = Model(dev)
    step = Plan(model.calls(), args.batch, dev)
    log(f"[bench] weights resident: {step.bytes / 1e9:.2f} GB algorithmic per step, "
        f"{len(step.plan)} launches")

    ms = time_graph(step.run, args.steps, args.warmup, dev)
    value = step.bytes / (ms * 1e-3) / 1e9
    n_launch = len(step.plan)
    mean_us = ms * 1e3 / n_launch
    log(f"[bench] decode step B={args.batch}: {ms:.4f} ms, {value:.1f} GB/s, "
        f"{mean_us:.3f} us per launch")

    extras = {}
    if not args.no_extras:
        for name, fn in sections(model, args, step, dev):
            extras[name] = fn()
            log(f"[bench] {name}: {extras[name]}")
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(model, args.batch, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu}")

    traffic = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 x bf16",
        "data": "synthetic",
        "config": {"workload": f"Llama-3-8B decode step (configs[1]): 32 layers x (q,k,v,o,"
                               f"gate,up,down) + lm_head at B={args.batch}, 4-bit g64 "
                               f"quantized_matmul, one HIP graph",
                   "bits": BITS, "group_size": GROUP, "batch": args.batch,
                   "algorithmic_GB_per_step": round(step.bytes / 1e9, 4),
                   "launches_per_step": n_launch,
                   "compute": "u4 weights x bf16 activations, fp32 accumulate, bf16 out"},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": round(traffic) if traffic else None,
                     "kernel": "qmvs_kernel (streaming matrix-core decode GEMV), every launch "
                               "of the step",
                     "bytes_per_launch": round(step.bytes / n_launch),
                     "mean_launch_us": round(mean_us, 3)},
        "cpu_baseline": cpu,
    }
    line.update(extras)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
