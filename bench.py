#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Workload: one Llama-3-8B decode step at batch B
(default 1) = 32 layers x (q, k, v, o, gate, up, down) + lm_head, i.e. 225
4-bit group-64 quantized GEMVs over 4.2 GB of distinct, HBM-resident weights
(no cache reuse between steps: the working set is 16x the 256 MB MALL). The
step is captured once in a HIP graph and replayed.

Printed JSON line:
  value        whole-step throughput, algorithmic bytes / step time (GB/s)
  roofline     the qmv kernel: algorithmic bytes per launch / mean launch
               duration (HIP events around each launch, on the launch stream)
  qmm          configs[2] prefill GEMMs (M=2048), TFLOP/s and % of bf16 peak
  qmv_batch    the same decode step at B = 1, 4, 8
  cpu_baseline the oracle's MLX-CPU-style quantized_matmul on the host cores,
               on a bounded sample (layer 0's seven projections at B)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "4-bit qmv GB/s (% HBM peak) + qmm TFLOPS (% MFMA peak), Llama-3-8B shapes"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
BITS, GROUP = 4, 64
HIDDEN, INTER, KV, VOCAB, LAYERS = 4096, 14336, 1024, 128256, 32
LAYER_SHAPES = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]


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

    def calls(self):
        for l, ws in enumerate(self.layers):
            for name, N, K in LAYER_SHAPES:
                yield f"L{l}.{name}", name, ws[name], N, K
        yield "lm_head", "lm_head", self.lm_head, VOCAB, HIDDEN


class DecodeStep:
    """Pre-bound C ABI calls for one decode step at batch B (no allocation)."""

    def __init__(self, model, B, dev):
        import torch

        from higgs_amd import _lib, gen

        self.lib = _lib.lib()
        self.B = B
        self.xh = gen.torch_x(1, (B, HIDDEN), dev)
        self.xi = gen.torch_x(2, (B, INTER), dev)
        self.ys = {}
        self.plan = []
        self.bytes = 0
        self.shape_of = []
        for label, name, (w, s, b), N, K in model.calls():
            x = self.xi if K == INTER else self.xh
            if name not in self.ys:
                self.ys[name] = torch.empty((B, N), dtype=torch.bfloat16, device=dev)
            y = self.ys[name]
            self.plan.append((y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(),
                              b.data_ptr(), B, N, K))
            self.bytes += qmv_bytes(B, N, K)
            self.shape_of.append((name, N, K))

    def run(self, stream_ptr, events=None):
        f = self.lib.hq_quantized_matmul
        for i, (y, x, w, s, b, M, N, K) in enumerate(self.plan):
            if events is not None:
                events[i][0].record()
            rc = f(y, x, w, s, b, M, N, K, 1, GROUP, BITS, 2, 2, stream_ptr)
            if events is not None:
                events[i][1].record()
            if rc:
                from higgs_amd import _lib
                raise _lib.HiggsQmmError(rc, _lib.last_error())


def time_graph(step, steps, warmup, dev):
    import torch

    stream = torch.cuda.current_stream(dev)
    for _ in range(2):
        step.run(stream.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            step.run(cap.cuda_stream)
    torch.cuda.synchronize()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, g


def per_launch_durations(step, dev, reps=3):
    """Mean duration (ms) of every launch of the step, timed with HIP events
    recorded on the launch stream around each launch (eager, not graphed)."""
    import torch

    stream = torch.cuda.current_stream(dev)
    n = len(step.plan)
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(n)] for _ in range(reps)]
    for r in range(reps):
        step.run(stream.cuda_stream, evs[r])
    torch.cuda.synchronize()
    return [sum(evs[r][i][0].elapsed_time(evs[r][i][1]) for r in range(reps)) / reps
            for i in range(n)]


def bench_qmm(model, dev, reps=5):
    """M=2048 prefill GEMMs on layer 0's gate and down weights."""
    import torch

    from higgs_amd import _lib, gen

    lib = _lib.lib()
    out = {}
    stream = torch.cuda.current_stream(dev).cuda_stream
    for name, N, K in (("gate_up", INTER, HIDDEN), ("down", HIDDEN, INTER)):
        w, s, b = model.layers[0]["gate" if name == "gate_up" else "down"]
        x = gen.torch_x(3, (2048, K), dev)
        y = torch.empty((2048, N), dtype=torch.bfloat16, device=dev)
        args = (y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), 2048, N, K,
                1, GROUP, BITS, 2, 2, stream)
        for _ in range(2):
            _lib.check(lib.hq_quantized_matmul(*args))
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            lib.hq_quantized_matmul(*args)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        tflops = 2.0 * 2048 * N * K / (ms * 1e-3) / 1e12
        out[name] = {"M": 2048, "N": N, "K": K, "ms": round(ms, 4),
                     "tflops": round(tflops, 2), "frac": round(tflops / BF16_PEAK_TFLOPS, 4)}
    return out


def cpu_baseline(model, B, target_s):
    """Oracle quantized_matmul (MLX-CPU-style restatement, oracle/hq_oracle.c
    hqo_qmm_mlx) on the host, over layer 0's seven projections at batch B."""
    import numpy as np

    import oracle as O
    from higgs_amd import gen

    sample = []
    nbytes = 0
    for name, N, K in LAYER_SHAPES:
        w, s, b = model.layers[0][name]
        import torch
        sample.append((w.cpu().numpy().view(np.uint32),
                       s.cpu().view(torch.int16).numpy().view(np.uint16),
                       b.cpu().view(torch.int16).numpy().view(np.uint16),
                       gen.np_x_bf16(5, (B, K)), N, K))
        nbytes += qmv_bytes(B, N, K)

    def one_pass(threads):
        for w, s, b, x, N, K in sample:
            O.qmm_mlx(x, O.BF16, w, s, b, O.BF16, GROUP, BITS, threads=threads)

    res = {}
    threads_all = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(os.cpu_count() or 1, 16)
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
    return {"value": round(gbs_all, 3), "unit": "GB/s", "cores": threads_all, "kind": "port",
            "value_1thread": round(res[1][0], 3),
            "sample": f"Llama-3-8B layer 0 q,k,v,o,gate,up,down at B={B} "
                      f"({nbytes / 1e6:.1f} MB algorithmic), {reps_all} passes at "
                      f"{threads_all} threads and {res[1][1]} at 1 thread, oracle hqo_qmm_mlx "
                      f"(float lanes, MLX CPU loop order)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=4.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip qmm and batch sweeps")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path", file=sys.stderr)
        sys.exit(2)

    import torch

    from higgs_amd import _lib

    dev = torch.device("cuda:0")
    log(f"[bench] {_lib.version()} on {torch.cuda.get_device_name(0)}")
    model = Model(dev)
    log("[bench] weights resident: %.2f GB" % (sum(
        w.numel() * 4 + s.numel() * 2 + b.numel() * 2
        for ws in model.layers for (w, s, b) in ws.values()) / 1e9))

    step = DecodeStep(model, args.batch, dev)
    ms, _graph = time_graph(step, args.steps, args.warmup, dev)
    value = step.bytes / (ms * 1e-3) / 1e9
    log(f"[bench] decode step B={args.batch}: {ms:.4f} ms, {value:.1f} GB/s")

    durs = per_launch_durations(step, dev)
    tot_bytes = step.bytes
    tot_ms = sum(durs)
    achieved = tot_bytes / (tot_ms * 1e-3) / 1e9
    per_shape = {}
    for (name, N, K), d in zip(step.shape_of, durs):
        e = per_shape.setdefault(name, {"N": N, "K": K, "launches": 0, "ms": 0.0})
        e["launches"] += 1
        e["ms"] += d
    for name, e in per_shape.items():
        e["us_per_launch"] = round(e["ms"] / e["launches"] * 1e3, 3)
        e["GB/s"] = round(qmv_bytes(args.batch, e["N"], e["K"]) / (e["ms"] / e["launches"] * 1e-3)
                          / 1e9, 1)
        del e["ms"]
    log(f"[bench] qmv kernel: {achieved:.1f} GB/s over {len(durs)} launches")

    extras = {}
    if not args.no_extras:
        extras["qmm"] = bench_qmm(model, dev)
        log(f"[bench] qmm: {extras['qmm']}")
        qb = {}
        for B in (1, 4, 8):
            st = step if B == args.batch else DecodeStep(model, B, dev)
            m, _ = time_graph(st, max(5, args.steps // 2), 2, dev)
            qb[str(B)] = {"ms_per_step": round(m, 4), "GB/s": round(st.bytes / (m * 1e-3) / 1e9, 1)}
        extras["qmv_batch"] = qb
        log(f"[bench] qmv batch sweep: {qb}")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(model, args.batch, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu}")

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
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"Llama-3-8B decode step, 32 layers x (q,k,v,o,gate,up,down) + "
                               f"lm_head, B={args.batch}, 4-bit g64 qmv (configs[1])",
                   "bits": BITS, "group_size": GROUP, "batch": args.batch,
                   "weights_GB": round(tot_bytes / 1e9, 3), "launches_per_step": len(step.plan),
                   "compute": "u4 weights x bf16 activations, fp32 accumulate, bf16 out"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"qmv (4-bit g64, bf16, M={args.batch})",
                     "bytes_per_launch": round(tot_bytes / len(durs)),
                     "mean_launch_us": round(tot_ms / len(durs) * 1e3, 3)},
        "qmv_shapes": per_shape,
        "cpu_baseline": cpu,
    }
    line.update(extras)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
