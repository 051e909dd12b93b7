"""Benchmark of the MI355X ggml backend on OpenASR's quantized decoder path.

Default workload: the Qwen3-0.6B-shaped decoder's per-token MUL_MAT set on
Q4_K weights at batch 8 (QKV 4096x1024, o 1024x2048, gate/up 3072x1024,
down 1024x3072 for 28 layers, plus the 151936x1024 lm_head) -- one "step" is
one pass of every weight matrix of one decode step, inputs resident in HBM.
Timing: HIP events on the backend's own stream (the plugin's profile hook),
with the timed region bracketed by device synchronisation.

Prints one JSON line (see the keys below). `--gpus N` with N > 1 exits: this
build targets one GPU per process and the path has no collectives.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
Q4K_BPW = 144 / 256
Q8_0_BPW = 34 / 32

# Qwen3-0.6B shape: (name, M, K) per layer, 28 layers, + lm_head
QWEN06_LAYER = [("qkv", 4096, 1024), ("o", 1024, 2048), ("gate", 3072, 1024), ("up", 3072, 1024),
                ("down", 1024, 3072)]
QWEN06_HEAD = ("lm_head", 151936, 1024)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--wtype", choices=["q4_K", "q8_0"], default="q4_K")
    p.add_argument("--batch", type=int, default=8)
    p.add_argument("--layers", type=int, default=28)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    return p.parse_args()


def main() -> int:
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU per process (asked for {a.gpus}); "
              "the decoder path has no multi-GPU collectives", file=sys.stderr)
        return 2
    from openasr_amd import ggml

    g = ggml
    wt = g.Q4_K if a.wtype == "q4_K" else g.Q8_0
    bpw = Q4K_BPW if wt == g.Q4_K else Q8_0_BPW
    plugin = g.plugin()
    log(f"[bench] backend {plugin.name}, workload qwen3-0.6b {a.wtype} mul_mat set, batch {a.batch}")

    shapes = []
    for layer in range(a.layers):
        for name, m, k in QWEN06_LAYER:
            shapes.append((f"L{layer}.{name}", m, k))
    shapes.append(QWEN06_HEAD)

    # one quantized matrix per distinct shape; each layer gets its own copy so
    # the step streams ~335 MB (Q4_K) of distinct weights, beyond the 256 MB MALL
    G = g.Graph(n_tensors=512, graph_size=1024)
    X = {}
    outs = []
    weights = []
    for name, m, k in shapes:
        if k not in X:
            X[k] = G.new(g.F32, k, a.batch, name=f"x{k}")
        W = G.new(wt, k, m, name=name, weight=True)
        weights.append((W, m, k))
        outs.append(G.lib.ggml_mul_mat(G.ctx, W, X[k]))
    G.build(*outs)
    G.allocate(plugin.buft)
    t0 = time.time()
    cache = {}
    for idx, (W, m, k) in enumerate(weights):
        key = (m, k)
        if key not in cache:
            w = g.synth_normal(1234, m * 131 + k, m * k, 0.0, 0.02).reshape(m, k)
            cache[key] = g.quantize(wt, w)
        G.set(W, cache[key])
    rng = np.random.default_rng(0)
    xs = {}
    for k, t in X.items():
        xs[k] = rng.standard_normal((a.batch, k)).astype(np.float32)
        G.set(t, xs[k])
    log(f"[bench] weights uploaded in {time.time() - t0:.1f}s")

    # correctness spot check of the lm_head output against the oracle (the checker)
    assert G.compute(plugin.backend) == 0

    # timed region: warmup, then K steps, HIP events around every launch group
    plugin.profile(G.gf, max(1, a.warmup))
    prof = plugin.profile(G.gf, a.steps)
    step_ms = sum(ms for _, ms in prof)
    gemv = [(lab, ms) for lab, ms in prof if lab.startswith("mul_mat")]
    total_w_bytes = sum(m * k * bpw for _, m, k in shapes)
    # dominant kernel: per-launch algorithmic bytes over its mean duration
    alg_bytes = [m * k * bpw + 4 * k * a.batch + 4 * m * a.batch for _, m, k in shapes]
    gemv_ms = [ms for _, ms in gemv]
    achieved_gbs = sum(alg_bytes) / (sum(gemv_ms) * 1e-3) / 1e9
    head_ms = gemv_ms[-1]
    head_gbs = alg_bytes[-1] / (head_ms * 1e-3) / 1e9
    log(f"[bench] step {step_ms:.3f} ms over {len(prof)} launch groups; mul_mat {achieved_gbs:.0f} GB/s "
        f"({achieved_gbs / HBM_PEAK_GBS:.1%} of peak); lm_head {head_ms * 1e3:.1f} us = {head_gbs:.0f} GB/s")

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(g, wt, cache, xs, a.batch)

    tokens_per_step = a.batch
    out = {
        "metric": "decode tokens/sec @ batch 8 (mul_mat weight stream of one Qwen3-0.6B decode step)",
        "value": round(tokens_per_step / (step_ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_K x q8_K int8 dot, f32 accumulate" if wt == g.Q4_K else "q8_0 x q8_0 int8 dot, f32 accumulate",
        "data": "synthetic (N(0,0.02) weights quantized, N(0,1) activations)",
        "config": {"workload": f"qwen3-0.6b-shaped {a.wtype} decoder mul_mat set, {a.layers} layers + lm_head",
                   "batch": a.batch, "weight_bytes_per_step": int(total_w_bytes), "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def cpu_baseline(g, wt, cache, xs, batch):
    """The oracle's mul_mat (the checker) on the host cores over a bounded
    sample of the same workload: the five per-layer matrices of one layer,
    repeated until ~10 s, scaled to tokens/s of a full 28-layer step."""
    from oracle import ref

    threads = os.cpu_count() or 1
    layer_bytes = 0
    t_total = 0.0
    reps = 0
    t_start = time.time()
    while time.time() - t_start < 10.0:
        for name, m, k in QWEN06_LAYER:
            wq = cache[(m, k)]
            t0 = time.perf_counter()
            ref.mul_mat(wt, wq, m, k, xs[k], threads=threads)
            t_total += time.perf_counter() - t0
            if reps == 0:
                layer_bytes += wq.nbytes
        reps += 1
    per_layer = t_total / reps
    m, k = QWEN06_HEAD[1], QWEN06_HEAD[2]
    head_bytes = cache[(m, k)].nbytes
    step_s = per_layer * 28 + per_layer * head_bytes / layer_bytes
    return {"value": round(batch / step_s, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle mul_mat over one layer's 5 matrices x{reps}, batch {batch}, scaled to 28 layers "
                      f"+ lm_head by weight bytes"}


if __name__ == "__main__":
    sys.exit(main())
