"""Benchmark of the MI355X ggml backend on OpenASR's quantized decoder step.

Workload (default): the Qwen3-0.6B-shaped decoder with Q4_K weights at
batch 8 -- eight sequences, each with an independent seeded 375-position
N(0,1) audio prefix plus 8 prompt tokens prefilled, then greedy decode with
an f16 KV cache sized for 1024 positions per sequence. One "step" is one
decode step of all eight sequences through the persistent decode graph
(28 layers + batched lm_head + first-max top-1), inputs resident in HBM.
The timed region is K consecutive greedy steps (each step is a synchronous
graph compute, so the region is bracketed by device synchronisation),
centred on the mean position of the workload's 512-token decode (untimed
steps, at least the warmup, decode the tokens before it).

Also reported (same run): the Qwen3-0.6B Q8_0 batch-1 decode rate, the
Qwen3-1.7B Q4_K batch-8 rate after 3000-position prefixes (4096-position KV),
the Whisper-tiny Q8_0 batch-1 rate over 1500 cross frames, per-kernel
times of one decode step from HIP events on the backend's own stream, the
roofline fraction of the dominant kernel (the quantized GEMV), and the CPU
oracle's batched decode rate on the host cores from the same KV state.

Prints one JSON line. `--gpus N` with N > 1 exits: the path runs one GPU per
process and has no collectives.
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


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=128, help="timed decode steps")
    p.add_argument("--warmup", type=int, default=8, help="untimed decode steps before the timed region")
    p.add_argument("--workload", default="qwen3-0.6b-q4_K-b8")
    p.add_argument("--no-b1", action="store_true", help="skip the batch-1 Q8_0 side measurement")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-whisper", action="store_true", help="skip the Whisper-tiny batch-1 side measurement")
    p.add_argument("--no-long", action="store_true", help="skip the Qwen3-1.7B long-context side measurement")
    p.add_argument("--no-encoder", action="store_true", help="skip the Qwen3-ASR audio encoder side measurement")
    p.add_argument("--encoder-only", action="store_true",
                   help="run only the audio encoder side measurement (for kernel traces of it)")
    p.add_argument("--no-full", action="store_true",
                   help="skip the side lines that time each workload's whole greedy decode")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--profile-iters", type=int, default=20)
    p.add_argument("--sweep", action="store_true", help="per-kernel sweep of mul_mat and flash_attn_ext shapes")
    p.add_argument("--sweep-reps", type=int, default=20)
    p.add_argument("--mfma-probe", action="store_true",
                   help="a short fixed program for hardware-counter runs of the wide kernels: mul_mat "
                        "151936x1024 at N=512 (Q4_K, Q8_0) and flash_attn_ext over 8192 positions with 64 queries")
    p.add_argument("--traffic-probe", action="store_true",
                   help="fixed short program for rocprofv3 --pmc runs (copy calibration + two decode steps)")
    return p.parse_args()


def weight_bytes(cfg, wtype) -> dict:
    """algorithmic weight bytes per decode step, per matrix kind"""
    from openasr_amd import ggml as g
    bpw = 144 / 256 if wtype == g.Q4_K else 34 / 32
    d, hd = cfg["d_model"], cfg["head_dim"]
    q_w, kv_w = cfg["n_head"] * hd, cfg["n_kv_head"] * hd
    per_layer = {"qkv": (q_w + 2 * kv_w) * d, "o": d * q_w, "gate": cfg["ffn"] * d, "up": cfg["ffn"] * d,
                 "down": d * cfg["ffn"]}
    out = {k: v * cfg["n_layers"] * bpw for k, v in per_layer.items()}
    out["lm_head"] = cfg["vocab"] * d * bpw
    return out


def workload_text(name: str) -> dict:
    """the metric, dtype, data and model fields of the bench line, from the
    workload's own shape, weight type and batch"""
    from openasr_amd import decoders as D
    from openasr_amd import ggml as g

    wl = D.WORKLOADS[name]
    sh = wl.shape
    size = {1024: "0.6B", 2048: "1.7B"}.get(sh["d_model"], f"d{sh['d_model']}")
    wt = {g.Q4_K: ("Q4_K", "q4_K weights x q8_K activations (int8 dot, f64 block sums)"),
          g.Q8_0: ("Q8_0", "q8_0 weights x q8_0 activations (int8 dot, f64 block sums)")}[wl.wtype]
    return {
        "metric": f"decode tokens/sec @ batch {wl.n_seq} (Qwen3-{size}-shaped {wt[0]} decoder); "
                  "quantized mul_mat HBM GB/s as % of peak",
        "dtype": f"{wt[1]}, f16 KV, f32 activations",
        "data": f"synthetic: random-init N(0,0.02) weights quantized to {wt[0]}, seeded N(0,1) "
                f"{wl.prefix}-position prefixes",
        "model": f"qwen3-{size.lower()}-shaped (hidden {sh['d_model']}, {sh['n_layers']} layers, "
                 f"{sh['n_head']}/{sh['n_kv_head']} heads, head_dim {sh['head_dim']}, ffn {sh['ffn']}, "
                 f"vocab {sh['vocab']})",
        "batch": wl.n_seq,
        "seq_len": wl.max_positions,
        "kernel": "k_gemv_q4_K" if wl.wtype == g.Q4_K else ("k_gemv1_q8_0" if wl.n_seq == 1 else "k_gemv_q8_0"),
    }


def run_workload(name: str, steps: int, warmup: int, profile_iters: int, want_cpu: bool, cpu_seconds: float,
                 cpu_variants: bool = True, full_run: bool = False):
    from openasr_amd import decoders as D
    from openasr_amd import ggml as g

    wl = D.WORKLOADS[name]
    plugin = g.plugin()
    t0 = time.time()
    w = D.QwenWeights(wl.wtype, seed=1234, **wl.shape)
    model = D.QwenModel(w, plugin.backend)
    sess = model.session(wl.n_seq, wl.max_positions)
    emb, prompt = D.workload_inputs(wl, seed=77)
    log(f"[bench] {name}: weights synthesised and uploaded in {time.time() - t0:.1f}s")

    t0 = time.time()
    sess.prefill_embeddings(emb)
    first = sess.prefill_tokens(prompt)
    prefill_s = time.time() - t0
    n_prefill = wl.n_seq * (wl.prefix + wl.prompt)
    log(f"[bench] prefill {n_prefill} positions in {prefill_s * 1e3:.1f} ms")

    # The workload's greedy decode runs at positions p_first .. p_first +
    # decode - 1 (the step at position p writes KV row p and attends over rows
    # 0..p, so the step time grows with p). The timed steps are centred on
    # the workload's mean position, so their rate is the whole decode's rate:
    # the untimed steps before them (at least `warmup`) decode the tokens
    # that precede that span.
    p_first = wl.prefix + wl.prompt
    steps = min(steps, wl.max_positions - p_first - warmup)
    centre = p_first + (wl.decode - 1) / 2
    lead = max(warmup, int(round(centre - (steps - 1) / 2)) - p_first)
    lead = min(lead, wl.max_positions - p_first - steps)
    out, _ = sess.generate(first, lead)
    cur = out[-1] if lead else first
    pos0 = sess.position(0)
    t0 = time.perf_counter()
    out, step_ms = sess.generate(cur, steps)
    elapsed = time.perf_counter() - t0
    tok_s = wl.n_seq * steps / elapsed
    timed_positions = [pos0, pos0 + steps - 1]
    log(f"[bench] {steps} decode steps at positions {timed_positions[0]}-{timed_positions[1]}: "
        f"{elapsed * 1e3 / steps:.3f} ms/step, {tok_s:.1f} tokens/s (median step {np.median(step_ms):.3f} ms)")

    # per-launch-group times of one decode step: HIP events on the backend stream around each group,
    # the groups queued behind a short spin so they run back to back
    prof = plugin.profile(sess.decode_graph(), profile_iters)
    kern = {}
    for lab, ms in prof:
        k = lab.split(":", 1)[0]
        kern.setdefault(k, [0.0, 0])
        kern[k][0] += ms
        kern[k][1] += 1
    wb = weight_bytes(wl.shape, wl.wtype)
    # every quantized GEMV launch of the step (plain, residual-epilogue and
    # gate+up SwiGLU launches all carry the "mul_mat" label prefix)
    gemv_key = "mul_mat_q4_K" if wl.wtype == g.Q4_K else "mul_mat_q8_0"
    gemv_ms = sum(v[0] for k, v in kern.items() if k.startswith("mul_mat"))
    gemv_n = sum(v[1] for k, v in kern.items() if k.startswith("mul_mat"))
    # activation bytes per step: int8 quants in, f32 results out, per matrix
    d, hd, ffn = wl.shape["d_model"], wl.shape["head_dim"], wl.shape["ffn"]
    q_w, kv_w = wl.shape["n_head"] * hd, wl.shape["n_kv_head"] * hd
    mats = [(q_w + 2 * kv_w, d), (d, q_w), (ffn, d), (ffn, d), (d, ffn)] * wl.shape["n_layers"]
    mats.append((wl.shape["vocab"], d))
    act_bytes = sum(k * wl.n_seq + 4 * m * wl.n_seq for m, k in mats)
    alg_bytes = sum(wb.values()) + act_bytes
    gemv_gbs = alg_bytes / (gemv_ms * 1e-3) / 1e9
    eager_ms = sum(ms for _, ms in prof)
    breakdown = {k: {"ms": round(v[0], 4), "launches": v[1]} for k, v in sorted(kern.items(), key=lambda kv: -kv[1][0])}
    log(f"[bench] profiled step {eager_ms:.3f} ms over {len(prof)} launch groups; {gemv_key}: {gemv_n} launches, "
        f"{gemv_ms:.3f} ms, {gemv_gbs:.0f} GB/s = {gemv_gbs / HBM_PEAK_GBS:.1%} of HBM peak")
    for k, v in breakdown.items():
        log(f"    {k:>16}: {v['ms']:.4f} ms over {v['launches']} launches")

    cpu = None
    if want_cpu:
        cpu = cpu_baseline(w, wl, sess, out[-1], cpu_seconds, variants=cpu_variants)
    full = None
    if full_run:
        # the workload's whole greedy decode from a fresh prefill, every step timed
        sess.free()
        sess = model.session(wl.n_seq, wl.max_positions)
        sess.prefill_embeddings(emb)
        first = sess.prefill_tokens(prompt)
        p0 = sess.position(0)
        n = min(wl.decode, wl.max_positions - p0)
        t0 = time.perf_counter()
        _, fms = sess.generate(first, n)
        dt = time.perf_counter() - t0
        full = {"steps": n, "positions": [p0, p0 + n - 1], "tokens_per_s": round(wl.n_seq * n / dt, 1),
                "ms_per_step": round(dt * 1e3 / n, 4), "first_step_ms": round(float(fms[0]), 4),
                "last_step_ms": round(float(fms[-1]), 4)}
        log(f"[bench] {name} full decode: {n} steps at positions {p0}-{p0 + n - 1}, {dt * 1e3 / n:.3f} ms/step, "
            f"{full['tokens_per_s']:.1f} tokens/s (first step {fms[0]:.3f} ms, last {fms[-1]:.3f} ms)")
    # the whole step's algorithmic bytes at the timed positions: every weight
    # once, each sequence's attended K/V rows (0..p, f16), the GEMV
    # activations; over the measured step time
    kv_row = wl.shape["n_layers"] * 2 * kv_w * 2
    kv_bytes = wl.n_seq * kv_row * float(np.mean([p + 1 for p in range(pos0, pos0 + steps)]))
    step_bytes = sum(wb.values()) + act_bytes + kv_bytes
    step_gbs = step_bytes / (elapsed / steps) / 1e9
    whole_step = {"alg_bytes": round(step_bytes), "weight_bytes": round(sum(wb.values())),
                  "kv_bytes": round(kv_bytes), "activation_bytes": act_bytes, "achieved": round(step_gbs, 1),
                  "frac": round(step_gbs / HBM_PEAK_GBS, 4)}
    log(f"[bench] whole step: {step_bytes / 1e6:.1f} MB (weights {sum(wb.values()) / 1e6:.1f}, attended KV "
        f"{kv_bytes / 1e6:.1f}, activations {act_bytes / 1e6:.1f}) per {elapsed * 1e3 / steps:.3f} ms = "
        f"{step_gbs:.0f} GB/s = {step_gbs / HBM_PEAK_GBS:.1%} of HBM peak")
    result = dict(tok_s=tok_s, ms_per_step=elapsed * 1e3 / steps, steps=steps, prefill_ms=prefill_s * 1e3,
                  n_prefill=n_prefill, gemv_ms=gemv_ms, gemv_launches=gemv_n, gemv_gbs=gemv_gbs,
                  weight_bytes=alg_bytes, eager_step_ms=eager_ms, breakdown=breakdown, cpu=cpu,
                  timed_positions=timed_positions, full=full, untimed_steps=lead, whole_step=whole_step)
    sess.free()
    model.free()
    w.free()
    return result


def encoder_flops(shape: dict, n_frames: int) -> float:
    """algorithmic multiply-add work of one encode, x 2 (conv stem, projections,
    attention scores and context)"""
    chunks = -(-n_frames // 100)
    c, d, f, L = shape["conv_channels"], shape["d_model"], shape["ffn"], shape["n_layers"]
    sizes = [100]
    mels = [shape["n_mels"]]
    for _ in range(3):
        sizes.append((sizes[-1] - 1) // 2 + 1)
        mels.append((mels[-1] - 1) // 2 + 1)
    rows = chunks * sizes[3]
    macs = chunks * (sizes[1] * mels[1] * c * 9 + sizes[2] * mels[2] * c * c * 9 + sizes[3] * mels[3] * c * c * 9)
    macs += rows * c * mels[3] * d                         # conv_out
    macs += L * rows * (4 * d * d + 2 * d * f)             # q, k, v, o, up, down
    macs += L * 2 * rows * rows * d                        # scores and context
    macs += rows * d * d + rows * d * shape["out_dim"]     # proj1, proj2
    return 2.0 * macs


def run_audio_encoder(n_frames: int = 3000, reps: int = 10):
    """Qwen3-ASR-0.6B-shaped audio encoder (18 layers of 896, 480 conv
    channels, 128 mel bins) over n_frames seeded N(0,1) mel frames, with f16
    projections (an fp16 pack) and Q8_0 ones (a quantized pack: the acoustic
    encoder's Q8_0 floor): the encode's wall time over `reps` calls"""
    from openasr_amd import decoders as D
    from openasr_amd import ggml as g

    plugin = g.plugin()
    shape = D.QWEN3_06B_AUDIO
    mel = np.random.default_rng(31).standard_normal((shape["n_mels"], n_frames)).astype(np.float32)
    flops = encoder_flops(shape, n_frames)
    res = {"workload": f"qwen3-asr-0.6b-shaped audio encoder, {n_frames} mel frames "
                       f"({D.qwen_audio_token_count(n_frames)} rows)", "gflop": round(flops / 1e9, 2)}
    for name, wt in (("f16", g.F16), ("q8_0", g.Q8_0)):
        w = D.QwenAudioWeights(wt, seed=5, **shape)
        enc = D.QwenAudioEncoder(w, plugin.backend)
        enc.encode(mel)  # builds the graph
        t0 = time.perf_counter()
        times = []
        for _ in range(reps):
            _, ms = enc.encode(mel)
            times.append(ms)
        wall = (time.perf_counter() - t0) * 1e3 / reps
        best = min(times)
        res[name] = {"ms": round(float(np.median(times)), 3), "best_ms": round(best, 3),
                     "wall_ms_with_io": round(wall, 3), "tflops": round(flops / (best * 1e-3) / 1e12, 2)}
        log(f"[bench] audio encoder {name}: {np.median(times):.2f} ms/encode (best {best:.2f}), "
            f"{flops / (best * 1e-3) / 1e12:.1f} TFLOP/s")
        enc.free()
        w.free()
    return res


def run_whisper(n_tokens: int, cpu_seconds: float):
    """Whisper-tiny-shaped Q8_0 decoder at batch 1: cross K/V precompute from
    1500 N(0,1) encoder frames, 4 prompt tokens, then `n_tokens` greedy steps
    through the persistent step graph; the CPU oracle's step timed beside it."""
    from openasr_amd import decoders as D
    from openasr_amd import ggml as g

    plugin = g.plugin()
    shape = D.WHISPER_TINY
    w = D.WhisperWeights(seed=4321, **shape)
    model = D.WhisperModel(w, plugin.backend)
    sess = model.session()
    enc, prompt = D.whisper_inputs(shape, n_prompt=4, seed=91)
    sess.set_encoder(enc)  # builds and warms the encoder graph
    t0 = time.perf_counter()
    sess.set_encoder(enc)
    cross_ms = (time.perf_counter() - t0) * 1e3
    tok = 0
    for t in prompt:
        tok = sess.step(int(t))
    n_tokens = min(n_tokens, shape["max_positions"] - len(prompt) - 1)
    p0 = sess.position()
    t0 = time.perf_counter()
    out, step_ms = sess.generate(tok, n_tokens)
    elapsed = time.perf_counter() - t0
    tok_s = n_tokens / elapsed
    log(f"[bench] whisper-tiny q8_0 b1: cross K/V {cross_ms:.2f} ms, {n_tokens} greedy steps {elapsed * 1e3 / n_tokens:.3f} "
        f"ms/step = {tok_s:.1f} tokens/s")
    res = {"tokens_per_s": round(tok_s, 1), "ms_per_step": round(elapsed * 1e3 / n_tokens, 4), "steps": n_tokens,
           "positions": [p0, p0 + n_tokens - 1],
           "cross_kv_ms": round(cross_ms, 3), "cpu_tokens_per_s": None}
    if cpu_seconds > 0:
        from oracle import ref
        threads = usable_cpus()
        r = ref.WhisperRef(w.cfg, w.pointer_table(), threads=threads)
        r.set_encoder(enc)
        cur, n = int(prompt[0]), 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds and n < shape["max_positions"] - 1:
            cur, _ = r.step(cur)
            n += 1
        dt = time.perf_counter() - t0
        res["cpu_tokens_per_s"] = round(n / dt, 2)
        res["cpu_threads"] = threads
        log(f"[bench] whisper cpu oracle: {n} steps in {dt:.1f}s on {threads} threads = {n / dt:.1f} tokens/s")
    sess.free()
    model.free()
    w.free()
    return res


def measured_copy_gbs(reps: int = 20) -> float:
    """HBM bandwidth a plain device copy reaches through the backend: a 1 GiB
    f32 CONT (read 1 GiB + write 1 GiB per compute), timed over graph replays"""
    from openasr_amd import ggml as g

    plugin = g.plugin()
    n = 256 << 20  # floats
    G = g.Graph(n_tensors=8, graph_size=16)
    src = G.new(g.F32, n)
    dst = G.lib.ggml_cont(G.ctx, G.lib.ggml_reshape_2d(G.ctx, src, 1 << 20, 256))
    G.build(dst)
    G.allocate(plugin.buft)
    G.set(src, np.zeros(n, np.float32))
    sec = _timed_graph(G, plugin.backend, reps)
    G.free()
    gbs = 2 * 4 * n / sec / 1e9
    log(f"[bench] device copy 1 GiB -> 1 GiB: {sec * 1e3:.3f} ms = {gbs:.0f} GB/s")
    return gbs


def usable_cpus() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_model() -> str:
    return cpu_description()["model"]


def cpu_description() -> dict:
    """host CPU as /proc/cpuinfo gives it: model name, physical cores (distinct
    (physical id, core id) pairs), logical CPUs, the SIMD ISA flags the
    oracle's kernels can use, and the cores this process may run on"""
    model, flags, cores, logical = "unknown", set(), set(), 0
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "processor":
                    logical += 1
                elif key == "model name":
                    model = val
                elif key == "flags":
                    flags = set(val.split())
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    core = val
                elif not key and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    isa = [f for f in ("sse4_2", "avx", "avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vl", "avx512_vnni",
                       "avx512_bf16", "avx_vnni", "amx_tile", "amx_int8") if f in flags]
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = logical
    return {"model": model, "physical_cores": len(cores) or None, "logical_cpus": logical, "isa": isa,
            "usable_cpus": affinity}


def cpu_baseline(w, wl, sess, tokens, seconds: float, variants: bool = True):
    """The CPU baseline: the batched decode step of the same workload on the
    host cores, continuing from the device's KV state, for a bounded sample of
    ~`seconds`. The timed leg is the ggml-cpu-class restatement
    (oracle/cpu_fast.c: int8 block dots in SIMD registers -- AVX-512 VNNI
    where the host has it -- with f32 block accumulation, ggml-cpu's f16 V
    accumulator, rows split over the threads) on every usable core, then on
    the reference's decoder thread policy (available / 2, at least 2,
    ggml_runtime/cpu_graph.rs:511-524) and on one thread. The oracle's own
    step (f64 block sums, the checker) is timed beside it for reference."""
    from oracle import ref

    threads = usable_cpus()
    legs = {"fast": ref.QwenFastBatch(w.cfg, w.pointer_table(), wl.max_positions, wl.n_seq, threads=threads),
            "oracle": ref.QwenRefBatch(w.cfg, w.pointer_table(), wl.max_positions, wl.n_seq, threads=threads)}
    for r in legs.values():
        for s in range(wl.n_seq):
            for layer in range(wl.shape["n_layers"]):
                k, v = sess.read_kv(layer, s)
                r.k[s][layer][...] = k
                r.v[s][layer][...] = v
            r.pos[s] = sess.position(s)
    start = int(legs["fast"].pos.min())
    pos0 = {name: r.pos.copy() for name, r in legs.items()}
    cur = {name: np.asarray(tokens, np.int32) for name in legs}

    def timed(name: str, th: int, budget: float):
        # every sample starts at the device's position (the cache rows past it
        # are rewritten), so each thread count decodes the same span
        r = legs[name]
        r.pos[...] = pos0[name]
        cur[name] = np.asarray(tokens, np.int32)
        r.threads = th
        n = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget and r.pos.max() < wl.max_positions - 1:
            cur[name] = r.step(cur[name])
            n += 1
        dt = time.perf_counter() - t0
        return n, dt, wl.n_seq * n / max(dt, 1e-9)

    n, dt, val = timed("fast", threads, seconds)
    isa = "AVX-512 VNNI" if ref.fast_uses_vnni() else "AVX2"
    log(f"[bench] cpu ggml-cpu-class restatement ({isa}): {n} batched decode steps in {dt:.1f}s on {threads} threads "
        f"= {val:.2f} tokens/s")
    res = {"value": round(val, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
           "label": "ggml-cpu-class restatement",
           "sample": f"{n} batched decode steps of {wl.name} (oracle/cpu_fast.c fast_qwen_decode_batch: {isa} int8 "
                     f"block dots with f32 block sums, f16 V accumulator, {threads} OpenMP threads) continuing from "
                     f"the device KV state at position {start}",
           "cpu": cpu_model(), "host": cpu_description()}
    if variants:
        half = max(2, threads // 2)
        _, _, val2 = timed("fast", half, seconds / 3)
        _, _, val1 = timed("fast", 1, seconds / 3)
        log(f"[bench] cpu ggml-cpu-class restatement: {val2:.2f} tokens/s on {half} threads, {val1:.2f} tokens/s on "
            "1 thread")
        res.update(tokens_per_s_half_threads=round(val2, 3), half_threads=half, tokens_per_s_1_thread=round(val1, 3))
    no, dto, valo = timed("oracle", threads, seconds / 3)
    log(f"[bench] cpu oracle (checker, f64 block sums): {no} steps in {dto:.1f}s on {threads} threads = {valo:.2f} "
        "tokens/s")
    res["oracle_tokens_per_s"] = round(valo, 3)
    return res


# ------------------------------------------------------------ kernel sweep --

MFMA_INT8_PEAK = 5000.0  # TFLOP/s-equivalent (int8 dense, published)
ROTATE_BYTES = 640 << 20  # rotate operands past the 256 MB last-level cache


def _timed_graph(G, backend, reps: int) -> float:
    """seconds per compute of an allocated graph, after eager + capture runs"""
    for _ in range(3):
        if G.compute(backend) != 0:
            raise RuntimeError("graph compute failed")
    t0 = time.perf_counter()
    for _ in range(reps):
        G.compute(backend)
    return (time.perf_counter() - t0) / reps


def sweep_mul_mat(plugin, g, M, K, wtype, N, reps, prec=0):
    bpw = 144 / 256 if wtype == g.Q4_K else 34 / 32
    wbytes = M * K * bpw
    copies = max(1, min(2048, int(ROTATE_BYTES // wbytes)))
    copies = max(1, min(copies, int((1 << 30) // (M * N * 4))))
    w = g.synth_normal(2024, 1, M * K, 0.0, 0.02).reshape(M, K)
    wq = g.quantize(wtype, w)
    x = g.synth_normal(2025, 2, K * N).reshape(N, K)
    G = g.Graph(n_tensors=4 * copies + 16, graph_size=4 * copies + 64)
    X = G.new(g.F32, K, N)
    Ws = [G.new(wtype, K, M, weight=True) for _ in range(copies)]
    outs = [G.lib.ggml_mul_mat(G.ctx, W, X) for W in Ws]
    for o in outs:
        G.lib.ggml_mul_mat_set_prec(o, prec)
    G.build(*outs)
    G.allocate(plugin.buft)
    for W in Ws:
        G.set(W, wq)
    G.set(X, x)
    dt = _timed_graph(G, plugin.backend, reps) / copies
    G.free()
    alg = wbytes + (K * N if N <= 16 else 4 * K * N) + 4 * M * N
    return dict(op="mul_mat", type=g.TYPE_NAMES[wtype], prec="f32" if prec == g.GGML_PREC_F32 else "default",
                M=M, K=K, N=N, copies=copies, us=dt * 1e6,
                gbs=alg / dt / 1e9, frac_hbm=alg / dt / 1e9 / HBM_PEAK_GBS,
                tops=2.0 * M * K * N / dt / 1e12)


def sweep_fattn(plugin, g, n_kv, n_q, reps, d=128, hq=16, hkv=8, prec=0):
    kv_bytes = 2 * n_kv * hkv * d * 2
    copies = max(1, min(256, int(ROTATE_BYTES // kv_bytes)))
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, hq, n_q, d)).astype(np.float32)
    k = rng.standard_normal((1, hkv, n_kv, d)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((1, hkv, n_kv, d)).astype(np.float16).view(np.uint16)
    mask = np.zeros((1, n_q, n_kv), np.float16)
    for i in range(n_q):  # the last n_q positions are causal
        mask[0, i, n_kv - n_q + i + 1:] = -np.inf
    G = g.Graph(n_tensors=4 * copies + 16, graph_size=2 * copies + 64)
    Q = G.new(g.F32, d, n_q, hq, 1)
    Mk = G.new(g.F16, n_kv, n_q, 1, 1)
    Ks = [G.new(g.F16, d, n_kv, hkv, 1, weight=True) for _ in range(copies)]
    Vs = [G.new(g.F16, d, n_kv, hkv, 1, weight=True) for _ in range(copies)]
    outs = [G.lib.ggml_flash_attn_ext(G.ctx, Q, Ks[i], Vs[i], Mk, 1.0 / np.sqrt(d), 0.0, 0.0) for i in range(copies)]
    for o in outs:
        G.lib.ggml_flash_attn_ext_set_prec(o, prec)
    G.build(*outs)
    G.allocate(plugin.buft)
    for i in range(copies):
        G.set(Ks[i], k)
        G.set(Vs[i], v)
    G.set(Q, q)
    G.set(Mk, mask.view(np.uint16))
    dt = _timed_graph(G, plugin.backend, reps) / copies
    G.free()
    alg = kv_bytes + 2 * hq * n_q * d * 4 + n_q * n_kv * 2
    return dict(op="flash_attn_ext", prec="f32" if prec == g.GGML_PREC_F32 else "default", D=d, hq=hq, hkv=hkv,
                n_kv=n_kv, n_q=n_q, copies=copies, us=dt * 1e6,
                gbs=alg / dt / 1e9, frac_hbm=alg / dt / 1e9 / HBM_PEAK_GBS,
                tflops=4.0 * hq * n_q * n_kv * d / dt / 1e12)


def run_sweep(reps: int) -> int:
    """mul_mat on Q8_0/Q4_K weights M x K in {1024^2, 3072x1024, 1024x3072,
    151936x1024} for N in {1, 8, 64, 512} and the batch-8 prefill products
    (N = 2048), wide ones at both precisions, and flash_attn_ext (16 query /
    8 kv heads, D 128, f16 KV of {512, 2048, 8192} positions, q_len {1, 64,
    256}; several queries at both precision contracts).
    Operands are rotated over copies totalling more than the 256 MB cache, so
    the rates are HBM rates. One JSON line per case."""
    from openasr_amd import ggml as g

    plugin = g.plugin()
    for wtype in (g.Q8_0, g.Q4_K):
        shapes = [(M, K, N) for M, K in ((1024, 1024), (3072, 1024), (1024, 3072), (151936, 1024))
                  for N in (1, 8, 64, 512)]
        # the prefill products of the Qwen3-0.6B / 1.7B batch-8 chunks (2048 columns)
        shapes += [(4096, 1024, 2048), (3072, 1024, 2048), (2048, 6144, 2048), (6144, 2048, 2048)]
        for M, K, N in shapes:
            # wide products at both precision contracts (the default takes the
            # f16 matrix-core form where planned)
            for prec in ((g.GGML_PREC_DEFAULT, g.GGML_PREC_F32) if N > 16 else (g.GGML_PREC_DEFAULT,)):
                r = sweep_mul_mat(plugin, g, M, K, wtype, N, reps, prec=prec)
                log(f"[sweep] mul_mat {r['type']:>4} {r['prec']:>7} {M:>6}x{K:<5} N={N:<4} {r['us']:9.2f} us  "
                    f"{r['gbs']:8.1f} GB/s ({r['frac_hbm']:.1%} HBM)  {r['tops']:7.2f} TOP/s")
                print(json.dumps(r), flush=True)
    for n_kv in (512, 2048, 8192):
        for n_q, prec in ((1, g.GGML_PREC_DEFAULT), (64, g.GGML_PREC_DEFAULT), (64, g.GGML_PREC_F32),
                          (256, g.GGML_PREC_DEFAULT), (256, g.GGML_PREC_F32)):
            r = sweep_fattn(plugin, g, n_kv, n_q, reps, prec=prec)
            log(f"[sweep] flash_attn_ext {r['prec']:>7} kv={n_kv:<5} q={n_q:<3} {r['us']:9.2f} us  "
                f"{r['gbs']:8.1f} GB/s ({r['frac_hbm']:.1%} HBM)  {r['tflops']:7.2f} TFLOP/s")
            print(json.dumps(r), flush=True)
    return 0


def run_traffic_probe(workload: str) -> int:
    """A short fixed program for hardware-counter runs (rocprofv3 --pmc):
    a 256 MiB f32 copy through the backend (known bytes: the counters' scale)
    followed by two eager decode steps of the workload. Prints nothing but
    progress; the counters come from the profiler's output."""
    from openasr_amd import decoders as D
    from openasr_amd import ggml as g

    plugin = g.plugin()
    n = 64 << 20  # floats
    G = g.Graph(n_tensors=8, graph_size=16)
    src = G.new(g.F32, n)
    dst = G.lib.ggml_cont(G.ctx, G.lib.ggml_reshape_2d(G.ctx, src, 1 << 20, 64))
    G.build(dst)
    G.allocate(plugin.buft)
    G.set(src, np.zeros(n, np.float32))
    assert G.compute(plugin.backend) == 0
    G.free()
    log("[probe] copy of 256 MiB done")
    wl = D.WORKLOADS[workload]
    w = D.QwenWeights(wl.wtype, seed=1234, **wl.shape)
    model = D.QwenModel(w, plugin.backend)
    sess = model.session(wl.n_seq, wl.max_positions)
    emb, prompt = D.workload_inputs(wl, seed=77)
    sess.prefill_embeddings(emb)
    cur = sess.prefill_tokens(prompt)
    log("[probe] prefill done")
    for _ in range(2):
        cur = sess.step(cur)
    log("[probe] two decode steps done")
    sess.free()
    model.free()
    w.free()
    return 0


def run_mfma_probe() -> int:
    """the prefill-shaped kernels once each (a few computes of one-copy
    graphs), for `rocprofv3 --pmc` runs: the tile GEMM at the vocabulary
    projection's shape and the wide attention, at the default precision (the
    f16 matrix-core forms) and then under GGML_PREC_F32 (the exact forms)"""
    from openasr_amd import ggml as g

    plugin = g.plugin()
    global ROTATE_BYTES
    ROTATE_BYTES = 1  # one copy of each operand
    for prec in (g.GGML_PREC_DEFAULT, g.GGML_PREC_F32):
        for wtype in (g.Q4_K, g.Q8_0):
            r = sweep_mul_mat(plugin, g, 151936, 1024, wtype, 512, 2, prec=prec)
            log(f"[probe] mul_mat {r['type']} {r['prec']} 151936x1024 N=512: {r['us']:.1f} us, "
                f"{r['tops']:.1f} TOP/s")
        r = sweep_fattn(plugin, g, 8192, 64, 2, prec=prec)
        log(f"[probe] flash_attn_ext {r['prec']} kv 8192 x 64 queries: {r['us']:.1f} us, {r['tflops']:.2f} TFLOP/s")
    return 0


def main() -> int:
    a = parse()
    if a.sweep:
        return run_sweep(a.sweep_reps)
    if a.mfma_probe:
        return run_mfma_probe()
    if a.traffic_probe:
        return run_traffic_probe(a.workload)
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU per process (asked for {a.gpus}); the decoder path has no "
              "multi-GPU collectives", file=sys.stderr)
        return 2
    from openasr_amd import ggml as g

    log(f"[bench] backend {g.plugin().name}")
    if a.encoder_only:
        print(json.dumps({"audio_encoder": run_audio_encoder()}))
        return 0
    main_r = run_workload(a.workload, a.steps, a.warmup, a.profile_iters, not a.no_cpu, a.cpu_seconds,
                          full_run=not a.no_full)
    b1 = None
    if not a.no_b1 and a.workload != "qwen3-0.6b-q8_0-b1":
        r1 = run_workload("qwen3-0.6b-q8_0-b1", min(a.steps, 128), a.warmup, a.profile_iters, not a.no_cpu,
                          min(4.0, a.cpu_seconds), cpu_variants=False, full_run=not a.no_full)
        b1 = {"tokens_per_s": round(r1["tok_s"], 1), "ms_per_step": round(r1["ms_per_step"], 4),
              "timed_positions": r1["timed_positions"], "mul_mat_q8_0_gbs": round(r1["gemv_gbs"], 1),
              "cpu_tokens_per_s": r1["cpu"]["value"] if r1["cpu"] else None, "full_decode": r1["full"]}
    long = None
    if not a.no_long and a.workload != "qwen3-1.7b-q4_K-b8":
        rl = run_workload("qwen3-1.7b-q4_K-b8", min(a.steps, 64), a.warmup, max(4, a.profile_iters // 4), False, 0)
        long = {"tokens_per_s": round(rl["tok_s"], 1), "ms_per_step": round(rl["ms_per_step"], 4),
                "prefill_positions": rl["n_prefill"], "prefill_ms": round(rl["prefill_ms"], 1),
                "mul_mat_q4_K_gbs": round(rl["gemv_gbs"], 1)}
    encoder = None
    if not a.no_encoder:
        encoder = run_audio_encoder()
    whisper = None
    if not a.no_whisper:
        whisper = run_whisper(224, 0 if a.no_cpu else min(5.0, a.cpu_seconds))
    copy_gbs = measured_copy_gbs()
    frac = main_r["gemv_gbs"] / HBM_PEAK_GBS
    # measured HBM bytes per GEMV launch (rocprofv3 FETCH_SIZE / WRITE_SIZE
    # runs of `bench.py --traffic-probe`, summarised by openasr_amd.pmc)
    traffic, traffic_source = None, None
    tpath = ROOT / "profiles" / f"gemv_traffic_{a.workload}.json"
    if tpath.exists():
        tj = json.loads(tpath.read_text())
        traffic = round(tj["decode_step"]["gemv_hbm_bytes_per_launch"], 1)
        traffic_source = (f"not measured in this run: profiles/{tpath.name} (rocprofv3 FETCH_SIZE and WRITE_SIZE "
                          f"passes of bench.py --traffic-probe) at commit {tj.get('commit', 'unrecorded')}")
    main_wl_text = workload_text(a.workload)
    out = {
        "metric": main_wl_text["metric"],
        "value": round(main_r["tok_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": main_r["steps"],
        "warmup": a.warmup,
        "ms_per_step": round(main_r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": main_wl_text["dtype"],
        "data": main_wl_text["data"],
        "config": {"workload": a.workload, "model": main_wl_text["model"], "global_batch": main_wl_text["batch"],
                   "seq_len": main_wl_text["seq_len"], "prefill_positions": main_r["n_prefill"],
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(main_r["gemv_gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(frac, 4), "traffic": traffic, "traffic_source": traffic_source,
                     "copy_gbs_measured": round(copy_gbs, 1),
                     "alg_bytes_per_launch": round(main_r["weight_bytes"] / max(1, main_r["gemv_launches"]), 1),
                     "launches": main_r["gemv_launches"],
                     "whole_step": main_r["whole_step"],
                     "kernel": f"{main_wl_text['kernel']}: the quantized GEMV launches of one decode step (per layer QKV, "
                               "o-proj+residual, gate+up SwiGLU, down+residual; lm_head), algorithmic bytes "
                               "(weights + int8 activations + f32 outputs) / summed launch time"},
        "cpu_baseline": main_r["cpu"],
        "timed_positions": main_r["timed_positions"],
        "untimed_steps_before": main_r["untimed_steps"],
        "full_decode": main_r["full"],
        "prefill_ms": round(main_r["prefill_ms"], 2),
        "eager_step_ms": round(main_r["eager_step_ms"], 4),
        "kernels": main_r["breakdown"],
        "batch1_q8_0": b1,
        "qwen3_1.7b_q4_K_b8_kv4096": long,
        "whisper_tiny_q8_0_b1": whisper,
        "qwen3_asr_audio_encoder": encoder,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
