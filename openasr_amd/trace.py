"""Per-kernel summary of one decode step from a rocprofv3 kernel trace of
`bench.py` (HIP-graph capture off, so every launch is a traced dispatch):

    OPENASR_MI355X_HIP_GRAPHS=0 rocprofv3 --kernel-trace --stats --output-format csv \\
        -d prof_bench -o run -- python3 bench.py --no-cpu --no-long --no-whisper \\
        --steps 16 --warmup 2 --profile-iters 4
    python -m openasr_amd.trace prof_bench/run_kernel_trace.csv

Decode steps are the launches between consecutive `k_argmax_final`
dispatches; the two workloads of the run (Qwen3-0.6B Q4_K batch 8, then Q8_0
batch 1) are told apart by the gap between them. Eight timed steps of each are
averaged (the first three argmax dispatches of a workload belong to prefill
and warmup).
"""

from __future__ import annotations

import argparse
import collections
import csv
import os
import sys


def short_name(kernel: str) -> str:
    """a kernel's name without its namespaces and argument list (kernels in an
    anonymous namespace carry "(anonymous namespace)::" before the name)"""
    k = kernel.replace("(anonymous namespace)::", "")
    return k.split("(")[0].replace("void ", "").replace("mi355x::", "")


def _steps(rows, which: int, n: int = 8, tail: bool = False):
    idx = [i for i, r in enumerate(rows) if "k_argmax_final" in r["Kernel_Name"]]
    groups = [[idx[0]]]
    for a, b in zip(idx, idx[1:]):
        if int(rows[b]["Start_Timestamp"]) - int(rows[a]["End_Timestamp"]) > 200e6:
            groups.append([])
        groups[-1].append(b)
    g = groups[which]
    # tail: the workload's last steps (a long prefill ends in many argmax dispatches of its own)
    a, b = (g[-1 - n], g[-1]) if tail else (g[3], g[3 + n])
    return rows[a + 1:b + 1], n


def table(trace: str, which: int, workload: str, tail: bool = False) -> str:
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    from openasr_amd import decoders as D
    from openasr_amd import ggml as g
    from openasr_amd.pmc import gemv_algorithmic_bytes

    with open(trace, newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    win, n = _steps(rows, which, tail=tail)
    st = collections.defaultdict(list)
    for r in win:
        name = short_name(r["Kernel_Name"])
        if name == "k_spin":  # the profiler's queue-filling spin, not part of a step
            continue
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        st[(name, grid, int(r["Workgroup_Size_X"]))].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    lines = ["| kernel | grid (threads) | workgroup | launches / step | avg us | min us | us / step |",
             "|---|---|---|---|---|---|---|"]
    tot = gemv = gemv_n = 0
    for k, v in sorted(st.items(), key=lambda kv: -sum(kv[1])):
        tot += sum(v)
        if k[0].startswith("k_gemv") or k[0].startswith("k_mmv"):
            gemv += sum(v)
            gemv_n += len(v)
        lines.append(f"| {k[0]} | {k[1]} | {k[2]} | {len(v) / n:.0f} | {sum(v) / len(v) / 1e3:.2f} | "
                     f"{min(v) / 1e3:.2f} | {sum(v) / n / 1e3:.1f} |")
    if workload == "whisper-tiny-q8_0-b1":
        # Q8_0 decoder matrices read per step: self q, k, v, o and cross q, o
        # (the cross K/V projections run once per utterance), fc1, fc2, and
        # the tied output projection; int8 activations in, f32 outputs out
        sh = D.WHISPER_TINY
        d, f, L = sh["d_model"], sh["ffn"], sh["n_layers"]
        mats = [(d, d)] * (6 * L) + [(f, d), (d, f)] * L + [(sh["vocab"], d)]
        alg = sum(m * k * 1.0625 + k + 4 * m for m, k in mats)
    else:
        wl = D.WORKLOADS[workload]
        alg, _ = gemv_algorithmic_bytes(wl.shape, wl.wtype == g.Q4_K, wl.n_seq)
    gemv_us = gemv / n / 1e3
    span = (int(win[-1]["End_Timestamp"]) - int(win[0]["Start_Timestamp"])) / n / 1e3
    lines += ["", f"Kernel time per decode step: {tot / n / 1e3:.1f} us over {len(win) / n:.0f} launches "
                  f"(first start to last end {span:.1f} us with eager launches and profiler overhead).",
              f"Quantized GEMV launches per step: {gemv_n / n:.0f}, {gemv_us:.1f} us; algorithmic bytes "
              f"{alg / 1e6:.1f} MB (weights + int8 activations + f32 outputs) -> {alg / (gemv_us * 1e-6) / 1e9:.0f} GB/s "
              f"= {alg / (gemv_us * 1e-6) / 1e9 / 8000:.1%} of 8 TB/s; average GEMV launch {gemv_us / (gemv_n / n):.2f} us."]
    return "\n".join(lines)


def encoder_tables(trace: str, reps: int = 10) -> str:
    """Per-kernel summary of the audio encoder from a trace of `bench.py
    --encoder-only` (HIP-graph capture off): an encode starts at its first
    IM2COL (the stem's three convolutions each run one, conv1's first); the
    run holds an f16 leg, then a Q8_0 leg, of 1 + `reps` encodes each, and
    the last `reps` of each leg are averaged."""
    with open(trace, newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    starts, n_im = [], 0
    for i, r in enumerate(rows):
        if "im2col" in r["Kernel_Name"]:
            if n_im % 3 == 0:
                starts.append(i)
            n_im += 1
    if len(starts) != 2 * (reps + 1):
        raise SystemExit(f"expected {2 * (reps + 1)} encodes, found {len(starts)}")
    starts.append(len(rows))
    out = []
    for leg, name in enumerate(("F16 projections", "Q8_0 projections")):
        agg = collections.defaultdict(list)
        first = leg * (reps + 1) + 1
        for e in range(first, first + reps):
            enc = rows[starts[e]:starts[e + 1]]
            for r in enc:
                kname = r["Kernel_Name"].replace("(anonymous namespace)::", "")
                key = (short_name(kname),
                       r["Grid_Size_X"], r["Grid_Size_Y"], r["Grid_Size_Z"], r["Workgroup_Size_X"])
                agg[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        lines = [f"## {name}", "", "| kernel | grid (threads x, y, z) | workgroup | launches / encode | avg us | us / encode |",
                 "|---|---|---|---|---|---|"]
        total = 0.0
        for (k, gx, gy, gz, wg), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
            per = sum(v) / reps
            total += per
            if per >= 20.0:
                lines.append(f"| {k} | {gx} x {gy} x {gz} | {wg} | {len(v) / reps:g} | {sum(v) / len(v):.2f} | {per:.1f} |")
        n_launch = sum(len(v) for v in agg.values()) / reps
        lines.append("")
        lines.append(f"Kernel time per encode: {total / 1e3:.3f} ms over {n_launch:g} launches "
                     "(kernels under 20 us an encode not listed).")
        out.append("\n".join(lines))
    return "\n\n".join(out)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--encoder", action="store_true",
                    help="summarise a trace of bench.py --encoder-only (the two audio encoder legs)")
    ap.add_argument("--only", default=None,
                    help="summarise the last steps of the trace as this workload (a WORKLOADS name, or "
                         "whisper-tiny-q8_0-b1 for the Whisper leg that ends a bench.py run)")
    a = ap.parse_args()
    if a.encoder:
        print(encoder_tables(a.trace))
        return 0
    if a.only:
        print(f"## {a.only}\n")
        print(table(a.trace, 0, a.only, tail=True))
        return 0
    print("## Q4_K weights, batch 8\n")
    print(table(a.trace, 0, "qwen3-0.6b-q4_K-b8"))
    print("\n## Q8_0 weights, batch 1\n")
    print(table(a.trace, 1, "qwen3-0.6b-q8_0-b1"))
    return 0


if __name__ == "__main__":
    sys.exit(main())
