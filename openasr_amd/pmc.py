"""Summaries of rocprofv3 hardware-counter runs of the decode benchmark.

`python bench.py --traffic-probe` is a fixed short program: a 256 MiB f32
copy through the backend (the copy kernel reads and writes exactly 256 MiB), then two
eager decode steps. Run it twice under `rocprofv3 --pmc FETCH_SIZE` and
`rocprofv3 --pmc WRITE_SIZE` (one counter per run, `--output-format csv`),
then

    python -m openasr_amd.pmc FETCH_DIR WRITE_DIR [--workload NAME] [--out JSON]

scales each counter by what it reads for the copy (bytes moved / counter
value) and reports HBM bytes per dispatch by kernel, and for the last decode
step the bytes the quantized GEMV launches moved against their algorithmic
bytes (weights + int8 activations + f32 outputs).

    python -m openasr_amd.pmc --counters RUN_DIR [--only NAME]

tabulates a run with several counters (e.g. the MFMA and VALU busy metrics
over `bench.py --mfma-probe`): per kernel and grid, the mean per dispatch.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import sys
from collections import defaultdict

COPY_BYTES = 256 << 20


def _rows(d: str):
    paths = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no counter_collection.csv under {d}")
    out = []
    for p in paths:
        with open(p, newline="") as f:
            out.extend(csv.DictReader(f))
    out.sort(key=lambda r: int(r["Dispatch_Id"]))
    return out


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "")
    return name.split("(")[0].replace("void ", "").replace("mi355x::", "")


def _per_dispatch(rows):
    """dispatch id -> (kernel, grid, counter KiB)"""
    return {int(r["Dispatch_Id"]): (_short(r["Kernel_Name"]), int(r["Grid_Size"]), float(r["Counter_Value"]))
            for r in rows}


def _copy_scale(disp, bytes_moved: int) -> float:
    """bytes moved / counter value of the calibration copy (the largest copy
    dispatch of the run: the 256 MiB one)"""
    vals = [v for k, g, v in disp.values() if k.startswith("k_copy")]
    if not vals:
        raise RuntimeError("the calibration copy is missing from the counter run")
    return bytes_moved / (max(vals) * 1024.0)


def _last_step(disp):
    """dispatch ids of the last decode step (between the last two argmax finals)"""
    ends = [i for i, (k, _, _) in sorted(disp.items()) if k == "k_argmax_final"]
    if len(ends) < 2:
        raise RuntimeError("fewer than two decode steps in the counter run")
    return [i for i in sorted(disp) if ends[-2] < i <= ends[-1]]


def gemv_algorithmic_bytes(shape: dict, wtype_q4k: bool, n_seq: int) -> tuple[float, int]:
    bpw = 144 / 256 if wtype_q4k else 34 / 32
    d, hd, ffn = shape["d_model"], shape["head_dim"], shape["ffn"]
    q_w, kv_w = shape["n_head"] * hd, shape["n_kv_head"] * hd
    mats = [(q_w + 2 * kv_w, d), (d, q_w), (ffn, d), (ffn, d), (d, ffn)] * shape["n_layers"]
    mats.append((shape["vocab"], d))
    total = sum(m * k * bpw + k * n_seq + 4 * m * n_seq for m, k in mats)
    launches = 4 * shape["n_layers"] + 1  # qkv, o(+res), gate+up, down(+res); lm_head
    return total, launches


def summarize(fetch_dir: str, write_dir: str, workload: str | None = None) -> dict:
    fd, wd = _per_dispatch(_rows(fetch_dir)), _per_dispatch(_rows(write_dir))
    fs, ws = _copy_scale(fd, COPY_BYTES), _copy_scale(wd, COPY_BYTES)
    kern = defaultdict(lambda: [0, 0.0, 0.0])
    for i, (k, g, v) in fd.items():
        key = f"{k}[{g}]"
        kern[key][0] += 1
        kern[key][1] += v * 1024.0 * fs
        if i in wd:
            kern[key][2] += wd[i][2] * 1024.0 * ws
    out = {"copy_bytes": COPY_BYTES, "fetch_scale": fs, "write_scale": ws,
           "kernels": {k: {"dispatches": n, "fetch_bytes_avg": f / n, "write_bytes_avg": w / n}
                       for k, (n, f, w) in sorted(kern.items())}}
    step = _last_step(fd)
    gemv = [i for i in step if fd[i][0].startswith("k_gemv_") or fd[i][0].startswith("k_mmv_")]
    traffic = sum(fd[i][2] * 1024.0 * fs + wd.get(i, ("", 0, 0.0))[2] * 1024.0 * ws for i in gemv)
    out["decode_step"] = {"gemv_launches": len(gemv), "gemv_hbm_bytes": traffic,
                          "gemv_hbm_bytes_per_launch": traffic / max(1, len(gemv))}
    if workload:
        sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
        from openasr_amd import decoders as D
        from openasr_amd import ggml as g
        wl = D.WORKLOADS[workload]
        alg, launches = gemv_algorithmic_bytes(wl.shape, wl.wtype == g.Q4_K, wl.n_seq)
        out["decode_step"].update(workload=workload, gemv_algorithmic_bytes=alg,
                                  gemv_algorithmic_bytes_per_launch=alg / launches,
                                  traffic_over_algorithmic=traffic / alg)
    return out


def markdown(s: dict) -> str:
    """the per-step GEMV figure and the per-kernel table of a summary"""
    d = s["decode_step"]
    lines = [f"Scale factors (bytes moved / counter bytes on the copy): FETCH_SIZE x {s['fetch_scale']:.4f}, "
             f"WRITE_SIZE x {s['write_scale']:.4f}.", "",
             "Last decode step, quantized GEMV launches only:", "",
             "| launches | HBM bytes (scaled FETCH+WRITE) | algorithmic bytes | ratio |", "|---|---|---|---|"]
    if "gemv_algorithmic_bytes" in d:
        lines.append(f"| {d['gemv_launches']} | {d['gemv_hbm_bytes'] / 1e6:.1f} MB "
                     f"({d['gemv_hbm_bytes_per_launch'] / 1e6:.3f} MB / launch) | "
                     f"{d['gemv_algorithmic_bytes'] / 1e6:.1f} MB ({d['gemv_algorithmic_bytes_per_launch'] / 1e6:.3f} "
                     f"MB / launch) | {d['traffic_over_algorithmic']:.3f} |")
    lines += ["", "Per kernel (all dispatches of the probe, prefill included; grid in threads):", "",
              "| kernel[grid] | dispatches | FETCH MB / dispatch | WRITE MB / dispatch |", "|---|---|---|---|"]
    for k, v in s["kernels"].items():
        lines.append(f"| {k} | {v['dispatches']} | {v['fetch_bytes_avg'] / 1e6:.3f} | {v['write_bytes_avg'] / 1e6:.3f} |")
    return "\n".join(lines)


def counters(run_dir: str) -> dict:
    """per kernel[grid] the mean per dispatch of every counter of a
    multi-counter run (one row per counter per dispatch in the CSV)"""
    per = defaultdict(dict)
    names = {}
    for r in _rows(run_dir):
        i = int(r["Dispatch_Id"])
        per[i][r["Counter_Name"]] = float(r["Counter_Value"])
        names[i] = f"{_short(r['Kernel_Name'])}[{r['Grid_Size']}]"
    kern = defaultdict(lambda: defaultdict(list))
    for i, cs in per.items():
        for c, v in cs.items():
            kern[names[i]][c].append(v)
    return {k: {"dispatches": len(next(iter(cs.values()))), **{c: sum(v) / len(v) for c, v in sorted(cs.items())}}
            for k, cs in sorted(kern.items())}


def counters_markdown(s: dict, only: str | None = None) -> str:
    keys = sorted({c for v in s.values() for c in v if c != "dispatches"})
    lines = ["| kernel[grid] | dispatches | " + " | ".join(keys) + " |", "|---" * (len(keys) + 2) + "|"]
    for k, v in s.items():
        if only and only not in k:
            continue
        lines.append(f"| {k} | {v['dispatches']} | " + " | ".join(f"{v.get(c, float('nan')):.4g}" for c in keys) + " |")
    return "\n".join(lines)


def main() -> int:
    if len(sys.argv) > 1 and sys.argv[1] == "--counters":
        ap = argparse.ArgumentParser()
        ap.add_argument("--counters", dest="run_dir", required=True)
        ap.add_argument("--only", default=None, help="kernels whose name contains this")
        a = ap.parse_args()
        print(counters_markdown(counters(a.run_dir), a.only))
        return 0
    ap = argparse.ArgumentParser()
    ap.add_argument("fetch_dir")
    ap.add_argument("write_dir")
    ap.add_argument("--workload", default=None)
    ap.add_argument("--out", default=None)
    ap.add_argument("--md", action="store_true", help="print the markdown tables instead of the JSON")
    ap.add_argument("--commit", default=None, help="the commit the counter runs were taken at (recorded in the JSON)")
    a = ap.parse_args()
    s = summarize(a.fetch_dir, a.write_dir, a.workload)
    if a.commit:
        s["commit"] = a.commit
    text = json.dumps(s, indent=1)
    if a.out:
        with open(a.out, "w") as f:
            f.write(text + "\n")
    print(markdown(s) if a.md else text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
