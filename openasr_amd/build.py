"""Build the native libraries in-tree.

  openasr_amd/lib/libggml-base.so    host-side ggml-base (g++)
  openasr_amd/lib/libggml-mi355x.so  the gfx950 backend plugin (hipcc)
  openasr_amd/lib/libopenasr-models.so  decoder graph builders / step loops (g++)
  oracle/build/libggml_cpu_ref.so    the CPU oracle (gcc; test infrastructure)

Run `python -m openasr_amd.build` (or __graft_entry__.build()). Every call
recompiles; objects go to _build/ (not committed).
"""

from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "openasr_amd"
LIB = PKG / "lib"
OBJ = ROOT / "_build"
INCLUDE = ROOT / "include"
ORACLE = ROOT / "oracle"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # results must not depend on whether the compiler fuses a*b+c: the CPU
    # reference evaluates every expression with separate roundings
    "-ffp-contract=off",
    # MFMA results in ordinary VGPRs: the integer sums are scaled by VALU
    # code right after each MFMA, and results in AGPRs would cost a
    # v_accvgpr_read per value first
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result",
]


def host_abi_fingerprint() -> str:
    """Fingerprint of the ABI headers the host and the plugin are built against."""
    h = hashlib.sha256()
    h.update(b"schema=openasr-mi355x-1\nbackend_api_version=3\n")
    for name in ("ggml_abi.h", "ggml_host.h"):
        h.update((INCLUDE / name).read_bytes())
    return h.hexdigest()


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")


def build_base(fp: str) -> Path:
    out = LIB / "libggml-base.so"
    srcs = sorted(str(p) for p in (PKG / "host").glob("*.cpp"))
    # no contraction of a * b + c: the weight quantizers reproduce ggml-base's
    # float operation order bit for bit
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", f"-I{INCLUDE}",
          f'-DOPENASR_HOST_ABI_FINGERPRINT="{fp}"', *srcs, "-o", str(out), "-ldl"])
    return out


def build_models() -> Path:
    out = LIB / "libopenasr-models.so"
    srcs = sorted(str(p) for p in (PKG / "decoders").glob("*.cpp"))
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", f"-I{INCLUDE}", *srcs, "-o", str(out),
          f"-L{LIB}", "-lggml-base", "-Wl,-rpath,$ORIGIN"])
    return out


def build_plugin(fp: str) -> Path:
    out = LIB / "libggml-mi355x.so"
    csrc = PKG / "csrc"
    srcs = sorted(csrc.glob("*.cpp")) + sorted((csrc / "kernels").glob("*.hip"))
    objs = []
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        for src in srcs:
            obj = OBJ / (src.stem + ".o")
            objs.append(obj)
            cmd = [HIPCC, *HIP_FLAGS, "-x", "hip", f"-I{INCLUDE}", f"-I{csrc}",
                   f'-DOPENASR_HOST_ABI_FINGERPRINT="{fp}"', "-c", str(src), "-o", str(obj)]
            jobs.append(ex.submit(_run, cmd))
        for j in jobs:
            j.result()
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(out),
          f"-L{LIB}", "-lggml-base", "-Wl,-rpath,$ORIGIN"])
    return out


def build_oracle() -> Path:
    out_dir = ORACLE / "build"
    out_dir.mkdir(exist_ok=True)
    out = out_dir / "libggml_cpu_ref.so"
    srcs = sorted(str(p) for p in ORACLE.glob("*.c"))
    _run(["gcc", "-O3", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-march=x86-64-v3", *srcs, "-o", str(out), "-lm"])
    return out


def build_all(plugin: bool = True) -> dict[str, Path]:
    LIB.mkdir(parents=True, exist_ok=True)
    OBJ.mkdir(parents=True, exist_ok=True)
    fp = host_abi_fingerprint()
    built = {"base": build_base(fp), "oracle": build_oracle()}
    built["models"] = build_models()
    if plugin:
        built["plugin"] = build_plugin(fp)
    return built


if __name__ == "__main__":
    for k, v in build_all().items():
        print(f"{k}: {v}")
