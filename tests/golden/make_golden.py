"""Writes tests/golden/oracle_fixtures.npz: seeded inputs and the CPU
oracle's outputs for the decoder path's operations, at sizes small enough to
commit. They are regression fixtures of this build's own restatement (the
reference holds no golden vectors for the path: its goldens are real-audio
transcripts that need real model packs), checked two ways by the tests: the
oracle must still reproduce every fixture bit for bit, and the device must
reproduce the op fixtures bit for bit.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import ref  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_fixtures.npz")


def fixtures() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20261201)
    f: dict[str, np.ndarray] = {}
    # weight quantizers (ggml_quantize_chunk) on N(0, 0.02) rows
    w = (rng.standard_normal((6, 512)) * 0.02).astype(np.float32)
    f["quant_in"] = w
    f["q8_0_bytes"] = ref.quantize_weights(ref.Q8_0, w)
    f["q4_K_bytes"] = ref.quantize_weights(ref.Q4_K, w)
    # activation quantizers (src1 -> vec_dot_type)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    f["act_in"] = x
    f["act_q8_0_bytes"] = np.concatenate([ref.quantize_act(ref.Q8_0, r) for r in x])
    f["act_q8_K_bytes"] = np.concatenate([ref.quantize_act(ref.Q8_K, r) for r in x])
    # mul_mat: Q4_K 96x512 and Q8_0 64x256, N = 5
    for name, typ, m, k in (("mm_q4_K", ref.Q4_K, 96, 512), ("mm_q8_0", ref.Q8_0, 64, 256)):
        wq = ref.quantize_weights(typ, (rng.standard_normal((m, k)) * 0.02).astype(np.float32))
        xa = rng.standard_normal((5, k)).astype(np.float32)
        f[name + "_w"] = wq
        f[name + "_x"] = xa
        f[name + "_y"] = ref.mul_mat(typ, wq, m, k, xa)
    # norms, rope, softmax, activations
    xn = (rng.standard_normal((4, 384)) * 2 + 0.5).astype(np.float32)
    f["norm_in"] = xn
    f["rms_norm_out"] = ref.rms_norm(xn, 1e-6)
    f["layer_norm_out"] = ref.norm(xn, 1e-5)
    xr = rng.standard_normal((3, 4, 128)).astype(np.float32)
    pos = np.array([0, 17, 1023], np.int32)
    f["rope_in"] = xr
    f["rope_pos"] = pos
    f["rope_out"] = ref.rope_neox(xr, pos, 128, 1e6)
    xs = rng.standard_normal((3, 70)).astype(np.float32) * 4
    mask = np.zeros((3, 70), np.float16)
    mask[1, 40:] = -np.inf
    f["softmax_in"] = xs
    f["softmax_mask"] = mask.view(np.uint16)
    f["softmax_out"] = ref.soft_max_ext(xs, mask.view(np.uint16), 0.125)
    xa = np.linspace(-8, 8, 257, dtype=np.float32)
    f["act_fn_in"] = xa
    f["silu_out"] = ref.silu(xa)
    f["gelu_out"] = ref.gelu(xa)
    # flash attention (chunked definition): GQA 2 query heads on 1 kv head, D 64,
    # 130 positions, one query position per sequence of 2, the second with its
    # last 30 masked
    q = rng.standard_normal((2, 2, 64)).astype(np.float32)
    kk = rng.standard_normal((2, 1, 130, 64)).astype(np.float16).view(np.uint16)
    vv = rng.standard_normal((2, 1, 130, 64)).astype(np.float16).view(np.uint16)
    fm = np.zeros((2, 130), np.float16)
    fm[1, 100:] = -np.inf
    f["fa_q"] = q
    f["fa_k"] = kk
    f["fa_v"] = vv
    f["fa_mask"] = fm.view(np.uint16)
    f["fa_out"] = np.stack([ref.flash_attn(q[s:s + 1], kk[s], vv[s], fm[s:s + 1].view(np.uint16), 0.125,
                                           fidelity=4) for s in range(2)])
    f["fa5_out"] = np.stack([ref.flash_attn(q[s:s + 1], kk[s], vv[s], fm[s:s + 1].view(np.uint16), 0.125,
                                            fidelity=5) for s in range(2)])
    return f


def main() -> int:
    np.savez_compressed(OUT, **fixtures())
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
