"""The benchmark's CPU baseline leg (oracle/cpu_fast.c, the "ggml-cpu-class
restatement": int8 block dots in SIMD registers with f32 block accumulation,
flash attention with an f16 V accumulator) against the oracle, which stays
the checker. The leg sums in f32 where the oracle sums in f64, so it is held
to float tolerance, not to bits."""

import numpy as np
import pytest

RNG = np.random.default_rng(77)


@pytest.mark.parametrize("wname,m,k", [("q4_K", 96, 1024), ("q4_K", 64, 3072), ("q8_0", 96, 1024),
                                       ("q8_0", 40, 384)])
@pytest.mark.parametrize("n", [1, 8])
def test_fast_mul_mat_against_oracle(ref, wname, m, k, n):
    """MUL_MAT of the baseline leg: within 1e-5 (relative to the largest
    output) of the oracle's f64 block sums on the same quantized operands,
    whichever SIMD path the host takes"""
    wt = ref.Q4_K if wname == "q4_K" else ref.Q8_0
    w = ref.quantize_weights(wt, (RNG.standard_normal((m, k)) * 0.02).astype(np.float32))
    x = RNG.standard_normal((n, k)).astype(np.float32)
    got = ref.fast_mul_mat(wt, w, m, k, x, threads=4)
    want = ref.mul_mat(wt, w, m, k, x)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("n_kv", [1, 70, 700])
def test_fast_attention_against_oracle(ref, n_kv):
    """the leg's decode attention against the oracle's ggml-cpu numerics
    (fidelity 1: f16 query, f16 V accumulator) within 2e-3 of the largest
    output, and against the f64 textbook within the f16 accumulator's error;
    masked positions ignored"""
    d = 128
    q = RNG.standard_normal((1, 1, d)).astype(np.float32)
    k = RNG.standard_normal((1, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((1, n_kv, d)).astype(np.float16)
    mask = np.zeros((1, n_kv), np.float16)
    mask[0, n_kv // 3: n_kv // 2] = -np.inf
    scale = 1 / np.sqrt(d)
    got = ref.fast_attn_one(q[0, 0], k[0].view(np.uint16), v[0].view(np.uint16), mask[0].view(np.uint16), scale)
    f1 = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=1)[0, 0]
    f0 = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=3)[0, 0]
    top = max(1e-6, float(np.abs(f0).max()))
    assert np.abs(got - f1).max() <= 2e-3 * top
    assert np.abs(got - f0).max() <= 2e-2 * top


def test_fast_decode_step_against_oracle(ref):
    """one batched decode step of a small Qwen3-shaped decoder from a shared
    KV state: the same greedy tokens as the oracle, logits within 3% of their
    range. The int8 activation quantization turns the leg's f32 block sums
    and f16 V accumulator into whole quantization steps here and there
    (~1% of the logits); a wiring mistake moves them by tens of percent."""
    from openasr_amd import decoders as D
    from openasr_amd import ggml as g
    shape = dict(d_model=256, n_layers=2, n_head=4, n_kv_head=2, head_dim=128, ffn=512, vocab=1000)
    w = D.QwenWeights(g.Q4_K, seed=5, **shape)
    n_seq, max_pos, past = 3, 128, 70
    table = w.pointer_table()
    a = ref.QwenRefBatch(w.cfg, table, max_pos, n_seq)
    b = ref.QwenFastBatch(w.cfg, table, max_pos, n_seq, threads=4)
    for s in range(n_seq):  # a shared random history in the caches
        for layer in range(shape["n_layers"]):
            kv = (RNG.standard_normal((2, shape["n_kv_head"], max_pos, shape["head_dim"])) * 0.5).astype(np.float16)
            for r in (a, b):
                r.k[s][layer][...] = kv[0].view(np.uint16)
                r.v[s][layer][...] = kv[1].view(np.uint16)
        a.pos[s] = b.pos[s] = past + s
    tokens = np.array([3, 500, 999], np.int32)
    ta, la = a.step(tokens, want_logits=True)
    tb, lb = b.step(tokens, want_logits=True)
    assert np.abs(la - lb).max() < 3e-2 * max(1.0, np.abs(la).max())
    assert np.array_equal(ta, tb)
    w.free()
