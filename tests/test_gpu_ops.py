"""Per-op parity of the MI355X plugin against the CPU oracle, through the C
ABI exactly as the host drives it: a ggml graph built with libggml-base,
allocated on the plugin's buffer type, computed by the plugin backend.

The bar is bit-identical results (2e-3 per op). Integer
block dots are exact and every cross-lane / cross-chunk sum is carried in f64
and rounded once, exp / sin / cos are evaluated by the same deterministic
sequence on both sides, and nothing is FMA-contracted, so device and oracle
agree bit for bit except for a vanishing fraction of values whose f64 sum
lands on an f32 rounding boundary. Attention is also held to the f64 textbook
result and must be at least as accurate as ggml-cpu's numerics (whose V
accumulator is f16).
"""

import ctypes
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(2024)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def assert_same_bits(a, b, max_frac=1e-5):
    """device == reference bit for bit, allowing a vanishing fraction of
    values that sit on an f32 rounding boundary of an f64-accumulated sum"""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    diff = a.view(np.int32) != b.view(np.int32)
    assert diff.mean() <= max_frac, f"{diff.sum()} of {diff.size} values differ, max rel {rel_err(a, b):.2e}"
    assert rel_err(a, b) < 1e-6


def run(ggml, gpu, G, out):
    G.build(out)
    G.allocate(gpu.buft)


# ------------------------------------------------------------- mul_mat --

MM_CASES = [
    ("q8_0", 64, 256), ("q8_0", 1024, 1024), ("q8_0", 3072, 1024), ("q8_0", 1024, 3072), ("q8_0", 384, 384),
    ("q8_0", 1536, 384), ("q8_0", 384, 1536), ("q4_K", 64, 256), ("q4_K", 1024, 1024), ("q4_K", 3072, 1024),
    ("q4_K", 1024, 3072), ("q4_K", 4096, 2048), ("q4_K", 2048, 6144),
    # 384 row tiles at 8 columns: two tiles a workgroup (one round of the CUs)
    ("q4_K", 6144, 2048),
    # M not a multiple of the tile GEMM's 64 rows (its last row tile has idle waves)
    ("q4_K", 1040, 512), ("q8_0", 1040, 384),
    # rows off the 16-row tile (a vocabulary of 51865: the single-column form at N = 1)
    ("q8_0", 1000, 384),
]


@pytest.mark.parametrize("wname,m,k", MM_CASES)
@pytest.mark.parametrize("n", [1, 2, 8, 13, 64, 100])
def test_mul_mat_quantized(ggml, gpu, ref, wname, m, k, n):
    wt = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
    print(f"mul_mat {wname} M={m} K={k} N={n}", flush=True)
    w = ggml.synth_normal(11, m * 7 + k, m * k, 0.0, 0.02).reshape(m, k)
    x = RNG.standard_normal((n, k)).astype(np.float32)
    wq = ggml.quantize(wt, w)
    G = ggml.Graph()
    W = G.new(wt, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    y = G.get(Y).reshape(n, m)
    want = ref.mul_mat(wt, wq, m, k, x)
    assert_same_bits(y, want)
    # the weight round-trips through the device layout byte for byte
    assert np.array_equal(G.get(W, np.uint8), wq)
    G.free()


@pytest.mark.parametrize("m,k", [(64, 256), (1024, 1024), (3072, 1024), (1000, 3072)])
@pytest.mark.parametrize("n", [1, 3, 8, 13])
def test_mul_mat_q3_K(ggml, gpu, ref, m, k, n):
    """MUL_MAT on Q3_K weights (the host's q3_k pack policy): the row-team
    GEMV over Q8_K columns, bit for bit the oracle's; the blocks come from
    random bytes with finite f16 scales (every such block is a valid Q3_K
    block), since nothing here writes Q3_K weights"""
    print(f"mul_mat q3_K M={m} K={k} N={n}", flush=True)
    rng = np.random.default_rng(m + 7 * k + n)
    nb = m * k // 256
    wq = rng.integers(0, 256, (nb, 110), dtype=np.uint8)
    wq[:, 108:110] = np.float16(rng.uniform(0.001, 0.01, nb)).view(np.uint8).reshape(nb, 2)
    wq = wq.reshape(-1)
    x = rng.standard_normal((n, k)).astype(np.float32)
    G = ggml.Graph()
    W = G.new(ggml.Q3_K, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    G.set(X, x)
    for _ in range(2):
        assert G.compute(gpu.backend) == 0
        y = G.get(Y).reshape(n, m)
        assert_same_bits(y, ref.mul_mat(ref.Q3_K, wq, m, k, x))
    G.free()


NORM_MM_CASES = [
    # norm, weights, M, K, N
    ("rms", "q4_K", 4096, 1024, 8), ("rms", "q4_K", 4096, 2048, 8), ("rms", "q4_K", 1024, 1024, 13),
    ("rms", "q4_K", 3072, 1024, 20), ("rms", "q8_0", 4096, 1024, 1), ("rms", "q8_0", 1024, 1024, 8),
    ("layer", "q8_0", 384, 384, 1), ("layer", "q8_0", 1536, 384, 3), ("layer", "q4_K", 1024, 1024, 2),
]


@pytest.mark.parametrize("norm,wname,m,k,n", NORM_MM_CASES)
def test_norm_then_mul_mat_prologue(ggml, gpu, ref, norm, wname, m, k, n):
    """RMS_NORM / NORM -> MUL(w) (-> ADD(b)) -> two MUL_MATs reading the
    normalised activations: the norm launch is folded into both GEMVs'
    activation prologue (no norm step in the plan), results bit-exact"""
    wt = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
    print(f"{norm}_norm -> mul_mat {wname} M={m} K={k} N={n}", flush=True)
    x = (RNG.standard_normal((n, k)) * 1.5 + 0.3).astype(np.float32)
    wn = RNG.standard_normal(k).astype(np.float32)
    bn = RNG.standard_normal(k).astype(np.float32) * 0.1
    wq1 = ggml.quantize(wt, ggml.synth_normal(12, m + k, m * k, 0.0, 0.02).reshape(m, k))
    wq2 = ggml.quantize(wt, ggml.synth_normal(13, m + k, m * k, 0.0, 0.02).reshape(m, k))
    G = ggml.Graph()
    X = G.new(ggml.F32, k, n)
    WN = G.new(ggml.F32, k, weight=True)
    BN = G.new(ggml.F32, k, weight=True)
    W1 = G.new(wt, k, m, weight=True)
    W2 = G.new(wt, k, m, weight=True)
    if norm == "rms":
        h = G.lib.ggml_mul(G.ctx, G.lib.ggml_rms_norm(G.ctx, X, 1e-6), WN)
    else:
        h = G.lib.ggml_add(G.ctx, G.lib.ggml_mul(G.ctx, G.lib.ggml_norm(G.ctx, X, 1e-5), WN), BN)
    Y = G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, W1, h), G.lib.ggml_mul_mat(G.ctx, W2, h))
    run(ggml, gpu, G, Y)
    for T, v in ((X, x), (WN, wn), (BN, bn), (W1, wq1), (W2, wq2)):
        G.set(T, v)
    assert G.compute(gpu.backend) == 0
    y = G.get(Y).reshape(n, m)
    hn = (ref.rms_norm(x, 1e-6) * wn) if norm == "rms" else (ref.norm(x, 1e-5) * wn + bn)
    want = ref.mul_mat(wt, wq1, m, k, hn) + ref.mul_mat(wt, wq2, m, k, hn)
    assert_same_bits(y, want)
    labels = [lab.split(":")[0] for lab, _ in gpu.profile(G.gf, 1)]
    assert not any("norm" in lab or "quantize" in lab for lab in labels), labels
    G.free()


TALL_CASES = [
    # weights, M, K, N: the vocabulary projections of the Qwen3 shapes, and a
    # tile count that leaves a partial batch, at K = 2048 (eight waves)
    ("q4_K", 151936, 1024, 8), ("q8_0", 151936, 1024, 1), ("q4_K", 151936, 1024, 16),
    ("q4_K", 32784, 2048, 3), ("q8_0", 32784, 2048, 8),
]


@pytest.mark.parametrize("wname,m,k,n", TALL_CASES)
def test_mul_mat_lm_head_full_size(ggml, gpu, ref, wname, m, k, n):
    """tall decode GEMVs (the streaming launch walks batches of tiles),
    bit-exact, same argmax"""
    wt = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
    print(f"tall mul_mat {wname} M={m} K={k} N={n}", flush=True)
    w = ggml.synth_normal(5, 99, m * k, 0.0, 0.02).reshape(m, k)
    wq = ggml.quantize(wt, w)
    x = RNG.standard_normal((n, k)).astype(np.float32)
    G = ggml.Graph()
    W = G.new(wt, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    y = G.get(Y).reshape(n, m)
    want = ref.mul_mat(wt, wq, m, k, x)
    assert_same_bits(y, want)
    assert np.array_equal(y.argmax(1), want.argmax(1))
    G.free()


SWEEP_CASES = [
    # the kernel-sweep points: every M x K at N = 512 in both formats, and the
    # vocabulary projection at N = 1, 8, 64 and 512
    *[(w, m, k, 512) for w in ("q8_0", "q4_K") for m, k in ((1024, 1024), (3072, 1024), (1024, 3072))],
    ("q4_K", 151936, 1024, 1), ("q8_0", 151936, 1024, 8), ("q4_K", 151936, 1024, 64), ("q8_0", 151936, 1024, 64),
    ("q4_K", 151936, 1024, 512), ("q8_0", 151936, 1024, 512),
]


@pytest.mark.parametrize("wname,m,k,n", SWEEP_CASES)
def test_mul_mat_sweep_points(ggml, gpu, ref, wname, m, k, n):
    """the mul_mat sweep's shapes at the column counts the other tests leave
    out, under GGML_PREC_F32 (the exact forms; wide products at the default
    precision run on the f16 matrix cores, tested below): bit-exact against
    the oracle, same argmax per column"""
    wt = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
    print(f"sweep mul_mat {wname} M={m} K={k} N={n}", flush=True)
    wq = ggml.quantize(wt, ggml.synth_normal(7, m + 3 * k, m * k, 0.0, 0.02).reshape(m, k))
    x = RNG.standard_normal((n, k)).astype(np.float32)
    G = ggml.Graph()
    W = G.new(wt, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    G.lib.ggml_mul_mat_set_prec(Y, ggml.GGML_PREC_F32)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    y = G.get(Y).reshape(n, m)
    want = ref.mul_mat(wt, wq, m, k, x)
    assert_same_bits(y, want)
    assert np.array_equal(y.argmax(1), want.argmax(1))
    G.free()


# the f16 matrix-core tile GEMM (quantized weights, wide columns, the
# default precision): weights, M, K, N, epilogue. The vocabulary projection
# at 512 columns and at 300 (a partial column tile) in both formats; the
# Qwen3-0.6B QKV and the Qwen3-1.7B down projection (with its residual) of a
# batch-8 prefill chunk; a Q8_0 projection with bias and GELU_ERF; rows off
# the 128-row tile with 160 columns and a bias (Q4_K) or 96 (Q8_0).
MMQ16_CASES = [
    ("q4_K", 151936, 1024, 512, None), ("q8_0", 151936, 1024, 512, None), ("q4_K", 151936, 1024, 300, None),
    ("q4_K", 4096, 1024, 2048, None), ("q4_K", 2048, 6144, 2048, "res"), ("q8_0", 3072, 1024, 2048, "bias_gelu"),
    ("q4_K", 32784, 2048, 160, "bias"), ("q8_0", 32784, 2048, 96, None),
]


@pytest.mark.parametrize("wname,m,k,n,tail", MMQ16_CASES)
def test_mul_mat_f16_matrix_cores(ggml, gpu, ref, wname, m, k, n, tail):
    """a quantized MUL_MAT over wide columns at the default precision runs on
    the f16 matrix cores (activations quantized as for the exact path, then
    both operands dequantized to f16, f32 sums): within 2e-3 of the oracle's
    exact product (with the epilogue's adds and GELU_ERF), same argmax in
    every column where the oracle's top-2 margin exceeds the error; graph
    replays give the same bits"""
    wt = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
    print(f"f16 tile gemm {wname} M={m} K={k} N={n} tail={tail}", flush=True)
    wq = ggml.quantize(wt, ggml.synth_normal(8, m + k, m * k, 0.0, 0.02).reshape(m, k))
    rng = np.random.default_rng(m + n)
    x = rng.standard_normal((n, k)).astype(np.float32)
    b = rng.standard_normal(m).astype(np.float32)
    r = rng.standard_normal((n, m)).astype(np.float32)
    G = ggml.Graph()
    L = G.lib
    W = G.new(wt, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    B = G.new(ggml.F32, m, weight=True)
    R = G.new(ggml.F32, m, n)
    Y = L.ggml_mul_mat(G.ctx, W, X)
    want = ref.mul_mat(wt, wq, m, k, x)
    if tail and "bias" in tail:
        Y = L.ggml_add(G.ctx, Y, B)
        want = want + b
    if tail and "res" in tail:
        Y = L.ggml_add(G.ctx, R, Y)
        want = want + r
    if tail and "gelu" in tail:
        from scipy.special import erf  # the exact GELU_ERF: the 2e-3 bar dwarfs its rounding
        Y = L.ggml_gelu_erf(G.ctx, Y)
        w64 = want.astype(np.float64)
        want = 0.5 * w64 * (1.0 + erf(w64 / math.sqrt(2.0)))
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    G.set(X, x)
    if tail and "bias" in tail:
        G.set(B, b)
    if tail and "res" in tail:
        G.set(R, r)
    assert G.compute(gpu.backend) == 0
    labels = plan_labels(gpu, G)
    assert f"mul_mat_f16_{wname}" in labels, labels
    y = G.get(Y).reshape(n, m)
    err = rel_err(y, want)
    print(f"  vs the exact product: {err:.2e}", flush=True)
    assert err < 2e-3
    assert np.isfinite(y).all()
    if tail is None:
        top2 = np.sort(want, axis=1)[:, -2:]
        clear = top2[:, 1] - top2[:, 0] > 2 * err * np.abs(want).max()
        assert np.array_equal(y.argmax(1)[clear], want.argmax(1)[clear])
    first = y.copy()
    for _ in range(2):  # captured, then replayed
        assert G.compute(gpu.backend) == 0
        assert np.array_equal(G.get(Y).reshape(n, m).view(np.uint32), first.view(np.uint32))
    G.free()


@pytest.mark.parametrize("wname,m,k,n", [("q4_K", 6144, 2048, 1024), ("q4_K", 3072, 1024, 2048),
                                         ("q8_0", 3072, 1024, 1408), ("q4_K", 3008, 1024, 1300)])
def test_mul_mat_swiglu_f16_matrix_cores(ggml, gpu, ref, wname, m, k, n):
    """the prefill FFN gate: MUL(SILU(MUL_MAT(gate, x)), MUL_MAT(up, x)) at
    the default precision is one f16 tile GEMM launch (a tile's 64 gate rows
    and the same 64 up rows, combined in its epilogue): within 2e-3 of
    silu(exact gate product) * exact up product from the oracle, graph
    replays bit-identical; under GGML_PREC_F32 the products stay exact and
    the graph bit for bit the oracle's"""
    wt = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
    print(f"f16 swiglu {wname} M={m} K={k} N={n}", flush=True)
    wg = ggml.quantize(wt, ggml.synth_normal(11, m + k, m * k, 0.0, 0.02).reshape(m, k))
    wu = ggml.quantize(wt, ggml.synth_normal(12, m + k, m * k, 0.0, 0.02).reshape(m, k))
    x = np.random.default_rng(m + k + n).standard_normal((n, k)).astype(np.float32)
    gate, up = ref.mul_mat(wt, wg, m, k, x), ref.mul_mat(wt, wu, m, k, x)
    for prec in (None, ggml.GGML_PREC_F32):
        G = ggml.Graph()
        L = G.lib
        Wg = G.new(wt, k, m, weight=True)
        Wu = G.new(wt, k, m, weight=True)
        X = G.new(ggml.F32, k, n)
        Pg, Pu = L.ggml_mul_mat(G.ctx, Wg, X), L.ggml_mul_mat(G.ctx, Wu, X)
        if prec is not None:
            L.ggml_mul_mat_set_prec(Pg, prec)
            L.ggml_mul_mat_set_prec(Pu, prec)
        Y = L.ggml_mul(G.ctx, L.ggml_silu(G.ctx, Pg), Pu)
        run(ggml, gpu, G, Y)
        G.set(Wg, wg)
        G.set(Wu, wu)
        G.set(X, x)
        assert G.compute(gpu.backend) == 0
        labels = plan_labels(gpu, G)
        y = G.get(Y).reshape(n, m)
        if prec is None:
            assert f"mul_mat_swiglu_f16_{wname}" in labels, labels
            g64 = gate.astype(np.float64)
            want = g64 / (1.0 + np.exp(-g64)) * up.astype(np.float64)
            err = rel_err(y, want)
            print(f"  vs the exact products: {err:.2e}", flush=True)
            assert err < 2e-3 and np.isfinite(y).all()
        else:
            assert not any("f16" in lab for lab in labels), labels
            assert_same_bits(y, ref.silu(gate) * up)
        first = y.copy()
        for _ in range(2):  # captured, then replayed
            assert G.compute(gpu.backend) == 0
            assert np.array_equal(G.get(Y).reshape(n, m).view(np.uint32), first.view(np.uint32))
        G.free()


def quantizer_edge_activations(n, k, seed):
    """activation columns whose 256-element blocks hit the quantizers' edge
    cases: +A and -A both at the block maximum (the first in element order
    sets the Q8_K sign; pairs in one lane, in neighbouring lanes, across the
    block, either sign first), all-zero blocks, a single non-zero element,
    values exactly at 127/A multiples, and tiny magnitudes"""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, k)).astype(np.float32)
    pairs = [(3, 9), (9, 3), (15, 16), (16, 15), (0, 255), (255, 0), (40, 41), (130, 7)]
    for c in range(n):
        for b in range(k // 256):
            blk = x[c, 256 * b:256 * (b + 1)]
            kind = (c * 7 + b) % 11
            if kind < len(pairs):
                i, j = pairs[kind]
                a = np.float32(4.0 + kind)
                blk[i], blk[j] = a, -a
                blk[(i + 100) % 256] = a if kind % 2 else -a  # a third copy after both
            elif kind == 8:
                blk[:] = 0.0
            elif kind == 9:
                blk[:] = 0.0
                blk[(c * 31 + b) % 256] = -0.75
            else:
                blk *= np.float32(1e-30)
    x[0, :32] = np.arange(-16, 16, dtype=np.float32) * np.float32(127.0 / 16.0)
    return x


@pytest.mark.parametrize("wname,m,k,n,norm", [
    ("q4_K", 1024, 1024, 8, False), ("q4_K", 1024, 3072, 8, False), ("q4_K", 4096, 1024, 8, True),
    ("q4_K", 1024, 2048, 1, False), ("q8_0", 1024, 1024, 8, False), ("q8_0", 1024, 1024, 1, False),
    ("q8_0", 4096, 1024, 1, True),
])
def test_mul_mat_activation_quantizer_edges(ggml, gpu, ref, wname, m, k, n, norm):
    """the GEMVs' in-LDS activation quantizer (plain and behind an RMS norm
    with unit weights, which keeps +-A ties exact) on the blocks of
    quantizer_edge_activations, bit-exact against the oracle"""
    wt = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
    print(f"quantizer edges {wname} M={m} K={k} N={n} norm={norm}", flush=True)
    wq = ggml.quantize(wt, ggml.synth_normal(14, m + k, m * k, 0.0, 0.02).reshape(m, k))
    x = quantizer_edge_activations(n, k, seed=m + k + n)
    if norm:  # keep every column's norm away from zero
        x[:, -1] = np.float32(3.0)
    G = ggml.Graph()
    W = G.new(wt, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    WN = G.new(ggml.F32, k, weight=True)
    h = G.lib.ggml_mul(G.ctx, G.lib.ggml_rms_norm(G.ctx, X, 1e-6), WN) if norm else X
    Y = G.lib.ggml_mul_mat(G.ctx, W, h)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    G.set(X, x)
    if norm:
        G.set(WN, np.ones(k, np.float32))
    assert G.compute(gpu.backend) == 0
    y = G.get(Y).reshape(n, m)
    xin = ref.rms_norm(x, 1e-6) * np.ones(k, np.float32) if norm else x
    want = ref.mul_mat(wt, wq, m, k, xin)
    assert_same_bits(y, want)
    G.free()


def test_mul_mat_f16_weights(ggml, gpu, ref):
    m, k, n = 96, 128, 5
    w = RNG.standard_normal((m, k)).astype(np.float16)
    x = RNG.standard_normal((n, k)).astype(np.float32)
    G = ggml.Graph()
    W = G.new(ggml.F16, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    run(ggml, gpu, G, Y)
    G.set(W, w.view(np.uint16))
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    want = ref.mul_mat(ref.F16, w.view(np.uint16), m, k, x)
    assert rel_err(G.get(Y).reshape(n, m), want) < 1e-5
    G.free()


# weight type, column type, M (rows), K, N (columns), weight batch, column batch
FLOAT_MM_CASES = [
    ("f16", "f32", 1024, 1280, 375, (1, 1), (1, 1)),    # an encoder projection, f16 weights
    ("f16", "f32", 1000, 4320, 97, (1, 1), (1, 1)),     # rows off the 64-row tile
    ("f16", "f16", 480, 9, 1500, (1, 1), (1, 1)),       # first conv of an f16 stem (K = 3 x 3, unaligned rows)
    ("f16", "f16", 480, 4320, 750, (1, 1), (1, 1)),     # later conv (K = 3 x 3 x 480)
    ("f32", "f32", 896, 896, 300, (1, 1), (1, 1)),      # f32 encoder weights
    ("f32", "f32", 1280, 5120, 64, (1, 1), (1, 1)),
    ("f32", "f16", 64, 100, 33, (1, 1), (1, 1)),
    ("f16", "f32", 100, 64, 40, (2, 1), (4, 2)),        # weight batch broadcast over column batches
    ("f32", "f32", 333, 128, 17, (8, 1), (16, 1)),      # score-shaped: kv heads x query heads
    ("f16", "f32", 256, 512, 13, (1, 1), (30, 1)),      # one matrix over 30 chunks of 13 columns (folded)
    ("f32", "f32", 128, 512, 3, (1, 1), (1, 1)),        # three columns, a long K
]


# every case at the default precision; the F32 x F32 ones under GGML_PREC_F32 too
FLOAT_MM_PREC_CASES = [c + ("default",) for c in FLOAT_MM_CASES] + \
    [c + ("f32",) for c in FLOAT_MM_CASES if c[:2] == ("f32", "f32")]


@pytest.mark.parametrize("wt,xt,m,k,n,wb,xb,prec", FLOAT_MM_PREC_CASES)
def test_mul_mat_float_matrix_cores(ggml, gpu, wt, xt, m, k, n, wb, xb, prec):
    """float MUL_MAT on the matrix-core GEMM against an f64 product of the
    same operands, the columns rounded to f16 for f16 weights (ggml-cpu's
    vec_dot_type rule): f32 sums in the matrix core's order, within 1e-4 of
    the largest output (the op tolerance is 2e-3). An F32 x F32 product at
    the default precision runs as three bf16 products of hi / lo operand
    halves (~1e-5); under GGML_PREC_F32 on f32 products"""
    print(f"float mul_mat {wt} x {xt} M={m} K={k} N={n} wb={wb} xb={xb} prec={prec}", flush=True)
    wdt = np.float16 if wt == "f16" else np.float32
    xdt = np.float16 if xt == "f16" else np.float32
    w = RNG.standard_normal((wb[1], wb[0], m, k)).astype(wdt)
    x = RNG.standard_normal((xb[1], xb[0], n, k)).astype(xdt)
    G = ggml.Graph()
    W = G.new(ggml.F16 if wt == "f16" else ggml.F32, k, m, wb[0], wb[1], weight=True)
    X = G.new(ggml.F16 if xt == "f16" else ggml.F32, k, n, xb[0], xb[1])
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    if prec == "f32":
        G.lib.ggml_mul_mat_set_prec(Y, ggml.GGML_PREC_F32)
    run(ggml, gpu, G, Y)
    G.set(W, w.view(np.uint16) if wt == "f16" else w)
    G.set(X, x.view(np.uint16) if xt == "f16" else x)
    assert G.compute(gpu.backend) == 0
    xr = x.astype(np.float16) if wt == "f16" else x
    r2, r3 = xb[0] // wb[0], xb[1] // wb[1]
    wf = np.repeat(np.repeat(w.astype(np.float64), r2, axis=1), r3, axis=0)
    want = np.matmul(xr.astype(np.float64), wf.transpose(0, 1, 3, 2))  # [b3, b2, n, m]
    got = G.get(Y).reshape(xb[1], xb[0], n, m)
    err = rel_err(got, want)
    print(f"  vs f64: {err:.2e}", flush=True)
    assert err < 1e-4
    G.free()


# ----------------------------------------------------- flash attention --

FA_CASES = [
    # d, hq, hkv, n_kv, n_q, n_seq
    (128, 16, 8, 512, 1, 1), (128, 16, 8, 1024, 1, 8), (128, 16, 8, 2048, 1, 1), (128, 16, 8, 8192, 1, 1),
    (128, 16, 8, 512, 64, 1), (128, 16, 8, 2048, 64, 2), (64, 6, 6, 448, 1, 1), (64, 6, 6, 1500, 1, 1),
    (64, 6, 6, 1500, 1, 3), (128, 16, 8, 8192, 64, 1), (128, 32, 8, 256, 1, 2), (64, 16, 2, 192, 1, 1),
]


@pytest.mark.parametrize("prec", ["f32", "default"])
@pytest.mark.parametrize("d,heads,t", [(64, 20, 750), (128, 8, 300), (64, 6, 100)])
def test_flash_attn_ext_f32_kv_head_views(ggml, gpu, ref, d, heads, t, prec):
    """the encoders' self-attention (nn/encoder.rs:735-800): Q, K and V are
    f32 projections [d * heads, t] viewed as heads (reshape [d, heads, t],
    permute to [d, t, heads]) without a CONT, under an f16 block mask. The
    f32 K / V are rounded to f16 (the conversion ggml's GPU backends make).
    GGML_PREC_F32: bit for bit the oracle's chunked attention over the
    f16-rounded K / V; the default precision (the matrix-core form): within
    2e-3 of the f64 textbook attention over the same operands"""
    print(f"flash_attn f32 K/V views D={d} heads={heads} t={t} prec={prec}", flush=True)
    G = ggml.Graph()
    L = G.lib
    P = [G.new(ggml.F32, d * heads, t) for _ in range(3)]
    M = G.new(ggml.F16, t, t)

    def heads_view(x):
        return L.ggml_permute(G.ctx, L.ggml_reshape_3d(G.ctx, x, d, heads, t), 0, 2, 1, 3)

    scale = 1.0 / math.sqrt(d)
    O = L.ggml_flash_attn_ext(G.ctx, heads_view(P[0]), heads_view(P[1]), heads_view(P[2]), M, scale, 0.0, 0.0)
    if prec == "f32":
        L.ggml_flash_attn_ext_set_prec(O, ggml.GGML_PREC_F32)
    run(ggml, gpu, G, O)
    x = [RNG.standard_normal((t, heads, d)).astype(np.float32) for _ in range(3)]
    for Pi, xi in zip(P, x):
        G.set(Pi, xi)
    # block-diagonal mask of 40-row windows, the chunked encoders' padding shape
    blk = np.arange(t) // 40
    mask = np.where(blk[:, None] == blk[None, :], 0.0, -np.inf).astype(np.float16)
    G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    out = G.get(O).reshape(t, heads, d)  # ggml result [d, heads, t]
    k16 = np.ascontiguousarray(x[1].transpose(1, 0, 2)).astype(np.float16)  # [heads, t, d]
    v16 = np.ascontiguousarray(x[2].transpose(1, 0, 2)).astype(np.float16)
    if prec == "f32":
        same = ref.flash_attn(x[0], k16.view(np.uint16), v16.view(np.uint16), mask.view(np.uint16), scale,
                              fidelity=5)
        assert_same_bits(out, same)
    else:
        exact = attention_f64(x[0].astype(np.float16).astype(np.float32), k16, v16, mask, scale)
        err = rel_err(out, exact)
        print(f"  matrix-core form vs f64 textbook: {err:.2e}")
        assert err < 2e-3
        assert "flash_attn_mfma" in plan_labels(gpu, G)
    G.free()


def attention_f64(q, k, v, mask, scale):
    """textbook softmax attention in f64; q [n_q, hq, d], k/v [hkv, n_kv, d]"""
    g = q.shape[1] // k.shape[0]
    kk = np.repeat(k.astype(np.float64), g, axis=0)  # [hq, n_kv, d]
    vv = np.repeat(v.astype(np.float64), g, axis=0)
    s = np.einsum("qhd,hkd->qhk", q.astype(np.float64), kk) * scale
    if mask is not None:
        s = s + mask.astype(np.float64)[:, None, :]
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    return np.einsum("qhk,hkd->qhd", p, vv) / p.sum(-1)[..., None]


@pytest.mark.parametrize("d,hq,hkv,n_kv,n_q,n_seq", FA_CASES)
def test_flash_attn_ext(ggml, gpu, ref, d, hq, hkv, n_kv, n_q, n_seq):
    print(f"flash_attn D={d} Hq={hq} Hkv={hkv} kv={n_kv} nq={n_q} seq={n_seq}", flush=True)
    q = RNG.standard_normal((n_seq, hq, n_q, d)).astype(np.float32)  # ggml [d, n_q, hq, n_seq]
    k = RNG.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    # per sequence a different number of valid positions; the last n_q are causal
    valid = [n_kv - 3 * s for s in range(n_seq)] if n_q == 1 else [n_kv - 64 * s for s in range(n_seq)]
    mask = np.full((n_seq, n_q, n_kv), -np.inf, np.float16)
    for s in range(n_seq):
        for i in range(n_q):
            mask[s, i, :valid[s] - n_q + i + 1] = 0
    cross = d == 64 and n_kv == 1500  # Whisper cross attention has no mask
    G = ggml.Graph()
    Q = G.new(ggml.F32, d, n_q, hq, n_seq)
    K = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    V = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    M = None if cross else G.new(ggml.F16, n_kv, n_q, 1, n_seq)
    scale = 1.0 / math.sqrt(d)
    O = G.lib.ggml_flash_attn_ext(G.ctx, Q, K, V, M, scale, 0.0, 0.0)
    # the full-precision contract keeps the chunked definition (the default
    # precision runs the float-tolerance forms, tested below)
    G.lib.ggml_flash_attn_ext_set_prec(O, ggml.GGML_PREC_F32)
    run(ggml, gpu, G, O)
    G.set(Q, q)
    G.set(K, k.view(np.uint16))
    G.set(V, v.view(np.uint16))
    if M is not None:
        G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    out = G.get(O).reshape(n_seq, n_q, hq, d)
    for s in range(n_seq):
        qs = np.ascontiguousarray(q[s].transpose(1, 0, 2))  # [n_q, hq, d]
        ms = None if cross else mask[s].view(np.uint16)
        same = ref.flash_attn(qs, k[s].view(np.uint16), v[s].view(np.uint16), ms, scale, fidelity=5)
        cpu = ref.flash_attn(qs, k[s].view(np.uint16), v[s].view(np.uint16), ms, scale, fidelity=1)
        # same arithmetic (f16 Q, 64-position chunks, f64 sums): bit for bit
        assert_same_bits(out[s], same)
        # ggml-cpu keeps the V accumulator in f16 (fidelity 1); its error grows
        # ~sqrt(n_kv) f16 ulps. The device is held to the f64 textbook result
        # and must be at least as close to it as the ggml-cpu numerics are.
        exact = attention_f64(qs.astype(np.float16).astype(np.float32), k[s], v[s],
                              None if cross else mask[s], scale)
        e_gpu, e_cpu = rel_err(out[s], exact), rel_err(cpu, exact)
        print(f"  seq {s}: gpu vs f64 {e_gpu:.2e}, ggml-cpu numerics vs f64 {e_cpu:.2e}, "
              f"gpu vs ggml-cpu numerics {rel_err(out[s], cpu):.2e}")
        assert e_gpu < 2e-5 and e_gpu <= e_cpu
    # again, captured and replayed: the same bits every time
    for _ in range(3):
        assert G.compute(gpu.backend) == 0
        assert_same_bits(G.get(O).reshape(n_seq, n_q, hq, d), out)
    G.free()


def test_flash_attn_fully_masked_chunks_are_skipped_exactly(ggml, gpu, ref):
    """positions past the valid length hold garbage; results must not change"""
    d, hq, hkv, n_kv = 128, 16, 8, 4096
    q = RNG.standard_normal((hq, 1, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((1, n_kv), np.float16)
    mask[0, 700:] = -np.inf
    k[:, 700:] = np.float16(60000)
    v[:, 700:] = np.float16(np.nan)
    G = ggml.Graph()
    Q = G.new(ggml.F32, d, 1, hq, 1)
    K = G.new(ggml.F16, d, n_kv, hkv, 1)
    V = G.new(ggml.F16, d, n_kv, hkv, 1)
    M = G.new(ggml.F16, n_kv, 1, 1, 1)
    O = G.lib.ggml_flash_attn_ext(G.ctx, Q, K, V, M, 1 / math.sqrt(d), 0.0, 0.0)
    G.lib.ggml_flash_attn_ext_set_prec(O, ggml.GGML_PREC_F32)
    run(ggml, gpu, G, O)
    G.set(Q, q)
    G.set(K, k.view(np.uint16))
    G.set(V, v.view(np.uint16))
    G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    out = G.get(O).reshape(hq, d)
    want = ref.flash_attn(np.ascontiguousarray(q.transpose(1, 0, 2)), k[:, :700].view(np.uint16).copy(),
                          v[:, :700].view(np.uint16).copy(), mask[:, :700].view(np.uint16).copy(),
                          1 / math.sqrt(d), fidelity=5)[0]
    assert np.isfinite(out).all()
    assert_same_bits(out, want)
    G.free()


# the matrix-core form (several queries at the default precision): d, hq,
# hkv, n_kv, n_q, n_seq, mask kind. Qwen3-0.6B prefill chunks over 512 ..
# 8192 positions (the few-query shapes split the span over workgroups), a
# partial query block and partial last tile, two sequences with their own
# spans, GQA 4 and 8, the encoders' full attention (D 64, one head a kv head)
# under a block mask, Whisper cross attention (no mask), three sequences of
# 200-query chunks over 4096 positions.
FA_MFMA_CASES = [
    (128, 16, 8, 512, 64, 1, "causal"), (128, 16, 8, 2048, 64, 2, "causal"), (128, 16, 8, 8192, 64, 1, "causal"),
    (128, 16, 8, 2048, 256, 1, "causal"), (128, 16, 8, 1000, 37, 1, "causal"), (128, 32, 8, 1024, 70, 1, "causal"),
    (128, 16, 2, 600, 20, 1, "causal"), (64, 20, 20, 750, 750, 1, "block"), (64, 6, 6, 1500, 100, 1, None),
    (128, 16, 8, 4096, 200, 3, "causal"),
]


@pytest.mark.parametrize("d,hq,hkv,n_kv,n_q,n_seq,mkind", FA_MFMA_CASES)
def test_flash_attn_ext_matrix_cores(ggml, gpu, ref, d, hq, hkv, n_kv, n_q, n_seq, mkind):
    """several queries at the default precision run on the matrix cores (f16
    Q K^T and P V, f32 sums and online softmax): within 2e-3 of the f64
    textbook attention over the f16-rounded operands, printed beside the
    ggml-cpu numerics' error; the same graph under GGML_PREC_F32 runs the
    chunked definition, bit for bit the oracle"""
    print(f"flash_attn mfma D={d} Hq={hq} Hkv={hkv} kv={n_kv} nq={n_q} seq={n_seq} mask={mkind}", flush=True)
    q = RNG.standard_normal((n_seq, hq, n_q, d)).astype(np.float32)
    k = RNG.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_seq, n_q, n_kv), np.float16)
    for s in range(n_seq):
        if mkind == "causal":
            mask[s] = causal_mask(n_q, n_kv, n_kv - 64 * s)
        elif mkind == "block":
            blk_q, blk_k = np.arange(n_q) // 100, np.arange(n_kv) // 100
            mask[s] = np.where(blk_q[:, None] == blk_k[None, :], 0.0, -np.inf)
    G = ggml.Graph()
    Q = G.new(ggml.F32, d, n_q, hq, n_seq)
    K = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    V = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    M = None if mkind is None else G.new(ggml.F16, n_kv, n_q, 1, n_seq)
    scale = 1.0 / math.sqrt(d)
    O = G.lib.ggml_flash_attn_ext(G.ctx, Q, K, V, M, scale, 0.0, 0.0)
    O32 = G.lib.ggml_flash_attn_ext(G.ctx, Q, K, V, M, scale, 0.0, 0.0)
    G.lib.ggml_flash_attn_ext_set_prec(O32, ggml.GGML_PREC_F32)
    G.build(O, O32)
    G.allocate(gpu.buft)
    G.set(Q, q)
    G.set(K, k.view(np.uint16))
    G.set(V, v.view(np.uint16))
    if M is not None:
        G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    labels = plan_labels(gpu, G)
    assert "flash_attn_mfma" in labels and "flash_attn_ext" in labels, labels
    out = G.get(O).reshape(n_seq, n_q, hq, d)
    out32 = G.get(O32).reshape(n_seq, n_q, hq, d)
    for s in range(n_seq):
        qs = np.ascontiguousarray(q[s].transpose(1, 0, 2))  # [n_q, hq, d]
        q16 = qs.astype(np.float16).astype(np.float32)
        ms = None if M is None else mask[s]
        exact = attention_f64(q16, k[s], v[s], ms, scale)
        mbits = None if ms is None else ms.view(np.uint16)
        same = ref.flash_attn(qs, k[s].view(np.uint16), v[s].view(np.uint16), mbits, scale, fidelity=5)
        assert_same_bits(out32[s], same)
        cpu = ref.flash_attn(qs, k[s].view(np.uint16), v[s].view(np.uint16), mbits, scale, fidelity=1)
        err, e_cpu = rel_err(out[s], exact), rel_err(cpu, exact)
        print(f"  seq {s}: matrix-core form vs f64 {err:.2e}, ggml-cpu numerics vs f64 {e_cpu:.2e}")
        assert err < 2e-3
        assert np.isfinite(out[s]).all()
    # replays of the captured graph give the same bits
    first = out.copy()
    assert G.compute(gpu.backend) == 0
    assert np.array_equal(G.get(O).reshape(first.shape).view(np.uint32), first.view(np.uint32))
    G.free()


# the single-query workgroup form (one query at the default precision, where
# it is planned: a workgroup for every CU, or spans of at most 512): d, hq,
# hkv, n_kv, n_seq, mask kind. The batch-8 Qwen3-1.7B decode over 4096
# positions (4 splits merged by the combine launch); 8192 positions at batch
# 4 (8 splits); 32 sequences over a 1024-position arena (one split a pair,
# finished in the launch); one head a kv head over a partial last tile; 4
# query heads a kv head with closed positions inside the span; Whisper-tiny
# self attention (448); cross attention without a mask over 1500 frames at
# batch 16 (two splits); 64-wide heads with 4 query heads a kv head. "lens":
# per sequence a live prefix (one sequence with none), everything past it
# garbage (NaN V, huge K).
FA_DEC_CASES = [
    (128, 16, 8, 4096, 8, "lens"), (128, 16, 8, 8192, 4, "lens"), (128, 16, 8, 1024, 32, "lens"),
    (128, 16, 16, 480, 1, "lens"), (128, 32, 8, 500, 2, "holes"), (64, 6, 6, 448, 1, "lens"),
    (64, 8, 8, 1500, 16, None), (64, 8, 2, 300, 3, "holes"),
]


@pytest.mark.parametrize("d,hq,hkv,n_kv,n_seq,mkind", FA_DEC_CASES)
def test_flash_attn_ext_decode_workgroup(ggml, gpu, d, hq, hkv, n_kv, n_seq, mkind):
    """one query at the default precision runs the workgroup form (f16 q K^T
    on the matrix cores, f32 online softmax and P V, the waves merged in the
    launch): within 2e-3 of the f64 textbook attention over the f16-rounded
    query; closed positions contribute nothing even when their K / V rows
    hold NaN or huge values; a query with no open position gives zeros;
    graph replays give the same bits"""
    print(f"flash_attn dec D={d} Hq={hq} Hkv={hkv} kv={n_kv} seq={n_seq} mask={mkind}", flush=True)
    rng = np.random.default_rng(n_kv * 7 + hq)
    q = rng.standard_normal((n_seq, hq, 1, d)).astype(np.float32)
    k = rng.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    v = rng.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_seq, 1, n_kv), np.float16)
    for s in range(n_seq):
        if mkind == "lens":
            live = 0 if (n_seq > 1 and s == n_seq - 1) else n_kv - 3 - (97 * s) % (n_kv - 4)
            mask[s, 0, live:] = -np.inf
            k[s, :, live:] = np.float16(60000)
            v[s, :, live:] = np.float16(np.nan)
        elif mkind == "holes":
            closed = rng.random(n_kv) < 0.3
            mask[s, 0, closed] = -np.inf
            v[s, :, closed] = np.float16(np.nan)
    G = ggml.Graph()
    Q = G.new(ggml.F32, d, 1, hq, n_seq)
    K = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    V = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    M = None if mkind is None else G.new(ggml.F16, n_kv, 1, 1, n_seq)
    scale = 1.0 / math.sqrt(d)
    O = G.lib.ggml_flash_attn_ext(G.ctx, Q, K, V, M, scale, 0.0, 0.0)
    G.build(O)
    G.allocate(gpu.buft)
    G.set(Q, q)
    G.set(K, k.view(np.uint16))
    G.set(V, v.view(np.uint16))
    if M is not None:
        G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    assert "flash_attn_dec" in plan_labels(gpu, G)
    out = G.get(O).reshape(n_seq, 1, hq, d)
    assert np.isfinite(out).all()
    for s in range(n_seq):
        qs = np.ascontiguousarray(q[s].transpose(1, 0, 2))  # [1, hq, d]
        q16 = qs.astype(np.float16).astype(np.float32)
        if M is not None and not (mask[s] == 0).any():
            assert not out[s].any(), "a query with no open position gives zeros"
            continue
        open_ = slice(None) if M is None else (mask[s, 0] == 0)
        ms = None if M is None else mask[s][:, open_]
        exact = attention_f64(q16, k[s][:, open_], v[s][:, open_], ms, scale)
        err = rel_err(out[s], exact)
        print(f"  seq {s}: workgroup form vs f64 {err:.2e}")
        assert err < 2e-3
    first = out.copy()
    for _ in range(2):  # captured, then replayed
        assert G.compute(gpu.backend) == 0
        assert np.array_equal(G.get(O).reshape(first.shape).view(np.uint32), first.view(np.uint32))
    G.free()


# one sequence's decode attention straight into a Q8_0 output projection (+
# residual): the attention's combine writes the projection's quantized
# activations, the one-column projection reads them. Qwen3-0.6B shape at a
# 1024-position arena with 450 live positions and at 4096 positions (64
# chunks); Whisper-tiny self attention (448 positions) and cross attention
# (1500, no mask).
ATTN_PROJ_CASES = [(128, 16, 8, 1024, 450, 1024), (128, 16, 8, 4096, 3000, 1024), (64, 6, 6, 448, 37, 384),
                   (64, 6, 6, 1500, None, 384)]


@pytest.mark.parametrize("prec", ["f32", "default"])
@pytest.mark.parametrize("d,hq,hkv,n_kv,live,m", ATTN_PROJ_CASES)
def test_attention_into_output_projection(ggml, gpu, ref, d, hq, hkv, n_kv, live, m, prec):
    """GGML_PREC_F32: bit for bit the oracle (the exact chunked attention,
    its combine writing the projection's activations); the default
    precision (whichever form is planned -- the workgroup form, quantizing
    its own output, over the 448-position span): within 2e-3 of the
    projection of the oracle's attention"""
    print(f"attention -> o-proj D={d} Hq={hq} Hkv={hkv} kv={n_kv} live={live} M={m} prec={prec}", flush=True)
    k_in = d * hq
    q = RNG.standard_normal((hq, 1, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    wq = ggml.quantize(ggml.Q8_0, ggml.synth_normal(3, 1, m * k_in, 0, 0.02).reshape(m, k_in))
    G = ggml.Graph()
    Q = G.new(ggml.F32, d, 1, hq, 1)
    K = G.new(ggml.F16, d, n_kv, hkv, 1)
    V = G.new(ggml.F16, d, n_kv, hkv, 1)
    M = None if live is None else G.new(ggml.F16, n_kv, 1, 1, 1)
    W = G.new(ggml.Q8_0, k_in, m, weight=True)
    X = G.new(ggml.F32, m, 1)
    O = G.lib.ggml_flash_attn_ext(G.ctx, Q, K, V, M, 1 / math.sqrt(d), 0.0, 0.0)
    if prec == "f32":
        G.lib.ggml_flash_attn_ext_set_prec(O, ggml.GGML_PREC_F32)
    R = G.lib.ggml_reshape_2d(G.ctx, O, k_in, 1)
    Y = G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, W, R), X)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    for it in range(3):  # the same graph again (captured, then replayed) on new inputs
        q = RNG.standard_normal((hq, 1, d)).astype(np.float32)
        x = RNG.standard_normal((1, m)).astype(np.float32)
        mask = np.zeros((1, n_kv), np.float16)
        if live is not None:
            mask[0, live + it:] = -np.inf
        G.set(Q, q)
        G.set(K, k.view(np.uint16))
        G.set(V, v.view(np.uint16))
        G.set(X, x)
        if M is not None:
            G.set(M, mask.view(np.uint16))
        assert G.compute(gpu.backend) == 0
        att = ref.flash_attn(np.ascontiguousarray(q.transpose(1, 0, 2)), k.view(np.uint16), v.view(np.uint16),
                             None if M is None else mask.view(np.uint16), 1 / math.sqrt(d), fidelity=5)
        want = ref.mul_mat(ggml.Q8_0, wq, m, k_in, att.reshape(1, k_in)) + x
        if prec == "f32":
            assert_same_bits(G.get(Y).reshape(1, m), want)
        else:
            assert rel_err(G.get(Y).reshape(1, m), want) < 2e-3
    G.free()


# ------------------------------------------------------------ row ops ---

def test_rms_norm_mul_fused(ggml, gpu, ref):
    x = RNG.standard_normal((8, 1024)).astype(np.float32) * 2
    w = RNG.standard_normal(1024).astype(np.float32)
    G = ggml.Graph()
    X = G.new(ggml.F32, 1024, 8)
    W = G.new(ggml.F32, 1024, weight=True)
    Y = G.lib.ggml_mul(G.ctx, G.lib.ggml_rms_norm(G.ctx, X, 1e-6), W)
    run(ggml, gpu, G, Y)
    G.set(X, x)
    G.set(W, w)
    assert G.compute(gpu.backend) == 0
    assert_same_bits(G.get(Y).reshape(8, 1024), ref.rms_norm(x, 1e-6) * w)
    G.free()


def test_qk_norm_per_head(ggml, gpu, ref):
    """RMSNorm over head_dim of a [128, heads, tokens] view (nn/decoder.rs:1937-1958)"""
    x = RNG.standard_normal((4, 16, 128)).astype(np.float32)
    w = RNG.standard_normal(128).astype(np.float32)
    G = ggml.Graph()
    X = G.new(ggml.F32, 128, 16, 4)
    W = G.new(ggml.F32, 128, weight=True)
    Y = G.lib.ggml_mul(G.ctx, G.lib.ggml_rms_norm(G.ctx, X, 1e-6), W)
    run(ggml, gpu, G, Y)
    G.set(X, x)
    G.set(W, w)
    assert G.compute(gpu.backend) == 0
    assert_same_bits(G.get(Y).reshape(4, 16, 128), ref.rms_norm(x, 1e-6) * w)
    G.free()


def test_layer_norm_affine_fused(ggml, gpu, ref):
    x = RNG.standard_normal((3, 384)).astype(np.float32) * 3 + 1
    w = RNG.standard_normal(384).astype(np.float32)
    b = RNG.standard_normal(384).astype(np.float32)
    G = ggml.Graph()
    X = G.new(ggml.F32, 384, 3)
    W = G.new(ggml.F32, 384, weight=True)
    B = G.new(ggml.F32, 384, weight=True)
    Y = G.lib.ggml_add(G.ctx, G.lib.ggml_mul(G.ctx, G.lib.ggml_norm(G.ctx, X, 1e-5), W), B)
    run(ggml, gpu, G, Y)
    G.set(X, x)
    G.set(W, w)
    G.set(B, b)
    assert G.compute(gpu.backend) == 0
    assert_same_bits(G.get(Y).reshape(3, 384), ref.norm(x, 1e-5) * w + b)
    G.free()


def test_rope_neox_positions(ggml, gpu, ref):
    t, h, d = 8, 16, 128
    x = RNG.standard_normal((t, h, d)).astype(np.float32)
    pos = np.array([0, 1, 5, 374, 383, 900, 1023, 4095], np.int32)
    G = ggml.Graph()
    X = G.new(ggml.F32, d, h, t)
    P = G.new(ggml.I32, t)
    Y = G.lib.ggml_rope_ext(G.ctx, X, P, None, d, 2, 4096, 1e6, 1.0, 0.0, 1.0, 32.0, 1.0)
    run(ggml, gpu, G, Y)
    G.set(X, x)
    G.set(P, pos)
    assert G.compute(gpu.backend) == 0
    # same theta sequence and the same deterministic sin/cos as the oracle
    assert_same_bits(G.get(Y).reshape(t, h, d), ref.rope_neox(x, pos, d, 1e6))
    G.free()


@pytest.mark.parametrize("d,k,ffn", [(384, 384, 1536), (1024, 2048, 1024)])
def test_single_column_epilogues(ggml, gpu, ref, d, k, ffn):
    """batch-1 Q8_0 MUL_MATs with their biases and activations folded into the
    single-column epilogue: LayerNorm(x)·w + b -> MUL_MAT + bias -> GELU, and
    MUL_MAT + bias + residual (two ADDs); bit-exact, no ADD or GELU launches"""
    print(f"single-column epilogues d={d} k={k} ffn={ffn}", flush=True)
    x = (RNG.standard_normal((1, k)) * 1.5).astype(np.float32)
    wn = RNG.standard_normal(k).astype(np.float32)
    bn = RNG.standard_normal(k).astype(np.float32) * 0.1
    b1 = RNG.standard_normal(ffn).astype(np.float32) * 0.1
    b2 = RNG.standard_normal(d).astype(np.float32) * 0.1
    r = RNG.standard_normal((1, d)).astype(np.float32)
    a = RNG.standard_normal((1, k)).astype(np.float32)
    w1 = ggml.quantize(ggml.Q8_0, ggml.synth_normal(31, ffn + k, ffn * k, 0.0, 0.02).reshape(ffn, k))
    w2 = ggml.quantize(ggml.Q8_0, ggml.synth_normal(32, d + k, d * k, 0.0, 0.02).reshape(d, k))
    G = ggml.Graph()
    X = G.new(ggml.F32, k, 1)
    A = G.new(ggml.F32, k, 1)
    R = G.new(ggml.F32, d, 1)
    WN = G.new(ggml.F32, k, weight=True)
    BN = G.new(ggml.F32, k, weight=True)
    B1 = G.new(ggml.F32, ffn, weight=True)
    B2 = G.new(ggml.F32, d, weight=True)
    W1 = G.new(ggml.Q8_0, k, ffn, weight=True)
    W2 = G.new(ggml.Q8_0, k, d, weight=True)
    h = G.lib.ggml_add(G.ctx, G.lib.ggml_mul(G.ctx, G.lib.ggml_norm(G.ctx, X, 1e-5), WN), BN)
    Y = G.lib.ggml_gelu(G.ctx, G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, W1, h), B1))
    Z = G.lib.ggml_add(G.ctx, G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, W2, A), B2), R)
    G.build(Y, Z)
    G.allocate(gpu.buft)
    for T, v in ((X, x), (A, a), (R, r), (WN, wn), (BN, bn), (B1, b1), (B2, b2), (W1, w1), (W2, w2)):
        G.set(T, v)
    assert G.compute(gpu.backend) == 0
    hn = ref.norm(x, 1e-5) * wn + bn
    want_y = ref.gelu(ref.mul_mat(ggml.Q8_0, w1, ffn, k, hn) + b1)
    want_z = (ref.mul_mat(ggml.Q8_0, w2, d, k, a) + b2) + r
    assert_same_bits(G.get(Y).reshape(1, ffn), want_y)
    assert_same_bits(G.get(Z).reshape(1, d), want_z)
    labels = [lab.split(":")[0] for lab, _ in gpu.profile(G.gf, 1)]
    assert "binary" not in labels and "unary" not in labels, labels
    G.free()


def test_single_column_sibling_projections(ggml, gpu, ref):
    """LayerNorm(x)·w + b feeding three Q8_0 MUL_MATs at batch 1 (q and v with
    a bias ADD, k without; Whisper's self-attention projections): one launch,
    bit-exact"""
    d = 384
    x = (RNG.standard_normal((1, d)) * 1.5).astype(np.float32)
    wn = RNG.standard_normal(d).astype(np.float32)
    bn = RNG.standard_normal(d).astype(np.float32) * 0.1
    bq = RNG.standard_normal(d).astype(np.float32) * 0.1
    bv = RNG.standard_normal(d).astype(np.float32) * 0.1
    ws = [ggml.quantize(ggml.Q8_0, ggml.synth_normal(40 + i, d, d * d, 0.0, 0.02).reshape(d, d)) for i in range(3)]
    G = ggml.Graph()
    X = G.new(ggml.F32, d, 1)
    WN, BN, BQ, BV = (G.new(ggml.F32, d, weight=True) for _ in range(4))
    WQ, WK, WV = (G.new(ggml.Q8_0, d, d, weight=True) for _ in range(3))
    h = G.lib.ggml_add(G.ctx, G.lib.ggml_mul(G.ctx, G.lib.ggml_norm(G.ctx, X, 1e-5), WN), BN)
    Q = G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, WQ, h), BQ)
    Kt = G.lib.ggml_mul_mat(G.ctx, WK, h)
    V = G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, WV, h), BV)
    G.build(Q, Kt, V)
    G.allocate(gpu.buft)
    for T, v in ((X, x), (WN, wn), (BN, bn), (BQ, bq), (BV, bv), (WQ, ws[0]), (WK, ws[1]), (WV, ws[2])):
        G.set(T, v)
    assert G.compute(gpu.backend) == 0
    hn = ref.norm(x, 1e-5) * wn + bn
    assert_same_bits(G.get(Q).reshape(1, d), ref.mul_mat(ggml.Q8_0, ws[0], d, d, hn) + bq)
    assert_same_bits(G.get(Kt).reshape(1, d), ref.mul_mat(ggml.Q8_0, ws[1], d, d, hn))
    assert_same_bits(G.get(V).reshape(1, d), ref.mul_mat(ggml.Q8_0, ws[2], d, d, hn) + bv)
    labels = [lab.split(":")[0] for lab, _ in gpu.profile(G.gf, 1)]
    assert sum(lab.startswith("mul_mat") for lab in labels) == 1 and "binary" not in labels, labels
    G.free()


@pytest.mark.parametrize("wt", ["f16", "f32"])
def test_float_sibling_projections(ggml, gpu, wt):
    """three float MUL_MATs of the same columns (an encoder block's q, k, v
    projections over 390 positions; q and v with a bias ADD, k without, row
    counts 128 / 192 / 64): one matrix-core launch, each product within 1e-5
    of an f64 product rounded as the graph does"""
    k, n, ms = 256, 390, (128, 192, 64)
    wdt = np.float16 if wt == "f16" else np.float32
    x = RNG.standard_normal((n, k)).astype(np.float32)
    ws = [(RNG.standard_normal((m, k)) * 0.05).astype(wdt) for m in ms]
    bq = RNG.standard_normal(ms[0]).astype(np.float32)
    bv = RNG.standard_normal(ms[2]).astype(np.float32)
    G = ggml.Graph()
    L = G.lib
    X = G.new(ggml.F32, k, n)
    Ws = [G.new(ggml.F16 if wt == "f16" else ggml.F32, k, m, weight=True) for m in ms]
    BQ, BV = G.new(ggml.F32, ms[0], weight=True), G.new(ggml.F32, ms[2], weight=True)
    Q = L.ggml_add(G.ctx, L.ggml_mul_mat(G.ctx, Ws[0], X), BQ)
    Kt = L.ggml_mul_mat(G.ctx, Ws[1], X)
    V = L.ggml_add(G.ctx, L.ggml_mul_mat(G.ctx, Ws[2], X), BV)
    G.build(Q, Kt, V)
    G.allocate(gpu.buft)
    for T, v in ((X, x), (BQ, bq), (BV, bv)):
        G.set(T, v)
    for T, w in zip(Ws, ws):
        G.set(T, w.view(np.uint16) if wt == "f16" else w)
    assert G.compute(gpu.backend) == 0
    xr = (x.astype(np.float16) if wt == "f16" else x).astype(np.float64)
    want = [(xr @ w.astype(np.float64).T).astype(np.float32) for w in ws]
    assert rel_err(G.get(Q).reshape(n, ms[0]), want[0] + bq) < 1e-5
    assert rel_err(G.get(Kt).reshape(n, ms[1]), want[1]) < 1e-5
    assert rel_err(G.get(V).reshape(n, ms[2]), want[2] + bv) < 1e-5
    labels = [lab.split(":")[0] for lab, _ in gpu.profile(G.gf, 1)]
    assert sum(lab.startswith("mul_mat") for lab in labels) == 1 and "binary" not in labels, labels
    G.free()


@pytest.mark.parametrize("wname", ["q8_0", "q4_K"])
def test_tile_gemm_sibling_projections(ggml, gpu, ref, wname):
    """three quantized MUL_MATs of the same 390 columns (an encoder block's
    q, k, v projections; q and v with a bias ADD, k without; row counts
    128 / 192 / 64): one tile-GEMM launch, bit for bit the oracle"""
    wt = {"q8_0": ggml.Q8_0, "q4_K": ggml.Q4_K}[wname]
    k, n, ms = 512, 390, (128, 192, 64)
    x = RNG.standard_normal((n, k)).astype(np.float32)
    ws = [ggml.quantize(wt, ggml.synth_normal(60 + i, 1, m * k, 0, 0.05).reshape(m, k)) for i, m in enumerate(ms)]
    bq = RNG.standard_normal(ms[0]).astype(np.float32)
    bv = RNG.standard_normal(ms[2]).astype(np.float32)
    G = ggml.Graph()
    L = G.lib
    X = G.new(ggml.F32, k, n)
    Ws = [G.new(wt, k, m, weight=True) for m in ms]
    BQ, BV = G.new(ggml.F32, ms[0], weight=True), G.new(ggml.F32, ms[2], weight=True)
    Q = L.ggml_add(G.ctx, L.ggml_mul_mat(G.ctx, Ws[0], X), BQ)
    Kt = L.ggml_mul_mat(G.ctx, Ws[1], X)
    V = L.ggml_add(G.ctx, L.ggml_mul_mat(G.ctx, Ws[2], X), BV)
    G.build(Q, Kt, V)
    G.allocate(gpu.buft)
    for T, v in [(X, x), (BQ, bq), (BV, bv)] + list(zip(Ws, ws)):
        G.set(T, v)
    assert G.compute(gpu.backend) == 0
    assert_same_bits(G.get(Q).reshape(n, ms[0]), ref.mul_mat(wt, ws[0], ms[0], k, x) + bq)
    assert_same_bits(G.get(Kt).reshape(n, ms[1]), ref.mul_mat(wt, ws[1], ms[1], k, x))
    assert_same_bits(G.get(V).reshape(n, ms[2]), ref.mul_mat(wt, ws[2], ms[2], k, x) + bv)
    labels = [lab.split(":")[0] for lab, _ in gpu.profile(G.gf, 1)]
    assert sum(lab.startswith("mul_mat") for lab in labels) == 1 and "binary" not in labels, labels
    G.free()


def test_silu_mul_and_gelu(ggml, gpu, ref):
    g = RNG.standard_normal((4, 3072)).astype(np.float32) * 3
    u = RNG.standard_normal((4, 3072)).astype(np.float32)
    G = ggml.Graph()
    Gt = G.new(ggml.F32, 3072, 4)
    U = G.new(ggml.F32, 3072, 4)
    Y = G.lib.ggml_mul(G.ctx, G.lib.ggml_silu(G.ctx, Gt), U)
    Z = G.lib.ggml_gelu(G.ctx, U)
    G.build(Y, Z)
    G.allocate(gpu.buft)
    G.set(Gt, g)
    G.set(U, u)
    assert G.compute(gpu.backend) == 0
    assert_same_bits(G.get(Y).reshape(4, 3072), ref.silu(g) * u)
    assert np.array_equal(G.get(Z).reshape(4, 3072), ref.gelu(u))  # same f16 table: bit exact
    G.free()


def test_relu_and_gelu_erf(ggml, gpu, ref):
    """RELU and GELU_ERF (erf by the fixed double series both sides run) bit
    for bit, over the range where erf bends and past its +-4 saturation"""
    x = np.concatenate([np.linspace(-9, 9, 4096), RNG.standard_normal(4096) * 3]).astype(np.float32).reshape(2, 4096)
    G = ggml.Graph()
    X = G.new(ggml.F32, 4096, 2)
    R = G.lib.ggml_relu(G.ctx, X)
    E = G.lib.ggml_gelu_erf(G.ctx, X)
    G.build(R, E)
    G.allocate(gpu.buft)
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    L = ref.lib()
    want_e = np.array([L.ref_gelu_erf(float(v)) for v in x.reshape(-1)], np.float32).reshape(2, 4096)
    assert np.array_equal(G.get(R).reshape(2, 4096), np.maximum(x, 0))
    assert np.array_equal(G.get(E).reshape(2, 4096).view(np.uint32), want_e.view(np.uint32))
    G.free()


def test_set_rows_batched_kv_write(ggml, gpu):
    """f32 -> f16 rows into a [128, maxpos, 8, n_seq] cache at per-sequence rows"""
    d, maxpos, hkv, n_seq = 128, 64, 8, 4
    cache = RNG.standard_normal((n_seq, hkv, maxpos, d)).astype(np.float16)
    src = RNG.standard_normal((n_seq, hkv, 1, d)).astype(np.float32)
    rows = np.array([3, 0, 63, 17], np.int32)
    G = ggml.Graph()
    Cc = G.new(ggml.F16, d, maxpos, hkv, n_seq)
    S = G.new(ggml.F32, d, 1, hkv, n_seq)
    I = G.new(ggml.I32, 1, 1, n_seq, 1)
    R = G.lib.ggml_set_rows(G.ctx, Cc, S, I)
    run(ggml, gpu, G, R)
    G.set(Cc, cache.view(np.uint16))
    G.set(S, src)
    G.set(I, rows)
    assert G.compute(gpu.backend) == 0
    got = G.get(Cc, np.uint16).reshape(n_seq, hkv, maxpos, d)
    want = cache.copy()
    for s in range(n_seq):
        want[s, :, rows[s], :] = src[s, :, 0, :].astype(np.float16)
    assert np.array_equal(got, want.view(np.uint16))
    G.free()


@pytest.mark.parametrize("wname", ["q8_0", "q4_K", "f32"])
def test_get_rows_dequant(ggml, gpu, ref, wname):
    rows, k = 300, 1024
    w = ggml.synth_normal(3, 4, rows * k, 0.0, 0.02).reshape(rows, k)
    ids = np.array([0, 299, 17, 17, 150], np.int32)
    G = ggml.Graph()
    if wname == "f32":
        W = G.new(ggml.F32, k, rows, weight=True)
        data, want = w, w[ids]
    else:
        t = ggml.Q8_0 if wname == "q8_0" else ggml.Q4_K
        W = G.new(t, k, rows, weight=True)
        data = ggml.quantize(t, w)
        want = ref.dequantize(t, data, rows * k).reshape(rows, k)[ids]
    I = G.new(ggml.I32, len(ids))
    Y = G.lib.ggml_get_rows(G.ctx, W, I)
    run(ggml, gpu, G, Y)
    G.set(W, data)
    G.set(I, ids)
    assert G.compute(gpu.backend) == 0
    assert np.array_equal(G.get(Y).reshape(len(ids), k), want)
    G.free()


def test_soft_max_argmax_cpy_cont(ggml, gpu, ref):
    x = RNG.standard_normal((6, 333)).astype(np.float32)
    x[2, 10] = x[2, 200] = 9.0  # tie
    mask = np.zeros((6, 333), np.float16)
    mask[:, 300:] = -np.inf
    G = ggml.Graph()
    X = G.new(ggml.F32, 333, 6)
    M = G.new(ggml.F16, 333, 6)
    S = G.lib.ggml_soft_max_ext(G.ctx, X, M, 0.7, 0.0)
    A = G.lib.ggml_argmax(G.ctx, X)
    A1 = G.lib.ggml_argmax_first(G.ctx, X)
    H = G.new(ggml.F16, 333, 6)
    Cp = G.lib.ggml_cpy(G.ctx, X, H)
    Tc = G.lib.ggml_cont(G.ctx, G.lib.ggml_transpose(G.ctx, X))
    G.build(S, A, A1, Cp, Tc)
    G.allocate(gpu.buft)
    G.set(X, x)
    G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    assert_same_bits(G.get(S).reshape(6, 333), ref.soft_max_ext(x, mask.view(np.uint16), 0.7))
    a_last, a_first = G.get(A).reshape(-1), G.get(A1).reshape(-1)
    assert list(a_last) == [ref.argmax_last(r) for r in x]
    assert list(a_first) == [ref.argmax_first(r) for r in x]
    assert a_last[2] == 200 and a_first[2] == 10
    assert np.array_equal(G.get(H, np.uint16).reshape(6, 333), x.astype(np.float16).view(np.uint16))
    assert np.array_equal(G.get(Tc).reshape(333, 6), x.T)
    G.free()


def test_abort_callback_and_graph_replay(ggml, gpu, ref):
    """same graph computed repeatedly: eager, captured, replayed -- identical
    results every time; an abort callback that fires stops the compute with
    GGML_STATUS_ABORTED and reports native cancellation"""
    import ctypes as C
    m, k = 1024, 1024
    wq = ggml.quantize(ggml.Q8_0, ggml.synth_normal(1, 1, m * k, 0, 0.02).reshape(m, k))
    G = ggml.Graph()
    W = G.new(ggml.Q8_0, k, m, weight=True)
    X = G.new(ggml.F32, k, 1)
    Y = G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, W, X), X)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    outs = []
    for it in range(5):
        x = RNG.standard_normal((1, k)).astype(np.float32)
        G.set(X, x)
        assert G.compute(gpu.backend) == 0
        y = G.get(Y).reshape(1, m)
        assert_same_bits(y, ref.mul_mat(ggml.Q8_0, wq, m, k, x) + x)
        outs.append(y)
    CB = C.CFUNCTYPE(C.c_bool, C.c_void_p)
    always = CB(lambda _: True)
    cap = ggml.cancel_capability()
    st = G.lib.ggml_backend_graph_compute_with_abort(gpu.backend, G.gf, C.cast(always, C.c_void_p), None,
                                                     C.byref(cap))
    assert st == 1 and cap.mechanism == 1
    never = CB(lambda _: False)
    st = G.lib.ggml_backend_graph_compute_with_abort(gpu.backend, G.gf, C.cast(never, C.c_void_p), None,
                                                     C.byref(cap))
    assert st == 0 and cap.mechanism == 1 and cap.observation_granularity == 1
    G.free()


IM2COL_CASES = [
    # ic, ih, iw, n, kh, kw, s0, s1, p0, p1, d0, d1, f16
    (1, 128, 100, 1, 3, 3, 2, 2, 1, 1, 1, 1, True),  # encoder stem conv1 over a 128-bin mel chunk
    (64, 64, 50, 1, 3, 3, 2, 2, 1, 1, 1, 1, True),  # conv2-shaped, fewer channels
    (3, 9, 11, 2, 2, 3, 1, 2, 2, 0, 2, 1, False),  # every parameter different per axis
    (4, 9, 11, 2, 2, 3, 1, 2, 2, 0, 2, 1, False),  # K % 4 == 0: four-element runs crossing channels
    (5, 7, 6, 3, 2, 2, 2, 1, 1, 1, 1, 2, True),  # K % 4 == 0, f16 columns, three images
]


@pytest.mark.gpu
@pytest.mark.parametrize("ic,ih,iw,n,kh,kw,s0,s1,p0,p1,d0,d1,f16", IM2COL_CASES)
def test_im2col(ggml, gpu, ref, ic, ih, iw, n, kh, kw, s0, s1, p0, p1, d0, d1, f16):
    x = RNG.standard_normal((n, ic, ih, iw)).astype(np.float32)
    G = ggml.Graph()
    Kt = G.new(ggml.F16 if f16 else ggml.F32, kw, kh, ic, 8)
    X = G.new(ggml.F32, iw, ih, ic, n)
    T = G.lib.ggml_im2col(G.ctx, Kt, X, s0, s1, p0, p1, d0, d1, True, ggml.F16 if f16 else ggml.F32)
    G.build(T)
    G.allocate(gpu.buft)
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    want = ref.im2col(x, kw, kh, s0, s1, p0, p1, d0, d1)
    if f16:
        got = G.get(T, np.uint16).reshape(want.shape)
        assert np.array_equal(got, want.astype(np.float16).view(np.uint16))
    else:
        assert np.array_equal(G.get(T).reshape(want.shape).view(np.uint32), want.view(np.uint32))
    G.free()


@pytest.mark.gpu
def test_im2col_1d(ggml, gpu, ref):
    x = RNG.standard_normal((3, 4, 50)).astype(np.float32)
    G = ggml.Graph()
    Kt = G.new(ggml.F16, 3, 4, 8)
    X = G.new(ggml.F32, 50, 4, 3)
    T = G.lib.ggml_im2col(G.ctx, Kt, X, 2, 0, 1, 0, 1, 0, False, ggml.F16)
    G.build(T)
    G.allocate(gpu.buft)
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    want = ref.im2col(x, 3, 0, 2, 0, 1, 0, 1, 0, is_2d=False)
    assert np.array_equal(G.get(T, np.uint16).reshape(want.shape), want.astype(np.float16).view(np.uint16))
    G.free()


@pytest.mark.gpu
def test_conv_2d_f32_kernel_chain(ggml, gpu, ref):
    """ggml_conv_2d with an f32 kernel as nn/conv.rs:82-110 builds it: IM2COL
    -> MUL_MAT(columns, kernel rows) -> reshape/permute/cont to [OW, OH, OC, N],
    against an f64 convolution"""
    n, ic, ih, iw, oc = 1, 4, 30, 26, 16
    x = RNG.standard_normal((n, ic, ih, iw)).astype(np.float32)
    w = RNG.standard_normal((oc, ic, 3, 3)).astype(np.float32)
    G = ggml.Graph()
    Kt = G.new(ggml.F32, 3, 3, ic, oc)
    X = G.new(ggml.F32, iw, ih, ic, n)
    cols = G.lib.ggml_im2col(G.ctx, Kt, X, 2, 2, 1, 1, 1, 1, True, ggml.F32)
    ct = ggml.tensor(cols)
    kdim, ow, oh = ct.ne[0], ct.ne[1], ct.ne[2]
    mm = G.lib.ggml_mul_mat(G.ctx, G.lib.ggml_reshape_2d(G.ctx, cols, kdim, ow * oh * n),
                            G.lib.ggml_reshape_2d(G.ctx, Kt, kdim, oc))
    y = G.lib.ggml_cont(G.ctx, G.lib.ggml_permute(G.ctx, G.lib.ggml_reshape_4d(G.ctx, mm, ow, oh, n, oc), 0, 1, 3, 2))
    G.build(y)
    G.allocate(gpu.buft)
    G.set(X, x)
    G.set(Kt, w)
    assert G.compute(gpu.backend) == 0
    cols_ref = ref.im2col(x, 3, 3, 2, 2, 1, 1, 1, 1).astype(np.float64)
    want = (cols_ref @ w.reshape(oc, -1).T.astype(np.float64)).transpose(0, 3, 1, 2)  # [N, OC, OH, OW]
    got = G.get(y).reshape(n, oc, oh, ow)
    assert rel_err(got, want) <= 2e-3
    G.free()


@pytest.mark.parametrize("wt,residual", [("f16", True), ("f32", True), ("f16", False)])
def test_float_mul_mat_bias_residual_epilogue(ggml, gpu, wt, residual):
    """the encoders' linear layers (nn/encoder.rs:655-671) and residual ADD:
    MUL_MAT -> ADD(bias row) -> ADD(residual) in one launch, with the f32
    roundings of the three ops (within 1e-5 of an f64 product rounded as
    the graph does); the intermediate nodes are never written"""
    m, k, n = 200, 384, 90
    wdt = np.float16 if wt == "f16" else np.float32
    w = (RNG.standard_normal((m, k)) * 0.05).astype(wdt)
    x = RNG.standard_normal((n, k)).astype(np.float32)
    b = RNG.standard_normal(m).astype(np.float32)
    r = RNG.standard_normal((n, m)).astype(np.float32)
    G = ggml.Graph()
    L = G.lib
    W = G.new(ggml.F16 if wt == "f16" else ggml.F32, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    B = G.new(ggml.F32, m, weight=True)
    R = G.new(ggml.F32, m, n)
    Y = L.ggml_add(G.ctx, L.ggml_mul_mat(G.ctx, W, X), B)
    if residual:
        Y = L.ggml_add(G.ctx, Y, R)
    run(ggml, gpu, G, Y)
    G.set(W, w.view(np.uint16) if wt == "f16" else w)
    G.set(X, x)
    G.set(B, b)
    if residual:
        G.set(R, r)  # not part of the graph otherwise
    assert G.compute(gpu.backend) == 0
    xr = x.astype(np.float16) if wt == "f16" else x
    want = (xr.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32) + b
    if residual:
        want = want + r
    assert rel_err(G.get(Y).reshape(n, m), want) < 1e-5
    G.free()


@pytest.mark.parametrize("wt,m,k,n", [("f16", 896, 3584, 390), ("f32", 256, 1000, 100), ("f16", 64, 4096, 16)])
def test_float_mul_mat_split_k(ggml, gpu, ref, wt, m, k, n):
    """float MUL_MAT with too few 64 x 64 tiles to fill the CUs (the audio
    encoder's 896-row projections over 390 positions) splits K over
    workgroups, a second launch adding the splits in order before the bias
    ADD and GELU_ERF of the epilogue: within 1e-5 of an f64 product rounded
    as the graph does (K = 1000 leaves a short last split)"""
    print(f"float mul_mat split K {wt} M={m} K={k} N={n}", flush=True)
    wdt = np.float16 if wt == "f16" else np.float32
    w = (RNG.standard_normal((m, k)) * 0.03).astype(wdt)
    x = RNG.standard_normal((n, k)).astype(np.float32)
    b = RNG.standard_normal(m).astype(np.float32)
    G = ggml.Graph()
    L = G.lib
    W = G.new(ggml.F16 if wt == "f16" else ggml.F32, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    B = G.new(ggml.F32, m, weight=True)
    Y = L.ggml_gelu_erf(G.ctx, L.ggml_add(G.ctx, L.ggml_mul_mat(G.ctx, W, X), B))
    run(ggml, gpu, G, Y)
    G.set(W, w.view(np.uint16) if wt == "f16" else w)
    G.set(X, x)
    G.set(B, b)
    assert G.compute(gpu.backend) == 0
    xr = x.astype(np.float16) if wt == "f16" else x
    pre = (xr.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32) + b
    want = np.vectorize(lambda v: ref.lib().ref_gelu_erf(float(v)), otypes=[np.float32])(pre)
    assert rel_err(G.get(Y).reshape(n, m), want) < 1e-5
    G.free()


@pytest.mark.parametrize("wname,tail", [("q8_0", "bias_res"), ("q4_K", "bias_res"), ("q8_0", "bias_gelu"),
                                        ("q4_K", "res"), ("q8_0", "gelu")])
def test_tile_gemm_epilogue(ggml, gpu, ref, wname, tail):
    """the quantized tile GEMM (N > 64: prefill, the audio encoder's
    projections) with what follows it folded into its epilogue -- a bias ADD
    (a row), a residual ADD (the output's shape), GELU_ERF -- bit for bit the
    oracle's MUL_MAT and the separate ops' f32 roundings"""
    wt = {"q8_0": ggml.Q8_0, "q4_K": ggml.Q4_K}[wname]
    m, k, n = 320, 512, 150
    wq = ggml.quantize(wt, ggml.synth_normal(5, 1, m * k, 0, 0.05).reshape(m, k))
    x = RNG.standard_normal((n, k)).astype(np.float32)
    b = RNG.standard_normal(m).astype(np.float32)
    r = RNG.standard_normal((n, m)).astype(np.float32)
    G = ggml.Graph()
    L = G.lib
    W = G.new(wt, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    B = G.new(ggml.F32, m, weight=True)
    R = G.new(ggml.F32, m, n)
    Y = L.ggml_mul_mat(G.ctx, W, X)
    want = ref.mul_mat(wt, wq, m, k, x)
    if "bias" in tail:
        Y = L.ggml_add(G.ctx, Y, B)
        want = want + b
    if "res" in tail:
        Y = L.ggml_add(G.ctx, R, Y)
        want = r + want
    if "gelu" in tail:
        Y = L.ggml_gelu_erf(G.ctx, Y)
        want = np.vectorize(lambda v: ref.lib().ref_gelu_erf(float(v)), otypes=[np.float32])(want)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    G.set(X, x)
    if "bias" in tail:
        G.set(B, b)
    if "res" in tail:
        G.set(R, r)
    assert G.compute(gpu.backend) == 0
    assert_same_bits(G.get(Y).reshape(n, m), want)
    G.free()


def test_conv_2d_f16_kernel(ggml, gpu, ref):
    """ggml_conv_2d with an f16 kernel (the Qwen audio encoder's conv stem,
    models/qwen/audio_encoder.rs:520-550): f16 columns x f16 kernel rows on
    the matrix-core GEMM, against an f64 convolution of the f16-rounded input
    (f32 sums: within 1e-4 of the largest output)"""
    n, ic, ih, iw, oc = 2, 8, 40, 24, 32
    x = RNG.standard_normal((n, ic, ih, iw)).astype(np.float32)
    w = (RNG.standard_normal((oc, ic, 3, 3)) * 0.2).astype(np.float16)
    G = ggml.Graph()
    Kt = G.new(ggml.F16, 3, 3, ic, oc, weight=True)
    X = G.new(ggml.F32, iw, ih, ic, n)
    y = G.lib.ggml_conv_2d(G.ctx, Kt, X, 2, 2, 1, 1, 1, 1)
    yt = ggml.tensor(y)
    ow, oh = yt.ne[0], yt.ne[1]
    assert (yt.ne[2], yt.ne[3]) == (oc, n)
    run(ggml, gpu, G, y)
    G.set(X, x)
    G.set(Kt, w.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    cols_ref = ref.im2col(x.astype(np.float16).astype(np.float32), 3, 3, 2, 2, 1, 1, 1, 1).astype(np.float64)
    want = (cols_ref @ w.reshape(oc, -1).T.astype(np.float64)).transpose(0, 3, 1, 2)  # [N, OC, OH, OW]
    got = G.get(y).reshape(n, oc, oh, ow)
    assert rel_err(got, want) < 1e-4
    G.free()


@pytest.mark.parametrize("ic,tail", [(1, "bias_gelu"), (16, "bias_gelu"), (16, "bias"), (16, "gelu"), (16, "")])
def test_conv_2d_tail_in_the_gemm(ggml, gpu, ref, ic, tail):
    """an f32-kernel ggml_conv_2d followed by the conv stem's bias ADD (one
    value a channel) and GELU_ERF (models/qwen/audio_encoder.rs:520-552):
    the column GEMM writes the permuted layout itself with the bias and GELU
    in its epilogue; against an f64 convolution, then the same f32 bias add
    and the oracle's GELU_ERF (f32 sums: within 1e-5 of the largest output)"""
    n, ih, iw, oc = 3, 32, 20, 24
    x = RNG.standard_normal((n, ic, ih, iw)).astype(np.float32)
    w = (RNG.standard_normal((oc, ic, 3, 3)) * 0.2).astype(np.float32)
    b = RNG.standard_normal(oc).astype(np.float32)
    G = ggml.Graph()
    Kt = G.new(ggml.F32, 3, 3, ic, oc, weight=True)
    X = G.new(ggml.F32, iw, ih, ic, n)
    B = G.new(ggml.F32, 1, 1, oc, weight=True)
    y = G.lib.ggml_conv_2d(G.ctx, Kt, X, 2, 2, 1, 1, 1, 1)
    yt = ggml.tensor(y)
    ow, oh = yt.ne[0], yt.ne[1]
    if "bias" in tail:
        y = G.lib.ggml_add(G.ctx, y, B)
    if "gelu" in tail:
        y = G.lib.ggml_gelu_erf(G.ctx, y)
    run(ggml, gpu, G, y)
    G.set(X, x)
    G.set(Kt, w)
    if "bias" in tail:
        G.set(B, b)
    assert G.compute(gpu.backend) == 0
    cols_ref = ref.im2col(x, 3, 3, 2, 2, 1, 1, 1, 1).astype(np.float64)
    want = (cols_ref @ w.reshape(oc, -1).T.astype(np.float64)).astype(np.float32).transpose(0, 3, 1, 2)
    if "bias" in tail:
        want = want + b[None, :, None, None]
    if "gelu" in tail:
        want = np.vectorize(lambda v: ref.lib().ref_gelu_erf(float(v)), otypes=[np.float32])(want)
    got = G.get(y).reshape(n, oc, oh, ow)
    assert rel_err(got, want) < 1e-5
    G.free()


def test_sinusoidal_position_table(ggml, gpu, ref):
    """the encoders' sinusoidal positions (nn/encoder.rs:575-590): angles =
    MUL_MAT(inverse timescales [1, half], positions [1, T]), SIN and COS of
    them, CONCAT along dim 0 (half-split layout); SIN / COS are the
    deterministic sincos both sides run (bit for bit), the angles an exact
    f32 product (K = 1), CONCAT a copy; and a CAST of the table to f16"""
    half, t = 64, 300
    inv = np.exp(-np.log(10000.0) * np.arange(half) / (half - 1)).astype(np.float32)
    pos = np.arange(t, dtype=np.float32)
    G = ggml.Graph()
    L = G.lib
    Inv = G.new(ggml.F32, 1, half, weight=True)
    Pos = G.new(ggml.F32, 1, t)
    ang = L.ggml_mul_mat(G.ctx, Inv, Pos)  # [half, t]
    table = L.ggml_concat(G.ctx, L.ggml_sin(G.ctx, ang), L.ggml_cos(G.ctx, ang), 0)  # [2 half, t]
    t16 = L.ggml_cast(G.ctx, table, ggml.F16)
    run(ggml, gpu, G, t16)
    G.set(Inv, inv)
    G.set(Pos, pos)
    assert G.compute(gpu.backend) == 0
    a = (pos[:, None] * inv[None, :]).astype(np.float32)  # [t, half], one exact-rounded product each
    s = np.zeros_like(a)
    c = np.zeros_like(a)
    fs, fc = ctypes.c_float(), ctypes.c_float()
    for idx, v in np.ndenumerate(a):
        ref.lib().ref_sincosf_det(float(v), ctypes.byref(fs), ctypes.byref(fc))
        s[idx], c[idx] = fs.value, fc.value
    want = np.concatenate([s, c], axis=1)  # [t, 2 half]
    got = G.get(table).reshape(t, 2 * half)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(G.get(t16).reshape(t, 2 * half).view(np.uint16), want.astype(np.float16).view(np.uint16))
    G.free()


@pytest.mark.parametrize("dim", [0, 1, 2, 3])
def test_concat_every_dim(ggml, gpu, dim):
    """CONCAT along each dim, f32 and of a permuted (strided) second operand"""
    shape_a = [6, 5, 4, 3]
    shape_b = list(shape_a)
    shape_b[dim] = 2
    a = RNG.standard_normal(shape_a[::-1]).astype(np.float32)
    b = RNG.standard_normal(shape_b[::-1]).astype(np.float32)
    G = ggml.Graph()
    A = G.new(ggml.F32, *shape_a)
    B = G.new(ggml.F32, *shape_b)
    C = G.lib.ggml_concat(G.ctx, A, B, dim)
    run(ggml, gpu, G, C)
    G.set(A, a)
    G.set(B, b)
    assert G.compute(gpu.backend) == 0
    want = np.concatenate([a, b], axis=3 - dim)
    assert np.array_equal(G.get(C).reshape(want.shape), want)
    G.free()


def test_refused_launch_fails_closed(ggml, gpu, ref):
    """A launch refused on the host (the plugin's test seam plays a launcher
    that refuses a shape) fails the compute with GGML_STATUS_FAILED -- in the
    eager first compute and in the compute that captures the HIP graph -- and
    no graph missing that launch is ever replayed: the computes after it
    capture again and give the right result."""
    import ctypes as C
    refuse = gpu.cdll.ggml_backend_mi355x_refuse_next_launch
    refuse.restype, refuse.argtypes = None, [C.c_void_p]
    m, k = 1024, 1024
    wq = ggml.quantize(ggml.Q8_0, ggml.synth_normal(3, 1, m * k, 0, 0.02).reshape(m, k))
    G = ggml.Graph()
    W = G.new(ggml.Q8_0, k, m, weight=True)
    X = G.new(ggml.F32, k, 1)
    Y = G.lib.ggml_add(G.ctx, G.lib.ggml_mul_mat(G.ctx, W, X), X)
    run(ggml, gpu, G, Y)
    G.set(W, wq)
    statuses = []
    for it in range(6):
        x = RNG.standard_normal((1, k)).astype(np.float32)
        G.set(X, x)
        G.set(Y, np.full((1, m), np.nan, np.float32))
        if it in (0, 1, 4):  # eager, capturing, and a compute after a graph was cached
            refuse(gpu.backend)
        st = G.compute(gpu.backend)
        statuses.append(st)
        y = G.get(Y).reshape(1, m)
        if st == 0:
            assert_same_bits(y, ref.mul_mat(ggml.Q8_0, wq, m, k, x) + x)
    assert statuses == [-1, -1, 0, 0, -1, 0], statuses
    G.free()


def test_failed_transfer_fails_next_compute(ggml, gpu):
    """A tensor transfer the plugin refuses (a Q8_0 tensor whose rows are not
    packed) is not lost: the next graph_compute on the device fails with
    GGML_STATUS_EXECUTION_FAILED instead of running on what the transfer
    failed to write, and the compute after that succeeds."""
    G = ggml.Graph()
    W = G.new(ggml.Q8_0, 64, 4, weight=True)
    X = G.new(ggml.F32, 64, 1)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    run(ggml, gpu, G, Y)
    # a view of W whose rows are 34 bytes wider than packed: set_tensor refuses it
    V = G.lib.ggml_view_2d(G.wctx, W, 32, 2, 2 * 34, 0)
    G.lib.ggml_backend_tensor_set(V, np.zeros(4 * 34 // 2, np.uint8).ctypes.data, 0, 2 * 34)
    G.set(X, np.ones((1, 64), np.float32))
    assert G.compute(gpu.backend) == 2
    assert G.compute(gpu.backend) == 0
    G.free()


def test_staged_uploads_keep_write_order(ggml, gpu):
    """Small tensor writes wait in pinned host memory and land at the next
    device use. Overlapping partial writes land in call order, a read sees
    every write before it, more writes than one apply launch takes all land
    (4-byte pieces at 4-byte offsets: the unaligned path), a write too large
    to stage lands after the staged ones before it, and a compute sees the
    writes queued just before it, and writes larger than one apply
    workgroup's piece land whole."""
    G = ggml.Graph()
    L = G.lib
    n = 131072  # 512 KB: a whole-tensor write takes the synchronous path
    X = G.new(ggml.F32, n)
    Y = L.ggml_scale(G.ctx, X, 2.0)
    run(ggml, gpu, G, Y)

    def put(arr, elem_off):
        arr = np.ascontiguousarray(arr, np.float32)
        assert L.ggml_backend_tensor_set(X, arr.ctypes.data, 4 * elem_off, arr.nbytes) == 0

    base = RNG.standard_normal(n).astype(np.float32)
    G.set(X, base)
    want = base.copy()
    put(np.full(100, 7.0), 100)
    put(np.full(50, -3.0), 150)
    want[100:200] = 7.0
    want[150:200] = -3.0
    assert np.array_equal(G.get(X).reshape(-1), want)
    for i in range(100):
        put([1000.0 + i], 1000 + 3 * i)
        want[1000 + 3 * i] = 1000.0 + i
    assert G.compute(gpu.backend) == 0
    assert np.array_equal(G.get(Y).reshape(-1), want * 2.0)
    # staged, then a synchronous whole-tensor write: the large one wins
    put(np.full(64, 5.0), 0)
    big = RNG.standard_normal(n).astype(np.float32)
    G.set(X, big)
    assert np.array_equal(G.get(X).reshape(-1), big)
    # staged writes right before a compute
    put(np.full(16, 9.0), 4096)
    big[4096:4112] = 9.0
    assert G.compute(gpu.backend) == 0
    assert np.array_equal(G.get(Y).reshape(-1), big * 2.0)
    # writes that span several apply workgroups in one launch: 100 KB aligned
    # (16-byte pieces), 9996 bytes at a 4-byte offset (the byte path), and a
    # one-piece write between them
    for arr, off in ((RNG.standard_normal(25600), 8192), (np.full(4, 3.0), 36000),
                     (RNG.standard_normal(2499), 40001)):
        put(arr, off)
        big[off:off + len(arr)] = arr
    assert G.compute(gpu.backend) == 0
    assert np.array_equal(G.get(Y).reshape(-1), big * 2.0)
    # a staged write into a buffer that is then freed
    put(np.full(8, 1.0), 0)
    G.free()


@pytest.mark.parametrize("n", [1, 3])
def test_reversed_row_top1_keeps_the_first_max(ggml, gpu, n):
    """the reversed-row top-1 graph (cpu_graph.rs:3772-3810) on logits with
    exact ties: GET_ROWS by V - 1 .. 0 (a one-element row per logit for one
    column, rows of the transposed matrix otherwise), CONT, ggml's last-max
    ARGMAX, then V - 1 - r is the FIRST of the equal maxima; plain ARGMAX on
    the same logits gives the last"""
    V = 151936
    G = ggml.Graph()
    L = G.lib
    X = G.new(ggml.F32, V, n)
    R = G.new(ggml.I32, V)
    if n == 1:
        r = L.ggml_get_rows(G.ctx, L.ggml_reshape_2d(G.ctx, X, 1, V), R)
        r = L.ggml_reshape_2d(G.ctx, L.ggml_cont(G.ctx, r), V, 1)
    else:
        tr = L.ggml_cont(G.ctx, L.ggml_transpose(G.ctx, X))
        r = L.ggml_cont(G.ctx, L.ggml_transpose(G.ctx, L.ggml_get_rows(G.ctx, tr, R)))
    top = L.ggml_argmax(G.ctx, r)
    last = L.ggml_argmax(G.ctx, X)
    G.build(top, last)
    G.allocate(gpu.buft)
    x = RNG.standard_normal((n, V)).astype(np.float32)
    firsts = []
    for c in range(n):
        idx = np.sort(RNG.choice(V, 4, replace=False))
        x[c, idx] = 9.0  # four equal maxima
        firsts.append(idx)
    G.set(X, x)
    G.set(R, np.arange(V - 1, -1, -1, dtype=np.int32))
    assert G.compute(gpu.backend) == 0
    got = G.get(top, np.int32).reshape(-1)
    got_last = G.get(last, np.int32).reshape(-1)
    for c in range(n):
        assert V - 1 - got[c] == firsts[c][0]
        assert got_last[c] == firsts[c][-1]
    G.free()


@pytest.mark.parametrize("n_q,n_seq", [(1, 2), (8, 1)])
def test_naive_masked_attention_chain(ggml, gpu, ref, n_q, n_seq):
    """the unfused attention the host emits with flash attention off
    (nn/decoder.rs:2147-2200): scores = MUL_MAT(K f16 [128, kv, 8, s],
    Q f32 [128, n_q, 16, s]) with the GQA broadcast of MUL_MAT's batch dims,
    SOFT_MAX_EXT(mask [kv, n_q, 1, s], scale), V^T by CONT(TRANSPOSE), the
    context MUL_MAT, then PERMUTE(0, 2, 1, 3) + CONT. Checked against the
    oracle's ops composed slice by slice (f16 rows x f16-rounded activations,
    summed in f64) within 2e-3, and against the flash_attn_ext result"""
    d, hq, hkv, n_kv = 128, 16, 8, 512
    print(f"naive attention chain n_q={n_q} n_seq={n_seq}", flush=True)
    q = RNG.standard_normal((n_seq, hq, n_q, d)).astype(np.float32)
    k = RNG.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((n_seq, hkv, n_kv, d)).astype(np.float16)
    valid = [n_kv - 37 * s for s in range(n_seq)]
    mask = np.full((n_seq, n_q, n_kv), -np.inf, np.float16)
    for s in range(n_seq):
        for i in range(n_q):
            mask[s, i, :valid[s] - n_q + i + 1] = 0
    scale = 1.0 / math.sqrt(d)
    G = ggml.Graph()
    L = G.lib
    Q = G.new(ggml.F32, d, n_q, hq, n_seq)
    K = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    V = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    M = G.new(ggml.F16, n_kv, n_q, 1, n_seq)
    scores = L.ggml_mul_mat(G.ctx, K, Q)
    probs = L.ggml_soft_max_ext(G.ctx, scores, M, scale, 0.0)
    vt = L.ggml_cont(G.ctx, L.ggml_transpose(G.ctx, V))
    att = L.ggml_cont(G.ctx, L.ggml_permute(G.ctx, L.ggml_mul_mat(G.ctx, vt, probs), 0, 2, 1, 3))
    FA = L.ggml_flash_attn_ext(G.ctx, Q, K, V, M, scale, 0.0, 0.0)
    G.build(att, FA)
    G.allocate(gpu.buft)
    G.set(Q, q)
    G.set(K, k.view(np.uint16))
    G.set(V, v.view(np.uint16))
    G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    got = G.get(att).reshape(n_seq, n_q, hq, d)
    fa = G.get(FA).reshape(n_seq, n_q, hq, d)
    g = hq // hkv
    for s in range(n_seq):
        for h in range(hq):
            kh, vh = k[s, h // g], v[s, h // g]
            sc = ref.mul_mat(ref.F16, kh.view(np.uint16), n_kv, d, q[s, h])           # [n_q, n_kv]
            p = ref.soft_max_ext(sc, mask[s].view(np.uint16), scale)
            ctx = ref.mul_mat(ref.F16, np.ascontiguousarray(vh.T).view(np.uint16), d, n_kv, p)  # [n_q, d]
            assert rel_err(got[s, :, h], ctx) < 2e-3, (s, h)
    assert rel_err(got, fa) < 2e-3
    G.free()


# ------------------------------------------- the HIP lane's GQA expansion --

def hip_lane_kv(L, G, K, V, d, n_kv, hq, hkv):
    """expand_attention_kv (nn/decoder.rs:1799-1841): RESHAPE [d, kv, 1, hkv],
    REPEAT [d, kv, g, hkv], RESHAPE [d, kv, hq]"""
    g = hq // hkv
    out = []
    for X in (K, V):
        X = L.ggml_reshape_4d(G.ctx, X, d, n_kv, 1, hkv)
        X = L.ggml_repeat_4d(G.ctx, X, d, n_kv, g, hkv)
        out.append(L.ggml_reshape_3d(G.ctx, X, d, n_kv, hq))
    return out


def causal_mask(n_q, n_kv, live):
    """query i at position live - n_q + i sees positions 0 .. that one"""
    mask = np.full((n_q, n_kv), -np.inf, np.float16)
    for i in range(n_q):
        mask[i, :live - n_q + i + 1] = 0
    return mask


def plan_labels(gpu, G):
    return [lab.split(":", 1)[0] for lab, _ in gpu.profile(G.gf, 1)]


@pytest.mark.parametrize("n_kv,live", [(1024, 383), (1024, 1024), (4096, 3008)])
@pytest.mark.parametrize("n_q", [8, 256])
@pytest.mark.parametrize("prec_f32", [True, False])
def test_naive_chain_over_repeat_expanded_kv(ggml, gpu, ref, n_kv, live, n_q, prec_f32):
    """the prefill attention of the unmodified host's HIP lane: K/V of the
    f16 caches expanded to the 16 query heads by RESHAPE / REPEAT / RESHAPE,
    the unfused chain (nn/decoder.rs:2154-2200) over the whole span under the
    causal mask, with GGML_PREC_F32 on both products as the host sets it for
    a ROCm backend (cpu_graph.rs:157-165) or without. One launch: no REPEAT,
    no scores or V^T in memory; bit for bit the oracle's chain"""
    d, hq, hkv = 128, 16, 8
    print(f"naive chain over expanded K/V: kv {n_kv} live {live} n_q {n_q} prec_f32 {prec_f32}", flush=True)
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = causal_mask(n_q, n_kv, live)
    scale = 1.0 / math.sqrt(d)
    G = ggml.Graph()
    L = G.lib
    Qs = G.new(ggml.F32, d, hq, n_q)  # the rotated query rows, [d, heads, tokens]
    K = G.new(ggml.F16, d, n_kv, hkv, 1)
    V = G.new(ggml.F16, d, n_kv, hkv, 1)
    M = G.new(ggml.F16, n_kv, n_q, 1, 1)
    Q = L.ggml_permute(G.ctx, L.ggml_reshape_4d(G.ctx, Qs, d, hq, n_q, 1), 0, 2, 1, 3)
    Kx, Vx = hip_lane_kv(L, G, K, V, d, n_kv, hq, hkv)
    scores = L.ggml_mul_mat(G.ctx, Kx, Q)
    probs = L.ggml_soft_max_ext(G.ctx, scores, M, scale, 0.0)
    vt = L.ggml_cont(G.ctx, L.ggml_transpose(G.ctx, Vx))
    cx = L.ggml_mul_mat(G.ctx, vt, probs)
    if prec_f32:
        L.ggml_mul_mat_set_prec(scores, ggml.GGML_PREC_F32)
        L.ggml_mul_mat_set_prec(cx, ggml.GGML_PREC_F32)
    att = L.ggml_cont(G.ctx, L.ggml_permute(G.ctx, cx, 0, 2, 1, 3))
    G.build(att)
    G.allocate(gpu.buft)
    G.set(Qs, q)
    G.set(K, k.view(np.uint16))
    G.set(V, v.view(np.uint16))
    G.set(M, mask.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    got = G.get(att).reshape(n_q, hq, d)
    want = ref.naive_attention(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale,
                               prec_f32=prec_f32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rel_err(got, want)
    # replayed (captured) computes give the same bits
    assert G.compute(gpu.backend) == 0 and G.compute(gpu.backend) == 0
    assert np.array_equal(G.get(att).reshape(n_q, hq, d).view(np.uint32), want.view(np.uint32))
    labels = plan_labels(gpu, G)
    assert "attn_naive" in labels and "repeat" not in labels, labels
    assert not any(l.startswith("mul_mat") or l in ("soft_max", "copy") for l in labels), labels
    G.free()


@pytest.mark.parametrize("n_q", [1, 64])
def test_flash_attn_ext_over_repeat_expanded_kv(ggml, gpu, n_q):
    """FLASH_ATTN_EXT reading REPEAT-expanded K/V (the HIP lane's decode
    attention) gives the bits of the same attention over the caches
    themselves (native GQA), and the expansion is never launched"""
    d, hq, hkv, n_kv, live = 128, 16, 8, 1024, 700
    print(f"flash_attn_ext over expanded K/V n_q={n_q}", flush=True)
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = causal_mask(n_q, n_kv, live)
    scale = 1.0 / math.sqrt(d)
    outs = []
    for expand in (False, True):
        G = ggml.Graph()
        L = G.lib
        Qs = G.new(ggml.F32, d, hq, n_q)
        K = G.new(ggml.F16, d, n_kv, hkv, 1)
        V = G.new(ggml.F16, d, n_kv, hkv, 1)
        M = G.new(ggml.F16, n_kv, n_q, 1, 1)
        Q = L.ggml_permute(G.ctx, L.ggml_reshape_4d(G.ctx, Qs, d, hq, n_q, 1), 0, 2, 1, 3)
        Kx, Vx = hip_lane_kv(L, G, K, V, d, n_kv, hq, hkv) if expand else (K, V)
        O = L.ggml_flash_attn_ext(G.ctx, Q, Kx, Vx, M, scale, 0.0, 0.0)
        G.build(O)
        G.allocate(gpu.buft)
        G.set(Qs, q)
        G.set(K, k.view(np.uint16))
        G.set(V, v.view(np.uint16))
        G.set(M, mask.view(np.uint16))
        assert G.compute(gpu.backend) == 0
        outs.append(G.get(O).copy())
        if expand:
            assert "repeat" not in plan_labels(gpu, G)
        G.free()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("tname", ["f32", "f16"])
def test_repeat_materialised(ggml, gpu, tname):
    """a REPEAT that is a graph output is launched: every dim tiled, equal to
    numpy's tile of the source"""
    typ, dt = (ggml.F32, np.float32) if tname == "f32" else (ggml.F16, np.float16)
    print(f"repeat {tname}", flush=True)
    x = RNG.standard_normal((2, 1, 3, 5)).astype(dt)  # [ne3, ne2, ne1, ne0]
    G = ggml.Graph()
    X = G.new(typ, 5, 3, 1, 2)
    R = G.lib.ggml_repeat_4d(G.ctx, X, 10, 6, 4, 2)
    G.build(R)
    G.allocate(gpu.buft)
    G.set(X, x if typ == ggml.F32 else x.view(np.uint16))
    assert G.compute(gpu.backend) == 0
    got = G.get(R)
    got = got if typ == ggml.F32 else got.view(np.float16)
    assert np.array_equal(got.reshape(2, 4, 6, 10), np.tile(x, (1, 4, 2, 2)))
    assert "repeat" in plan_labels(gpu, G)
    G.free()
