"""ggml_backend_mi355x_graph_compute_static -- the graph compute that
allocates no device memory -- against ggml_backend_graph_compute on the same
graphs and inputs, bit for bit: a graph whose plan uses every kind of scratch
(the tile GEMM's quantized activations, the decode attention's chunk
partials, argmax partials), computed twice in a row, the second time with
smaller inputs (fewer columns, a shorter KV span), so the second call runs on
an array that still holds the first call's contents. The device's allocation
ledger (memory ABI v1) must not move across a call."""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def build(ggml, gpu, n, kv, seed):
    rng = np.random.default_rng(seed)
    m, k, d, hq, hkv = 1024, 1024, 128, 16, 8
    G = ggml.Graph()
    L = G.lib
    W = G.new(ggml.Q4_K, k, m, weight=True)
    X = G.new(ggml.F32, k, n)
    Y = L.ggml_mul_mat(G.ctx, W, X)
    A = L.ggml_argmax(G.ctx, Y)
    Q = G.new(ggml.F32, d, 1, hq, 1)
    K = G.new(ggml.F16, d, kv, hkv, 1)
    V = G.new(ggml.F16, d, kv, hkv, 1)
    Mk = G.new(ggml.F16, kv, 1, 1, 1)
    O = L.ggml_flash_attn_ext(G.ctx, Q, K, V, Mk, 1.0 / np.sqrt(d), 0.0, 0.0)
    G.build(Y, A, O)
    G.allocate(gpu.buft)
    w = ggml.quantize(ggml.Q4_K, ggml.synth_normal(seed, 1, m * k, 0, 0.02).reshape(m, k))
    G.set(W, w)
    G.set(X, rng.standard_normal((n, k)).astype(np.float32))
    G.set(Q, rng.standard_normal((1, hq, 1, d)).astype(np.float32))
    G.set(K, rng.standard_normal((1, hkv, kv, d)).astype(np.float16).view(np.uint16))
    G.set(V, rng.standard_normal((1, hkv, kv, d)).astype(np.float16).view(np.uint16))
    live = kv - kv // 5  # a masked tail, as the decode step's fixed span has
    mask = np.zeros(kv, np.float16)
    mask[live:] = -np.inf
    G.set(Mk, mask.view(np.uint16))
    return G, (Y, A, O)


def outputs(G, outs):
    return [G.get(t).copy() for t in outs]


def test_static_compute_matches_graph_compute(ggml, gpu):
    lib = gpu.cdll
    lib.ggml_backend_mi355x_graph_compute_static.restype = C.c_int
    lib.ggml_backend_mi355x_graph_compute_static.argtypes = [C.c_void_p, C.c_void_p]
    lib.ggml_backend_mi355x_static_scratch_bytes.restype = C.c_size_t
    assert lib.ggml_backend_mi355x_static_scratch_bytes() == 64 << 20
    for n, kv, seed in ((100, 4096, 1), (16, 512, 2)):
        G, outs = build(ggml, gpu, n, kv, seed)
        for t in outs:  # poison the outputs: every value must be written
            G.set(t, np.full(G.get(t).shape, -1, G.get(t).dtype))
        mem = ggml.MemoryApi(gpu.reg, gpu.dev, gpu.backend)
        s0 = mem.stats()[0]
        assert lib.ggml_backend_mi355x_graph_compute_static(gpu.backend, G.gf) == 0
        got = outputs(G, outs)
        # the call allocated nothing: the device ledger did not move
        s1 = mem.stats()[0]
        assert s1.allocation_count == s0.allocation_count and s1.generation == s0.generation
        assert s1.backend_owned_workspace_bytes == s0.backend_owned_workspace_bytes
        assert s1.backend_owned_live_bytes == s0.backend_owned_live_bytes
        assert G.compute(gpu.backend) == 0
        want = outputs(G, outs)
        for g, w_ in zip(got, want):
            assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                                  w_.view(np.uint32) if w_.dtype == np.float32 else w_)
        G.free()


def test_static_compute_refuses_oversized_scratch(ggml, gpu):
    """a plan whose scratch exceeds the fixed array is refused with
    GGML_STATUS_ALLOC_FAILED before any launch"""
    lib = gpu.cdll
    lib.ggml_backend_mi355x_graph_compute_static.restype = C.c_int
    lib.ggml_backend_mi355x_graph_compute_static.argtypes = [C.c_void_p, C.c_void_p]
    G = ggml.Graph()
    k, n = 2048, 40000  # Q8_K activations of 40000 columns: ~86 MB
    W = G.new(ggml.Q4_K, k, 256, weight=True)
    X = G.new(ggml.F32, k, n)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    G.build(Y)
    G.allocate(gpu.buft)
    assert lib.ggml_backend_mi355x_graph_compute_static(gpu.backend, G.gf) == -2
    G.free()
