"""The device reproduces the committed oracle fixtures
(tests/golden/oracle_fixtures.npz) bit for bit, op by op, through the C ABI."""

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name,typ,m,k", [("mm_q4_K", "Q4_K", 96, 512), ("mm_q8_0", "Q8_0", 64, 256)])
def test_mul_mat_fixture(ggml, gpu, fx, name, typ, m, k):
    print(f"golden {name}", flush=True)
    wt = getattr(ggml, typ)
    x = fx[name + "_x"]
    G = ggml.Graph()
    W = G.new(wt, k, m, weight=True)
    X = G.new(ggml.F32, k, x.shape[0])
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    G.build(Y)
    G.allocate(gpu.buft)
    G.set(W, fx[name + "_w"])
    G.set(X, x)
    assert G.compute(gpu.backend) == 0
    assert np.array_equal(bits(G.get(Y).reshape(x.shape[0], m)), bits(fx[name + "_y"]))
    G.free()


def test_row_op_fixtures(ggml, gpu, fx):
    print("golden row ops", flush=True)
    xn, xr, pos = fx["norm_in"], fx["rope_in"], fx["rope_pos"]
    xs, xa = fx["softmax_in"], fx["act_fn_in"]
    G = ggml.Graph()
    N = G.new(ggml.F32, xn.shape[1], xn.shape[0])
    R = G.new(ggml.F32, 128, xr.shape[1], xr.shape[0])
    P = G.new(ggml.I32, xr.shape[0])
    S = G.new(ggml.F32, xs.shape[1], xs.shape[0])
    M = G.new(ggml.F16, xs.shape[1], xs.shape[0])
    A = G.new(ggml.F32, xa.shape[0])
    outs = [G.lib.ggml_rms_norm(G.ctx, N, 1e-6), G.lib.ggml_norm(G.ctx, N, 1e-5),
            G.lib.ggml_rope_ext(G.ctx, R, P, None, 128, 2, 4096, 1e6, 1.0, 0.0, 1.0, 32.0, 1.0),
            G.lib.ggml_soft_max_ext(G.ctx, S, M, 0.125, 0.0), G.lib.ggml_silu(G.ctx, A), G.lib.ggml_gelu(G.ctx, A)]
    G.build(*outs)
    G.allocate(gpu.buft)
    for T, v in ((N, xn), (R, xr), (P, pos), (S, xs), (M, fx["softmax_mask"]), (A, xa)):
        G.set(T, v)
    assert G.compute(gpu.backend) == 0
    want = ["rms_norm_out", "layer_norm_out", "rope_out", "softmax_out", "silu_out", "gelu_out"]
    for o, key in zip(outs, want):
        assert np.array_equal(bits(G.get(o)).reshape(-1), bits(fx[key]).reshape(-1)), key
    G.free()


def test_flash_attn_fixture(ggml, gpu, fx):
    print("golden flash_attn", flush=True)
    q, k, v, m = fx["fa_q"], fx["fa_k"], fx["fa_v"], fx["fa_mask"]
    n_seq, hq, d = q.shape
    hkv, n_kv = k.shape[1], k.shape[2]
    G = ggml.Graph()
    Q = G.new(ggml.F32, d, 1, hq, n_seq)
    K = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    V = G.new(ggml.F16, d, n_kv, hkv, n_seq)
    M = G.new(ggml.F16, n_kv, 1, 1, n_seq)
    O = G.lib.ggml_flash_attn_ext(G.ctx, Q, K, V, M, 0.125, 0.0, 0.0)
    G.lib.ggml_flash_attn_ext_set_prec(O, ggml.GGML_PREC_F32)  # the exact chunked definition
    G.build(O)
    G.allocate(gpu.buft)
    G.set(Q, q)
    G.set(K, k)
    G.set(V, v)
    G.set(M, m)
    assert G.compute(gpu.backend) == 0
    out = G.get(O).reshape(n_seq, 1, hq, d)
    assert np.array_equal(bits(out), bits(fx["fa5_out"]))
    G.free()
