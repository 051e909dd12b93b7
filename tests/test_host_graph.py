"""Host-side graph construction through the C ABI (no device): op shapes,
strides and op_params packing follow ggml's documented semantics, which is
what the device plugin decodes. Mirrors the graph the OpenASR LLM block
emits (crates/openasr-core/src/nn/decoder.rs:1850-2145).
"""

import ctypes as C
import struct

import numpy as np


def ne(g, t):
    tt = g.tensor(t)
    return tuple(int(tt.ne[i]) for i in range(4))


def nb(g, t):
    tt = g.tensor(t)
    return tuple(int(tt.nb[i]) for i in range(4))


def test_shapes_of_decoder_ops(ggml):
    G = ggml.Graph()
    L = G.lib
    x = G.new(ggml.F32, 1024, 8)
    w = G.new(ggml.Q4_K, 1024, 4096, weight=True)
    y = L.ggml_mul_mat(G.ctx, w, x)
    assert ne(ggml, y) == (4096, 8, 1, 1) and ggml.tensor(y).type == ggml.F32
    q = L.ggml_view_2d(G.ctx, y, 2048, 8, 4096 * 4, 0)
    assert nb(ggml, q)[1] == 4096 * 4
    qc = L.ggml_cont(G.ctx, q)
    q3 = L.ggml_reshape_3d(G.ctx, qc, 128, 16, 8)
    qp = L.ggml_permute(G.ctx, q3, 0, 2, 3, 1)  # decode batch permute of nn/decoder.rs:1970-1975
    assert ne(ggml, qp) == (128, 1, 16, 8)
    assert nb(ggml, qp) == (4, 128 * 16 * 4 * 8, 128 * 4, 128 * 16 * 4)
    kc = G.new(ggml.F16, 128, 1024, 8, 8)
    mask = G.new(ggml.F16, 1024, 1, 1, 8)
    fa = L.ggml_flash_attn_ext(G.ctx, qp, kc, kc, mask, 0.125, 0.0, 0.0)
    assert ne(ggml, fa) == (128, 16, 1, 8)
    params = ggml.tensor(fa).op_params
    assert struct.unpack("f", struct.pack("i", params[0]))[0] == 0.125
    pos = G.new(ggml.I32, 8)
    r = L.ggml_rope_ext(G.ctx, q3, pos, None, 128, 2, 1024, 1e6, 1.0, 0.0, 1.0, 32.0, 1.0)
    p = ggml.tensor(r).op_params
    assert (p[1], p[2], p[4]) == (128, 2, 1024)
    assert struct.unpack("f", struct.pack("i", p[5]))[0] == 1e6
    idx = G.new(ggml.I32, 1, 1, 8, 1)
    kn = G.new(ggml.F32, 128, 1, 8, 8)
    sr = L.ggml_set_rows(G.ctx, kc, kn, idx)
    srt = ggml.tensor(sr)
    assert srt.view_src == kc and ne(ggml, sr) == ne(ggml, kc)
    G.build(fa, sr)
    n = L.ggml_graph_n_nodes(G.gf)
    L.ggml_op_name.restype = C.c_char_p
    L.ggml_op_name.argtypes = [C.c_int]
    ops = [L.ggml_op_name(ggml.tensor(L.ggml_graph_node(G.gf, i)).op).decode() for i in range(n)]
    assert len(set(L.ggml_graph_node(G.gf, i) for i in range(n))) == n  # no duplicates
    # evaluation order: parents first
    assert ops.index("MUL_MAT") < ops.index("CONT") < ops.index("FLASH_ATTN_EXT")
    assert ops[-1] == "SET_ROWS" and "ROPE" not in ops  # rope is not an ancestor of either output
    G.free()


def test_get_rows_and_argmax_shapes(ggml):
    G = ggml.Graph()
    L = G.lib
    emb = G.new(ggml.Q8_0, 384, 51865, weight=True)
    ids = G.new(ggml.I32, 3)
    rows = L.ggml_get_rows(G.ctx, emb, ids)
    assert ne(ggml, rows) == (384, 3, 1, 1) and ggml.tensor(rows).type == ggml.F32
    logits = G.new(ggml.F32, 51865, 3)
    am = L.ggml_argmax(G.ctx, logits)
    assert ne(ggml, am) == (3, 1, 1, 1) and ggml.tensor(am).type == ggml.I32
    G.free()


def test_quantize_chunk_q8_0_matches_oracle(ggml, ref):
    x = ggml.synth_normal(7, 1, 64 * 1024, 0.0, 0.02).reshape(64, 1024)
    assert np.array_equal(ggml.quantize(ggml.Q8_0, x), ref.quantize_weights(ref.Q8_0, x))


def test_quantize_chunk_q4_K_valid_blocks(ggml, ref):
    x = ggml.synth_normal(7, 2, 16 * 1024, 0.0, 0.02).reshape(16, 1024)
    q = ggml.quantize(ggml.Q4_K, x)
    y = ref.dequantize(ref.Q4_K, q, x.size).reshape(x.shape)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert rel < 0.12  # 4-bit with 6-bit scales: ~8% relative rms error on Gaussian weights


def test_synth_normal_is_deterministic_and_sliceable(ggml):
    a = ggml.synth_normal(42, 3, 10000)
    b = ggml.synth_normal(42, 3, 5000, first=5000)
    assert np.array_equal(a[5000:], b)
    assert abs(a.mean()) < 0.05 and abs(a.std() - 1) < 0.05
    assert not np.array_equal(a, ggml.synth_normal(42, 4, 10000))
