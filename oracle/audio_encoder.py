"""numpy restatement of the Qwen3-ASR audio encoder graph (the decoder's
prefix producer), as the host builds it for a GPU backend:
  mel chunk layout, positions, mask   models/qwen/audio_encoder.rs:324-360, 798-845
  conv stem                           audio_encoder.rs:480-552, nn/conv.rs:39-52, 82-111
  channel permute, conv_out, positions audio_encoder.rs:553-605, nn/encoder.rs:575-610
  encoder block                       nn/encoder.rs:654-870, nn/attn.rs:89-126,
                                      nn/norm.rs:10-31, nn/ffn.rs:22-50
  ln_post, proj1, GELU_ERF, proj2     audio_encoder.rs:615-672

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the device
encoder; the product never imports it.

Every op's result is rounded to f32 as the graph stores it. The operands
follow the device's and ggml's conversion rules, so that what is left
between the two is the summation order of float products: columns rounded to
f16 for f16 projections or quantized to Q8_0 activations for Q8_0 ones
(ggml-cpu's vec_dot_type), the attention's query, K and V rounded to f16
(f32 K / V are converted to f16 on a GPU backend), LayerNorm and GELU_ERF
through the pinned oracle functions. Products are summed in f64.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from oracle import ref

CHUNK_FRAMES = 100  # QWEN3_AUDIO_CHUNK_FRAMES (audio_encoder.rs:52)
LN_EPS = 1.0e-5     # QWEN3_AUDIO_LAYER_NORM_EPSILON (:53)
F32, F16, Q8_0 = 0, 1, 8

# tensor kinds (enum oa_qwen_audio_tensor_kind)
(ATTN_NORM_W, ATTN_NORM_B, Q, Q_B, K, K_B, V, V_B, O, O_B, FFN_NORM_W, FFN_NORM_B, UP, UP_B, DOWN,
 DOWN_B) = range(16)
(CONV1_W, CONV1_B, CONV2_W, CONV2_B, CONV3_W, CONV3_B, CONV_OUT, CONV_OUT_B, LN_POST_W, LN_POST_B, PROJ1,
 PROJ1_B, PROJ2, PROJ2_B, INV_TIMESCALES) = range(100, 115)


def conv_out_len(n: int) -> int:
    """floor((n + 2p - d(k - 1) - 1) / s) + 1 with k 3, s 2, p 1, d 1 (runtime_contract.rs:29-45)"""
    return (n - 1) // 2 + 1


def token_count(n_frames: int) -> int:
    """qwen3_audio_token_count_for_mel_frames (audio_encoder.rs:859-867)"""
    if n_frames <= 0:
        return 0
    return -(-n_frames // CHUNK_FRAMES) * conv_out_len(conv_out_len(conv_out_len(CHUNK_FRAMES)))


def _f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32)


def _vec(w, layer: int, kind: int) -> np.ndarray:
    return w.array(layer, kind).view(np.float32)


def _matrix(w, layer: int, kind: int, rows: int, k: int, wtype: int) -> np.ndarray:
    """[rows, k] projection as f64 (dequantized)"""
    raw = w.array(layer, kind)
    if wtype == F32:
        return raw.view(np.float32).reshape(rows, k).astype(np.float64)
    if wtype == F16:
        return raw.view(np.float16).reshape(rows, k).astype(np.float64)
    return ref.dequantize(Q8_0, raw, rows * k).reshape(rows, k).astype(np.float64)


def _columns(x: np.ndarray, wtype: int) -> np.ndarray:
    """x [T, K] f32 as the projection consumes it: f16-rounded, Q8_0-quantized or as is"""
    if wtype == F16:
        return x.astype(np.float16).astype(np.float64)
    if wtype == Q8_0:
        k = x.shape[1]
        return np.stack([ref.dequantize(Q8_0, ref.quantize_act(Q8_0, r), k) for r in x]).astype(np.float64)
    return x.astype(np.float64)


# how the projections sum their products: "f64" (exact to f64, then one
# rounding) or "f32" (float32 BLAS, another order and rounding per step) --
# the spread between the two bounds what the order of float sums alone moves
SUMS = {"mode": "f64"}


def linear(x: np.ndarray, wm: np.ndarray, b: np.ndarray, wtype: int) -> np.ndarray:
    """linear_with_bias (nn/encoder.rs:655-671): MUL_MAT (f32 result), then ADD(bias) in f32"""
    xc = _columns(x, wtype)
    if SUMS["mode"] == "f32":
        y = _f32(xc).astype(np.float32) @ _f32(wm).T
    else:
        y = _f32(xc @ wm.T)
    return _f32(y + b)


def layer_norm(x: np.ndarray, wv: np.ndarray, bv: np.ndarray) -> np.ndarray:
    """apply_affine_layer_norm (nn/norm.rs:10-31): NORM, MUL(w), ADD(b)"""
    return _f32(_f32(ref.norm(x, LN_EPS) * wv) + bv)


def gelu_erf(x: np.ndarray) -> np.ndarray:
    f = ref.lib().ref_gelu_erf
    return np.vectorize(lambda v: f(float(v)), otypes=[np.float32])(x)


def sincos(a: np.ndarray):
    """the deterministic sine / cosine the device runs for SIN / COS"""
    s, c = np.empty_like(a), np.empty_like(a)
    fs, fc = C.c_float(), C.c_float()
    for idx, v in np.ndenumerate(a):
        ref.lib().ref_sincosf_det(float(v), C.byref(fs), C.byref(fc))
        s[idx], c[idx] = fs.value, fc.value
    return s, c


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, heads: int) -> np.ndarray:
    """FLASH_ATTN_EXT over the head views with a zero mask: per head softmax(q
    k^T / sqrt(hd)) v with q, k, v rounded to f16, in f64; [rows, heads * hd]"""
    rows, d = q.shape
    hd = d // heads
    out = np.zeros((rows, d), np.float64)
    r16 = lambda a: a.astype(np.float16).astype(np.float64)  # noqa: E731
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = r16(q[:, sl]) @ r16(k[:, sl]).T * np.float64(np.float32(1.0 / np.sqrt(hd)))
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, sl] = (p @ r16(v[:, sl])) / p.sum(axis=1, keepdims=True)
    return _f32(out)


def encode(w, mel: np.ndarray, sums: str = "f64") -> np.ndarray:
    """mel [n_mels, n_frames] -> [rows, out_dim] (w: openasr_amd.decoders.QwenAudioWeights);
    sums: how the projections sum their products (SUMS)"""
    SUMS["mode"] = sums
    try:
        return _encode(w, mel)
    finally:
        SUMS["mode"] = "f64"


def _encode(w, mel: np.ndarray) -> np.ndarray:
    c = w.cfg
    n_mels, n_frames = mel.shape
    chunks = -(-n_frames // CHUNK_FRAMES)
    cof = conv_out_len(conv_out_len(conv_out_len(CHUNK_FRAMES)))
    rows = chunks * cof
    fb = conv_out_len(conv_out_len(conv_out_len(n_mels)))
    # pack_mel_into_chunked_layout: [chunk][mel][100 frames], the tail zero-padded
    packed = np.zeros((chunks, 1, n_mels, CHUNK_FRAMES), np.float32)
    for ch in range(chunks):
        seg = mel[:, ch * CHUNK_FRAMES:(ch + 1) * CHUNK_FRAMES]
        packed[ch, 0, :, :seg.shape[1]] = seg
    # conv stem: conv_2d (f32 kernel: f32 columns) + bias + GELU_ERF, three times
    x = packed
    ic = 1
    for kw, kb in ((CONV1_W, CONV1_B), (CONV2_W, CONV2_B), (CONV3_W, CONV3_B)):
        oc = c.conv_channels
        kern = _vec(w, -1, kw).reshape(oc, ic * 9).astype(np.float64)
        cols = ref.im2col(x, 3, 3, 2, 2, 1, 1, 1, 1).astype(np.float64)  # [N, OH, OW, ic 9]
        y = _f32(cols @ kern.T).transpose(0, 3, 1, 2)                   # [N, OC, OH, OW]
        y = _f32(y + _vec(w, -1, kb)[None, :, None, None])
        x = gelu_erf(y)
        ic = oc
    # [N, C, F, 13] -> [N, 13, C F]; conv_out; + bias; + positions
    x = np.ascontiguousarray(x.transpose(0, 3, 1, 2)).reshape(chunks, cof, c.conv_channels * fb)
    d = c.d_model
    x = linear(x.reshape(chunks * cof, -1), _matrix(w, -1, CONV_OUT, d, c.conv_channels * fb, c.wtype),
               _vec(w, -1, CONV_OUT_B), c.wtype).reshape(chunks, cof, d)
    inv = _vec(w, -1, INV_TIMESCALES)
    ang = _f32(np.arange(cof, dtype=np.float32)[:, None] * inv[None, :])
    s, co = sincos(ang)
    pos = np.concatenate([s, co], axis=1)  # [13, d], half-split channels
    x = _f32(x + pos[None]).reshape(rows, d)
    for layer in range(c.n_layers):
        mat = lambda kind, r, k: _matrix(w, layer, kind, r, k, c.wtype)  # noqa: E731
        vec = lambda kind: _vec(w, layer, kind)  # noqa: E731
        h = layer_norm(x, vec(ATTN_NORM_W), vec(ATTN_NORM_B))
        q = linear(h, mat(Q, d, d), vec(Q_B), c.wtype)
        k = linear(h, mat(K, d, d), vec(K_B), c.wtype)
        v = linear(h, mat(V, d, d), vec(V_B), c.wtype)
        att = attention(q, k, v, c.n_heads)
        x = _f32(linear(att, mat(O, d, d), vec(O_B), c.wtype) + x)
        h = layer_norm(x, vec(FFN_NORM_W), vec(FFN_NORM_B))
        u = gelu_erf(linear(h, mat(UP, c.ffn, d), vec(UP_B), c.wtype))
        x = _f32(linear(u, mat(DOWN, d, c.ffn), vec(DOWN_B), c.wtype) + x)
    x = layer_norm(x, _vec(w, -1, LN_POST_W), _vec(w, -1, LN_POST_B))
    x = gelu_erf(linear(x, _matrix(w, -1, PROJ1, d, d, c.wtype), _vec(w, -1, PROJ1_B), c.wtype))
    return linear(x, _matrix(w, -1, PROJ2, c.out_dim, d, c.wtype), _vec(w, -1, PROJ2_B), c.wtype)
