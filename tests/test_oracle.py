"""Pins the CPU oracle (oracle/ggml_cpu_ref.c) before anything is checked
against it. Each test fixes the oracle by something other than its own
formula: numpy's independent f16 codec, hand-packed known-answer blocks,
f64 brute force over dequantized operands, closed forms, and invariants
(GQA == explicit K/V repetition, masked positions contribute nothing).
The reference holds no golden vectors for this path (its arithmetic lives
in the un-vendored openasr-ggml fork), so these are the pins.
"""

import math
from fractions import Fraction

import numpy as np
import pytest

RNG = np.random.default_rng(1234)


# ------------------------------------------------------------------ f16 --

def test_fp16_matches_numpy_codec(ref):
    L = ref.lib()
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e-8, 6e-8, 5.96e-8, 2.98e-8,
                         6.1035e-5, 6.1e-5, np.inf, -np.inf, 0.1, 1.0 / 3.0, 2049.0, 2051.0, 4097.0],
                        dtype=np.float32)
    x = np.concatenate([specials, RNG.standard_normal(20000).astype(np.float32) * 10.0 ** RNG.integers(-8, 5, 20000)])
    x = x.astype(np.float32)
    got = np.array([L.ref_fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = np.array([L.ref_fp16_to_fp32(int(h)) for h in range(0, 65536, 7)], dtype=np.float32)
    want_back = np.arange(0, 65536, 7, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(back), np.isnan(want_back))
    ok = ~np.isnan(want_back)
    assert np.array_equal(back[ok], want_back[ok])


# ----------------------------------------------------------------- Q8_0 --

def test_q8_0_weight_known_answer(ref):
    x = (np.arange(32, dtype=np.float32) - 15.5) * 0.25  # amax = 3.875
    q = ref.quantize_weights(ref.Q8_0, x.reshape(1, 32))
    d = np.frombuffer(q[:2].tobytes(), dtype=np.float16)[0]
    assert d == np.float16(3.875 / 127.0)
    qs = q[2:34].view(np.int8)
    # round half away from zero: x*127/3.875 for x=-3.875 -> -127
    want = np.array([math.copysign(math.floor(abs(v * (1.0 / np.float32(3.875 / 127.0))) + 0.5), v) for v in x])
    assert np.array_equal(qs.astype(np.int64), want.astype(np.int64))
    z = ref.quantize_weights(ref.Q8_0, np.zeros((1, 32), np.float32))
    assert not z.any()


def test_q8_0_activation_rounds_half_to_even(ref):
    # amax = 127 makes the multiplier exactly 1.0: 2.5 -> 2 (x86 ggml-cpu), 3.5 -> 4
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 2.5, 3.5, -2.5
    qa = ref.quantize_act(ref.Q8_0, x)[2:34].view(np.int8)
    assert list(qa[:4]) == [127, 2, 4, -2]
    qw = ref.quantize_weights(ref.Q8_0, x.reshape(1, 32))[2:34].view(np.int8)
    assert list(qw[:4]) == [127, 3, 4, -3]  # weights: half away from zero


def test_q8_0_roundtrip_error_bound(ref):
    x = RNG.standard_normal((8, 256)).astype(np.float32)
    q = ref.quantize_weights(ref.Q8_0, x)
    y = ref.dequantize(ref.Q8_0, q, x.size).reshape(x.shape)
    d = np.abs(x.reshape(-1, 32)).max(axis=1) / 127.0
    d16 = q.reshape(-1, 34)[:, :2].copy().view(np.float16)[:, 0].astype(np.float64)
    err = np.abs(x - y).reshape(-1, 32).max(axis=1)
    # half a step, plus the stored scale's f16 rounding times the largest quant
    assert np.all(err <= d * 0.5 + 127 * np.abs(d16 - d) + 1e-7)


# ----------------------------------------------------------------- Q4_K --

def pack_q4_K(d, dmin, sc, mn, q):
    """Independent block packer from the block_q4_K spec: 6-bit scales of
    sub-blocks 0..3 in bytes 0..3 (mins 4..7); sub-blocks 4..7 keep their
    low nibbles in bytes 8..11 (scale low, min high) and their top two bits
    in bits 6..7 of bytes 0..3 (scales) and 4..7 (mins)."""
    s = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= mn[j] & 63
        else:
            s[j + 4] |= (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    qs = np.zeros(128, np.uint8)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    hdr = np.array([d, dmin], np.float16).view(np.uint8)
    return np.concatenate([hdr, s, qs])


def test_q4_K_dequant_known_answer(ref):
    sc = np.array([1, 7, 13, 63, 17, 33, 48, 62])
    mn = np.array([0, 5, 63, 9, 31, 16, 47, 2])
    q = RNG.integers(0, 16, 256)
    d, dmin = np.float16(0.0125), np.float16(0.0031)
    blk = pack_q4_K(d, dmin, sc, mn, q)
    assert blk.size == 144
    got = ref.dequantize(ref.Q4_K, blk, 256)
    want = np.array([np.float32(d) * np.float32(sc[i // 32]) * q[i] - np.float32(dmin) * np.float32(mn[i // 32])
                     for i in range(256)], np.float32)
    assert np.allclose(got, want, rtol=0, atol=1e-6)


def test_q4_K_quantizer_roundtrip(ref):
    x = (RNG.standard_normal((4, 512)) * 0.02).astype(np.float32)
    q = ref.quantize_weights(ref.Q4_K, x)
    y = ref.dequantize(ref.Q4_K, q, x.size).reshape(x.shape)
    # 4-bit grid over each 32-weight sub-block range: error well under a step
    rng = (x.reshape(-1, 32).max(1) - np.minimum(x.reshape(-1, 32).min(1), 0))
    err = np.abs(x - y).reshape(-1, 32).max(1)
    assert np.all(err <= rng / 15.0 * 0.75 + 1e-6)


def test_q4_K_quantizer_recovers_an_exact_grid(ref):
    """Weights on an exact Q4_K grid, x = (k_j q - n_j) 2^-12 with 6-bit step
    codes k_j and min codes n_j (63 among each) and every sub-block spanning
    q = 0..15: any fit that keeps an exact solution must code d = dmin =
    2^-12, scales k, mins n and quants q -- the bytes the independent packer
    writes. Pins the 6-bit coding against the largest scale, the f16 super
    scales, the requantization and the packing, whatever the search's
    candidate order."""
    for trial in range(4):
        k = RNG.integers(1, 64, 8)
        n = RNG.integers(0, 64, 8)
        k[RNG.integers(0, 8)] = 63
        n[RNG.integers(0, 8)] = 63
        q = RNG.integers(0, 16, 256)
        for j in range(8):
            pos = RNG.choice(32, 2, replace=False)
            q[32 * j + pos[0]], q[32 * j + pos[1]] = 0, 15
        x = np.array([(k[i // 32] * q[i] - n[i // 32]) * 2.0 ** -12 for i in range(256)], np.float32)
        want = pack_q4_K(np.float16(2.0 ** -12), np.float16(2.0 ** -12), k, n, q)
        got = ref.quantize_weights(ref.Q4_K, x.reshape(1, -1))
        assert np.array_equal(got, want), trial


def test_q4_K_quantizer_closed_forms(ref):
    """An all-zero block codes to zero bytes; a constant positive block c is
    the top quant of step c/15 (min 0), a constant negative block the offset
    alone (step 0): both dequantize to c within the f16 super scale's
    rounding (|c| / 945 a normal f16, so that rounding is relative)."""
    assert not ref.quantize_weights(ref.Q4_K, np.zeros((1, 256), np.float32)).any()
    for c in (0.37, 0.09, -0.52, -0.2):
        x = np.full((1, 256), c, np.float32)
        blk = ref.quantize_weights(ref.Q4_K, x)
        y = ref.dequantize(ref.Q4_K, blk, 256)
        assert np.allclose(y, c, rtol=2 ** -10, atol=0), c
        qs = blk[16:]
        if c > 0:
            assert np.all(qs == 0xFF), c  # quant 15 in both nibbles
        else:
            assert not qs.any(), c


def test_q4_K_quantizer_host_and_oracle_agree(ref, ggml):
    """ggml_quantize_chunk of the host library (the bytes packs and the
    device consume) and the oracle's restatement of the same quantizer give
    the same bytes on N(0, s) rows, mixed-magnitude sub-blocks, blocks with
    one outlier, constant and subnormal blocks."""
    rows = [RNG.standard_normal(1024) * s for s in (0.02, 1.0, 300.0)]
    mixed = RNG.standard_normal(1024) * np.repeat(10.0 ** RNG.uniform(-4, 1, 32), 32)
    outlier = RNG.standard_normal(1024) * 0.01
    outlier[::97] = 3.0
    rows += [mixed, outlier, np.full(1024, 0.25), np.full(1024, -1e-3),
             RNG.standard_normal(1024) * 1e-40, np.abs(RNG.standard_normal(1024))]
    x = np.stack(rows).astype(np.float32)
    assert np.array_equal(ggml.quantize(ggml.Q4_K, x), ref.quantize_weights(ref.Q4_K, x))


# ----------------------------------------------------------------- Q8_K --

def test_q8_K_known_answer_and_invariants(ref):
    x = RNG.standard_normal(512).astype(np.float32)
    x[10] = 5.0
    x[20] = -5.0  # same magnitude later: the first one (+5) sets the sign
    blk = ref.quantize_act(ref.Q8_K, x)
    b0 = blk[:292]
    d = b0[:4].view(np.float32)[0]
    qs = b0[4:260].view(np.int8).astype(np.int64)
    bsums = b0[260:292].view(np.int16).astype(np.int64)
    assert qs[10] == -127 and qs[20] == 127
    assert d == pytest.approx(-5.0 / 127.0, rel=1e-6)
    assert np.array_equal(bsums, qs.reshape(16, 16).sum(1))
    y = ref.dequantize(ref.Q8_K, blk, 512)
    assert np.max(np.abs(y - x)) <= 5.0 / 127.0 * 0.5 * 1.01 + np.abs(x).max() / 127 * 0.01


# ----------------------------------------------------------- dot products --

def test_vec_dot_q8_0_equals_f64_dot_of_dequantized(ref):
    L = ref.lib()
    for n in (32, 256, 1024):
        w = RNG.standard_normal(n).astype(np.float32)
        a = RNG.standard_normal(n).astype(np.float32)
        qw = ref.quantize_weights(ref.Q8_0, w.reshape(1, -1))
        qa = ref.quantize_act(ref.Q8_0, a)
        got = L.ref_vec_dot_q8_0_q8_0(n, qw.ctypes.data, qa.ctypes.data)
        want = np.dot(ref.dequantize(ref.Q8_0, qw, n).astype(np.float64), ref.dequantize(ref.Q8_0, qa, n))
        assert got == pytest.approx(want, rel=1e-5, abs=1e-5)


def test_vec_dot_q4_K_equals_f64_dot_of_dequantized(ref):
    L = ref.lib()
    for n in (256, 1024, 3072):
        w = (RNG.standard_normal(n) * 0.02).astype(np.float32)
        a = RNG.standard_normal(n).astype(np.float32)
        qw = ref.quantize_weights(ref.Q4_K, w.reshape(1, -1))
        qa = ref.quantize_act(ref.Q8_K, a)
        got = L.ref_vec_dot_q4_K_q8_K(n, qw.ctypes.data, qa.ctypes.data)
        want = np.dot(ref.dequantize(ref.Q4_K, qw, n).astype(np.float64),
                      ref.dequantize(ref.Q8_K, qa, n).astype(np.float64))
        assert got == pytest.approx(want, rel=2e-5, abs=2e-5)


@pytest.mark.parametrize("wtype", ["q8_0", "q4_K"])
def test_mul_mat_brute_force_and_column_invariance(ref, wtype):
    t = ref.Q8_0 if wtype == "q8_0" else ref.Q4_K
    m, k, n = 48, 512, 8
    w = (RNG.standard_normal((m, k)) * 0.02).astype(np.float32)
    x = RNG.standard_normal((n, k)).astype(np.float32)
    qw = ref.quantize_weights(t, w)
    y = ref.mul_mat(t, qw, m, k, x)
    wd = ref.dequantize(t, qw, m * k).reshape(m, k).astype(np.float64)
    at = ref.Q8_0 if t == ref.Q8_0 else ref.Q8_K
    xd = np.stack([ref.dequantize(at, ref.quantize_act(at, x[j]), k) for j in range(n)]).astype(np.float64)
    want = xd @ wd.T
    assert np.allclose(y, want, rtol=1e-5, atol=1e-5)
    for j in range(n):
        yj = ref.mul_mat(t, qw, m, k, x[j:j + 1])
        assert np.array_equal(yj[0], y[j])


# ------------------------------------------------------------- row ops ---

def test_norms_closed_form(ref):
    x = RNG.standard_normal((5, 1024)).astype(np.float32) * 3 + 1
    eps = 1e-6
    want = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + eps)
    assert np.allclose(ref.rms_norm(x, eps), want, rtol=2e-6, atol=1e-6)
    mu = x.astype(np.float64).mean(1, keepdims=True)
    want = (x - mu) / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-5)
    assert np.allclose(ref.norm(x, 1e-5), want, rtol=2e-6, atol=1e-6)


def test_rope_neox_closed_form(ref):
    t, h, d = 6, 3, 128
    x = RNG.standard_normal((t, h, d)).astype(np.float32)
    pos = np.array([0, 1, 7, 100, 383, 1023], np.int32)
    y = ref.rope_neox(x, pos, d, 1e6)
    assert np.array_equal(y[0], x[0])  # position 0 is the identity
    half = d // 2
    inv = 1e6 ** (-2.0 * np.arange(half) / d)
    ang = pos[:, None].astype(np.float64) * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x0, x1 = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    want = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], -1)
    # theta is built by repeated f32 multiplication, as ggml does: a few ulp of angle
    assert np.allclose(y, want, rtol=1e-4, atol=1e-4)
    y2 = ref.rope_neox(x, pos, 64, 1e6)  # partial rotation passes the tail through
    assert np.array_equal(y2[..., 64:], x[..., 64:])


def test_activations_closed_form(ref):
    x = np.linspace(-12, 12, 2001).astype(np.float32)
    assert np.allclose(ref.silu(x), x / (1 + np.exp(-x.astype(np.float64))), rtol=1e-6, atol=1e-7)
    g = ref.gelu(x)
    xh = x.astype(np.float16).astype(np.float64)
    exact = 0.5 * xh * (1 + np.tanh(np.sqrt(2 / np.pi) * xh * (1 + 0.044715 * xh * xh)))
    table = exact.astype(np.float16).astype(np.float32)
    inner = (x > -10) & (x < 10)
    # f16 table value: within one f16 ulp of f16(gelu(f16(x))); in the far
    # negative tail the f32 formula's 1 + tanh cancellation adds ~|x| f32 ulps
    ulp = np.abs(np.spacing(table.astype(np.float16))).astype(np.float32)
    assert np.all(np.abs(g[inner] - table[inner]) <= ulp[inner] + 8 * np.abs(x[inner]) * 2.0 ** -24)
    assert np.all(g[x <= -10] == 0) and np.array_equal(g[x >= 10], x[x >= 10])


def test_soft_max_and_argmax(ref):
    x = RNG.standard_normal((4, 37)).astype(np.float32)
    mask = np.zeros((4, 37), np.float16)
    mask[:, 30:] = -np.inf
    y = ref.soft_max_ext(x, mask.view(np.uint16), 0.5)
    z = x.astype(np.float64) * 0.5 + mask.astype(np.float64)
    want = np.exp(z - z.max(1, keepdims=True))
    want /= want.sum(1, keepdims=True)
    assert np.allclose(y, want, rtol=1e-6, atol=1e-7)
    v = np.array([1.0, 3.0, 2.0, 3.0, -1.0], np.float32)
    assert ref.argmax_first(v) == 1 and ref.argmax_last(v) == 3


# ------------------------------------------------------- flash attention --

def textbook_attention(q, k, v, mask, scale, group):
    n_q, hq, d = q.shape
    out = np.zeros((n_q, hq, d))
    for i in range(n_q):
        for h in range(hq):
            kv = h // group
            s = (k[kv].astype(np.float64) @ q[i, h].astype(np.float64)) * scale
            if mask is not None:
                s = s + mask[i].astype(np.float64)
            if np.all(np.isinf(s)):
                continue
            p = np.exp(s - s.max())
            out[i, h] = (p @ v[kv].astype(np.float64)) / p.sum()
    return out


def test_flash_attn_textbook_gqa_and_masking(ref):
    n_q, hq, hkv, n_kv, d = 3, 4, 2, 40, 64
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_q, n_kv), np.float16)
    mask[0, 25:] = -np.inf
    mask[1, :] = -np.inf  # fully masked row -> zeros
    scale = 1 / math.sqrt(d)
    qh = q.astype(np.float16).astype(np.float32)
    want = textbook_attention(qh, k, v, mask, scale, hq // hkv)
    exact = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=False)
    assert np.allclose(exact, textbook_attention(q, k, v, mask, scale, 2), rtol=1e-5, atol=1e-5)
    fid = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=True)
    assert np.abs(fid - want).max() <= 2e-3 * np.abs(want).max()
    assert not fid[1].any() and not exact[1].any()
    # GQA == explicit repetition of each kv head over its query group
    krep = np.repeat(k, 2, axis=0)
    vrep = np.repeat(v, 2, axis=0)
    rep = ref.flash_attn(q, krep.view(np.uint16), vrep.view(np.uint16), mask.view(np.uint16), scale, fidelity=False)
    assert np.array_equal(rep, exact)
    # masked positions contribute nothing: garbage there changes nothing
    k2, v2 = k.copy(), v.copy()
    k2[:, 25:] = 100
    v2[:, 25:] = -50
    m0 = np.zeros((1, n_kv), np.float16)
    m0[0, 25:] = -np.inf
    a = ref.flash_attn(q[:1], k.view(np.uint16), v.view(np.uint16), m0.view(np.uint16), scale, fidelity=False)
    b = ref.flash_attn(q[:1], k2.view(np.uint16), v2.view(np.uint16), m0.view(np.uint16), scale, fidelity=False)
    assert np.array_equal(a, b)


# ---------------------------------------------------- deterministic math --

def ulp_dist(a, b):
    """distance in f32 ulps between float32 arrays"""
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7fffffff), ai)
    bi = np.where(bi < 0, -(bi & 0x7fffffff), bi)
    return np.abs(ai - bi)


def test_det_expf_correctly_rounded(ref):
    L = ref.lib()
    x = np.concatenate([np.linspace(-103, 88.7, 20001), RNG.standard_normal(20000) * 10,
                        [0.0, -0.0, 1.0, -1.0, 1e-8, -1e-8, 88.72, -87.3]]).astype(np.float32)
    got = np.array([L.ref_expf_det(float(v)) for v in x], np.float32)
    want = np.exp(x.astype(np.float64)).astype(np.float32)  # f64 exp rounded once
    d = ulp_dist(got, want)
    assert d.max() <= 1 and np.mean(d == 0) > 0.999
    assert L.ref_expf_det(-200.0) == 0.0 and math.isinf(L.ref_expf_det(100.0))


def test_det_sincos_within_one_ulp(ref):
    L = ref.lib()
    x = np.concatenate([np.linspace(-5000, 5000, 40001), RNG.standard_normal(5000) * 3]).astype(np.float32)
    s = C_float = np.zeros(1, np.float32)
    sv = np.zeros(x.size, np.float32)
    cv = np.zeros(x.size, np.float32)
    for i, v in enumerate(x):
        a = np.zeros(1, np.float32)
        b = np.zeros(1, np.float32)
        L.ref_sincosf_det(float(v), a.ctypes.data, b.ctypes.data)
        sv[i], cv[i] = a[0], b[0]
    xs = x.astype(np.float64)
    ws, wc = np.sin(xs).astype(np.float32), np.cos(xs).astype(np.float32)
    # absolute error bound: half an ulp of 1 plus the f32 rounding
    assert np.abs(sv.astype(np.float64) - np.sin(xs)).max() < 1.2e-7
    assert np.abs(cv.astype(np.float64) - np.cos(xs)).max() < 1.2e-7
    assert np.mean(sv == ws) > 0.99 and np.mean(cv == wc) > 0.99


def test_flash_attn_two_pass_mode(ref):
    n_q, hq, hkv, n_kv, d = 4, 4, 2, 300, 128
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_q, n_kv), np.float16)
    mask[:, 250:] = -np.inf
    mask[3] = -np.inf
    scale = 1 / math.sqrt(d)
    qh = q.astype(np.float16).astype(np.float32)
    want = textbook_attention(qh, k, v, mask, scale, 2)
    got = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=3)
    assert np.abs(got - want).max() < 1e-6 * np.abs(want).max()
    assert not got[3].any()


@pytest.mark.parametrize("n_kv,holes", [(1, []), (64, []), (65, []), (300, [(30, 130)]), (1000, [(0, 200), (640, 700)])])
def test_flash_attn_chunked_mode(ref, n_kv, holes):
    """fidelity 4 (64-position chunks with their own maxima, combined in
    order) against the f64 textbook: chunk edges, a chunk masked out in the
    middle, leading masked chunks, a single position"""
    n_q, hq, hkv, d = 2, 4, 2, 128
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_q, n_kv), np.float16)
    for a, b in holes:
        mask[:, a:b] = -np.inf
    scale = 1 / math.sqrt(d)
    qh = q.astype(np.float16).astype(np.float32)
    want = textbook_attention(qh, k, v, mask, scale, hq // hkv)
    got = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=4)
    assert np.abs(got - want).max() < 1e-6 * max(1.0, np.abs(want).max())
    two_pass = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=3)
    assert np.abs(got - two_pass).max() < 1e-6 * max(1.0, np.abs(want).max())
    # garbage (even NaN) under the mask changes nothing
    k2, v2 = k.copy(), v.copy()
    for a, b in holes:
        k2[:, a:b] = np.float16(60000)
        v2[:, a:b] = np.float16(np.nan)
    got2 = ref.flash_attn(q, k2.view(np.uint16), v2.view(np.uint16), mask.view(np.uint16), scale, fidelity=4)
    assert np.array_equal(got, got2)


@pytest.mark.parametrize("n_kv,holes", [(1, []), (64, []), (65, []), (300, [(30, 130)]), (1000, [(0, 200), (640, 700)])])
def test_flash_attn_f32_chunked_mode(ref, n_kv, holes):
    """fidelity 5 (the chunks of fidelity 4 with f32 chains inside a chunk)
    against the f64 textbook and fidelity 4; garbage under the mask changes
    nothing; a lone live position returns its V row exactly"""
    n_q, hq, hkv, d = 2, 4, 2, 128
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_q, n_kv), np.float16)
    for a, b in holes:
        mask[:, a:b] = -np.inf
    scale = 1 / math.sqrt(d)
    qh = q.astype(np.float16).astype(np.float32)
    want = textbook_attention(qh, k, v, mask, scale, hq // hkv)
    got = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=5)
    assert np.abs(got - want).max() < 2e-6 * max(1.0, np.abs(want).max())
    f4 = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, fidelity=4)
    assert np.abs(got - f4).max() < 2e-6 * max(1.0, np.abs(want).max())
    k2, v2 = k.copy(), v.copy()
    for a, b in holes:
        k2[:, a:b] = np.float16(60000)
        v2[:, a:b] = np.float16(np.nan)
    got2 = ref.flash_attn(q, k2.view(np.uint16), v2.view(np.uint16), mask.view(np.uint16), scale, fidelity=5)
    assert np.array_equal(got, got2)
    one = np.full((1, n_kv), -np.inf, np.float16)
    one[0, n_kv // 2] = 0
    lone = ref.flash_attn(q[:1], k.view(np.uint16), v.view(np.uint16), one.view(np.uint16), scale, fidelity=5)
    for h in range(hq):
        assert np.array_equal(lone[0, h], v[h // (hq // hkv), n_kv // 2].astype(np.float32))


def _round_f32(x: Fraction) -> float:
    """a rational rounded to the nearest float32 (ties to even), exactly"""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)  # below that, the subnormal quantum 2**-149
    quantum = Fraction(2) ** (e - 23)
    m = a / quantum
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(n * quantum)


def _fma32(a: float, b: float, c: float) -> float:
    return _round_f32(Fraction(a) * Fraction(b) + Fraction(c))


def test_flash_attn_f32_chunked_mode_brute_force(ref):
    """fidelity 5 bit for bit against a scalar restatement with exact
    rational fused multiply-adds (one rounding each): score chains over the
    dims in order, p*V chains and the sum of p over the live positions in
    order, the chunk combine in f64. Two chunks, masked holes in both."""
    L = ref.lib()
    n_q, hq, hkv, n_kv, d = 2, 2, 1, 70, 16
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_q, n_kv), np.float16)
    mask[0, 5:9] = -np.inf
    mask[1, 60:66] = -np.inf
    mask[1, 0] = np.float16(-1.5)
    scale = np.float32(0.3)
    got = ref.flash_attn(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), float(scale), fidelity=5)
    qh = q.astype(np.float16).astype(np.float32)
    kf, vf = k.astype(np.float32), v.astype(np.float32)
    for i in range(n_q):
        for h in range(hq):
            chunks = []
            for c0 in range(0, n_kv, 64):
                live = [j for j in range(c0, min(n_kv, c0 + 64)) if mask[i, j] != -np.inf]
                s = {}
                for j in live:
                    acc = 0.0
                    for t in range(d):
                        acc = _fma32(float(kf[0, j, t]), float(qh[i, h, t]), acc)
                    s[j] = np.float32(np.float32(acc) * scale) + np.float32(mask[i, j])
                mc = max(s.values()) if live else -np.inf
                l, a = np.float32(0), [0.0] * d
                for j in live:
                    p = np.float32(L.ref_expf_det(float(np.float32(s[j] - mc))))
                    l = np.float32(l + p)
                    a = [_fma32(float(p), float(vf[0, j, t]), a[t]) for t in range(d)]
                chunks.append((mc, l, a))
            M = max(c[0] for c in chunks)
            Ls, O = 0.0, [0.0] * d
            for mc, l, a in chunks:
                if mc == -np.inf:
                    continue
                w = np.float32(L.ref_expf_det(float(np.float32(mc - M))))
                if w == 0:
                    continue
                Ls += float(w) * float(l)
                O = [O[t] + float(w) * a[t] for t in range(d)]
            want = np.array([0.0 if Ls == 0 else O[t] / Ls for t in range(d)], np.float32)
            assert np.array_equal(got[i, h], want), (i, h)


@pytest.mark.parametrize("n_kv,holes", [(1, []), (64, []), (65, []), (300, [(30, 130)]),
                                        (1000, [(0, 200), (640, 700)])])
@pytest.mark.parametrize("prec_f32", [True, False])
def test_naive_attention_against_textbook(ref, n_kv, holes, prec_f32):
    """the unfused attention chain (MUL_MAT(K, Q) -> SOFT_MAX_EXT -> MUL_MAT of
    V^T by P, nn/decoder.rs:2154-2200) against the f64 textbook: within f32
    rounding with GGML_PREC_F32 (Q and P kept f32), within the f16 rounding
    of Q and P without it; GQA by the batch broadcast equals explicitly
    repeated K/V (what expand_attention_kv builds) bit for bit; garbage under
    the mask changes nothing; a lone live position returns its V row"""
    n_q, hq, hkv, d = 2, 4, 2, 128
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_q, n_kv), np.float16)
    for a, b in holes:
        mask[:, a:b] = -np.inf
    scale = 1 / math.sqrt(d)
    qq = q if prec_f32 else q.astype(np.float16).astype(np.float32)
    want = textbook_attention(qq, k, v, mask, scale, hq // hkv)
    got = ref.naive_attention(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), scale, prec_f32)
    bar = 2e-6 if prec_f32 else 1e-3
    assert np.abs(got - want).max() < bar * max(1.0, np.abs(want).max())
    g = hq // hkv
    kr, vr = np.repeat(k, g, axis=0), np.repeat(v, g, axis=0)
    rep = ref.naive_attention(q, kr.view(np.uint16), vr.view(np.uint16), mask.view(np.uint16), scale, prec_f32)
    assert np.array_equal(got.view(np.uint32), rep.view(np.uint32))
    k2, v2 = k.copy(), v.copy()
    for a, b in holes:
        k2[:, a:b] = np.float16(60000)
        v2[:, a:b] = np.float16(np.nan)
    got2 = ref.naive_attention(q, k2.view(np.uint16), v2.view(np.uint16), mask.view(np.uint16), scale, prec_f32)
    assert np.array_equal(got.view(np.uint32), got2.view(np.uint32))
    one = np.full((1, n_kv), -np.inf, np.float16)
    one[0, n_kv // 2] = 0
    lone = ref.naive_attention(q[:1], k.view(np.uint16), v.view(np.uint16), one.view(np.uint16), scale, prec_f32)
    for h in range(hq):
        assert np.array_equal(lone[0, h], v[h // g, n_kv // 2].astype(np.float32))


def _pairwise(xs):
    """a 64-entry list summed by the pairwise tree (level k adds neighbouring
    sums of 2^k entries), in f64"""
    xs = list(xs)
    w = 1
    while w < len(xs):
        for j in range(0, len(xs), 2 * w):
            xs[j] = xs[j] + xs[j + w]
        w *= 2
    return xs[0]


@pytest.mark.parametrize("prec_f32", [True, False])
def test_naive_attention_brute_force(ref, prec_f32):
    """the chain's fixed order, bit for bit, against a scalar restatement with
    exact rational fused multiply-adds (one rounding each): score chains over
    the dims in order, then * scale + mask; exp(s - max); the f64 sum of each
    64-position chunk by the pairwise tree, the chunk sums in order; P = e *
    (1 / sum) in f32 (rounded to f16 without GGML_PREC_F32); context chains
    over the positions in order. Two chunks, masked holes, a row whose first
    position carries a finite mask value. A planted mistake differs: with
    GGML_PREC_F32 an unfused score chain (product, then add: two roundings;
    without it the f16 operands' products are exact and the two agree), and
    without it P left unrounded."""
    L = ref.lib()
    n_q, hq, hkv, n_kv, d = 2, 2, 1, 70, 16
    q = RNG.standard_normal((n_q, hq, d)).astype(np.float32)
    k = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    v = RNG.standard_normal((hkv, n_kv, d)).astype(np.float16)
    mask = np.zeros((n_q, n_kv), np.float16)
    mask[0, 5:9] = -np.inf
    mask[1, 60:66] = -np.inf
    mask[1, 0] = np.float16(-1.5)
    scale = np.float32(0.3)
    got = ref.naive_attention(q, k.view(np.uint16), v.view(np.uint16), mask.view(np.uint16), float(scale), prec_f32)
    kf, vf = k.astype(np.float32), v.astype(np.float32)
    planted_differs = False
    for i in range(n_q):
        for h in range(hq):
            qv = q[i, h] if prec_f32 else q[i, h].astype(np.float16).astype(np.float32)
            s, s_unfused = {}, {}
            for j in range(n_kv):
                if mask[i, j] == -np.inf:
                    continue
                acc, acc2 = 0.0, np.float32(0)
                for t in range(d):
                    acc = _fma32(float(kf[0, j, t]), float(qv[t]), acc)
                    acc2 = np.float32(acc2 + np.float32(kf[0, j, t] * qv[t]))
                s[j] = np.float32(np.float32(acc) * scale) + np.float32(mask[i, j])
                s_unfused[j] = np.float32(acc2 * scale) + np.float32(mask[i, j])
            planted_differs |= any(s[j] != s_unfused[j] for j in s)
            M = max(s.values())
            e = [np.float32(L.ref_expf_det(float(np.float32(s[j] - M)))) if j in s else np.float32(0)
                 for j in range(n_kv)]
            total = 0.0
            for c0 in range(0, n_kv, 64):
                total = total + _pairwise([float(e[j]) if j < n_kv else 0.0 for j in range(c0, c0 + 64)])
            inv = np.float32(1.0 / total)
            out, out_p32 = [0.0] * d, [0.0] * d
            for j in range(n_kv):
                p = np.float32(e[j] * inv)
                if p != 0:
                    out_p32 = [_fma32(float(p), float(vf[0, j, t]), out_p32[t]) for t in range(d)]
                if not prec_f32:
                    p = np.float32(np.float16(p))
                if p == 0:
                    continue
                out = [_fma32(float(p), float(vf[0, j, t]), out[t]) for t in range(d)]
            want = np.array(out, np.float32)
            assert np.array_equal(got[i, h].view(np.uint32), want.view(np.uint32)), (i, h)
            if not prec_f32:
                planted_differs |= not np.array_equal(np.array(out_p32, np.float32), want)
    assert planted_differs


def test_whisper_cross_kv_matches_brute_force(ref):
    """the oracle's cross K/V precompute (K = Wk enc, V = Wv enc + bv, f16)
    against an f64 product of the dequantized weight with the Q8_0-quantized
    encoder states, on a reduced shape"""
    from openasr_amd import decoders as D
    shape = dict(D.WHISPER_TINY, vocab=512, n_frames=96, n_layers=1)
    w = D.WhisperWeights(seed=5, **shape)
    enc = RNG.standard_normal((shape["n_frames"], shape["d_model"])).astype(np.float32)
    r = ref.WhisperRef(w.cfg, w.pointer_table())
    r.set_encoder(enc)
    d = shape["d_model"]
    tbl = w.pointer_table()
    import ctypes as C
    nbytes = d * ref.row_size(ref.Q8_0, d)
    wk = np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(tbl[13]))
    wv = np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(tbl[14]))
    bv = np.ctypeslib.as_array((C.c_float * d).from_address(tbl[15])).astype(np.float64)
    xq = np.stack([ref.dequantize(ref.Q8_0, ref.quantize_act(ref.Q8_0, enc[f:f + 1]), d) for f in range(len(enc))])
    for wq, bias, got in ((wk, None, r.ck[0]), (wv, bv, r.cv[0])):
        W = ref.dequantize(ref.Q8_0, wq, d * d).reshape(d, d).astype(np.float64)
        want = xq.reshape(len(enc), d).astype(np.float64) @ W.T
        if bias is not None:
            want = want + bias
        g16 = got.view(np.float16).astype(np.float64)
        assert np.abs(g16 - want).max() <= 1e-3 * np.abs(want).max() + 1e-6
    w.free()


def test_erf_det_coefficients_are_the_series_rounded(ref):
    """the 64 coefficients of the deterministic erf are the Maclaurin series'
    (-1)^n / (n! (2n+1)), each the nearest double to the exact rational"""
    from fractions import Fraction
    L = ref.lib()
    for n in range(64):
        assert L.ref_erf_coef(n) == float(Fraction((-1) ** n, math.factorial(n) * (2 * n + 1))), n


def test_erf_det_within_one_ulp_of_math_erf(ref):
    """the deterministic erf (the series by Horner's rule in double) against
    math.erf rounded to f32: within one f32 ulp everywhere, equal for the vast
    majority, odd, saturating to +-1 where erf rounds there"""
    L = ref.lib()
    xs = np.concatenate([np.linspace(-5, 5, 20001), RNG.standard_normal(5000) * 2.0,
                         [0.0, -0.0, 1e-30, 3.9, 3.99, 4.0, -4.0, 1e-8]]).astype(np.float32)
    got = np.array([L.ref_erff_det(float(x)) for x in xs], np.float32)
    want = np.array([math.erf(float(x)) for x in xs], np.float32)
    d = ulp_dist(got, want)
    assert d.max() <= 1
    assert (d == 0).mean() > 0.99
    assert all(L.ref_erff_det(float(x)) == -L.ref_erff_det(float(-x)) for x in xs[:2000])
    assert L.ref_erff_det(5.0) == 1.0 and L.ref_erff_det(-7.5) == -1.0


def test_gelu_erf_and_relu_closed_forms(ref):
    L = ref.lib()
    for x in np.linspace(-6, 6, 1201).astype(np.float32):
        want = 0.5 * float(x) * (1.0 + math.erf(float(x) / math.sqrt(2.0)))
        assert abs(L.ref_gelu_erf(float(x)) - want) <= 2e-7 * max(1.0, abs(want))
        assert L.ref_relu(float(x)) == (float(x) if x > 0 else 0.0)


def pack_q3_K(d16, scales, quants):
    """a Q3_K super-block written from its published layout by an
    independent packer: scales (16 values in -32..31) coded as 6-bit values
    + 32 split into low nibbles (bytes 0..7) and high bit pairs (bytes
    8..11), quants (256 values in -4..3) split into two low bits in qs and
    the third bit in hmask (set for q >= 0)"""
    c = [s + 32 for s in scales]
    sb = bytearray(12)
    for i in range(16):
        sb[i % 8] |= (c[i] & 0xF) << (4 * (i // 8))
        sb[8 + i % 4] |= (c[i] >> 4) << (2 * (i // 4))
    hm, qs = bytearray(32), bytearray(64)
    for e, q in enumerate(quants):
        h, j, l = e // 128, (e % 128) // 32, e % 32
        u = q + 4  # 0..7: bit 2 is the hmask bit, bits 0..1 go to qs
        qs[32 * h + l] |= (u & 3) << (2 * j)
        hm[l] |= (u >> 2) << (4 * h + j)
    return bytes(hm) + bytes(qs) + bytes(sb) + np.uint16(d16).tobytes()


def test_q3_K_dequant_known_answer(ref):
    """the oracle's Q3_K decoding inverts the independent packer: every
    scale index and quant position comes back (a transposed index, a wrong
    bit of hmask or a dropped -32 / -4 offset fails)"""
    rng = np.random.default_rng(3)
    for trial in range(6):
        scales = rng.integers(-32, 32, 16).tolist()
        quants = rng.integers(-4, 4, 256).tolist()
        if trial == 0:
            scales, quants = list(range(-32, 32, 4)), [(e % 8) - 4 for e in range(256)]
        d16 = int(np.float16(0.5 + trial).view(np.uint16))
        blk = np.frombuffer(pack_q3_K(d16, scales, quants), dtype=np.uint8)
        assert blk.size == 110
        for i in range(16):
            assert ref.lib().ref_q3_K_scale(ref._p(np.ascontiguousarray(blk[96:108])), i) == scales[i]
        y = ref.dequantize(ref.Q3_K, blk, 256)
        d = np.float32(np.float16(0.5 + trial))
        want = np.array([np.float32(d * np.float32(scales[e // 16])) * np.float32(quants[e]) for e in range(256)],
                        dtype=np.float32)
        np.testing.assert_array_equal(y, want)


def test_vec_dot_q3_K_equals_f64_dot_of_dequantized(ref):
    """the Q3_K x Q8_K dot equals the f64 dot of the two dequantized rows
    (the Q8_K side dequantizes through f32 products, hence the tolerance)"""
    rng = np.random.default_rng(33)
    k = 1024
    blocks = b"".join(pack_q3_K(int(np.float16(rng.uniform(0.01, 0.1)).view(np.uint16)),
                                rng.integers(-32, 32, 16).tolist(), rng.integers(-4, 4, 256).tolist())
                      for _ in range(k // 256))
    w = np.frombuffer(blocks, dtype=np.uint8).copy()
    for t in range(4):
        x = rng.standard_normal(k).astype(np.float32)
        xq = ref.quantize_act(ref.Q8_K, x)
        got = ref.lib().ref_vec_dot_q3_K_q8_K(k, ref._p(w), ref._p(xq))
        wd = ref.dequantize(ref.Q3_K, w, k).astype(np.float64)
        xd = ref.dequantize(ref.Q8_K, xq, k).astype(np.float64)
        assert got == pytest.approx(np.dot(wd, xd), rel=2e-5, abs=2e-5)


def test_mul_mat_q3_K_brute_force(ref):
    """MUL_MAT on Q3_K weights: every column equals the per-row dot"""
    rng = np.random.default_rng(34)
    m, k, n = 5, 512, 3
    w = np.frombuffer(b"".join(pack_q3_K(int(np.float16(rng.uniform(0.01, 0.1)).view(np.uint16)),
                                         rng.integers(-32, 32, 16).tolist(), rng.integers(-4, 4, 256).tolist())
                               for _ in range(m * k // 256)), dtype=np.uint8).copy()
    x = rng.standard_normal((n, k)).astype(np.float32)
    y = ref.mul_mat(ref.Q3_K, w, m, k, x)
    rb = ref.row_size(ref.Q3_K, k)
    assert rb == k // 256 * 110
    for c in range(n):
        xq = ref.quantize_act(ref.Q8_K, x[c])
        for r in range(m):
            wr = np.ascontiguousarray(w[r * rb:(r + 1) * rb])
            assert y[c, r] == np.float32(ref.lib().ref_vec_dot_q3_K_q8_K(k, ref._p(wr), ref._p(xq)))
