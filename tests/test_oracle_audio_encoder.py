"""Pins of the audio encoder's checker (oracle/audio_encoder.py), the numpy
restatement the device encoder is compared with, on the CPU.

1. Against an independent f64 textbook encoder written from the reference
   graph (models/qwen/audio_encoder.rs:480-672, nn/encoder.rs:575-870):
   direct 3x3 stride-2 convolutions over zero-padded 100-frame chunks,
   channel-major features after the stem's permute, per-chunk sinusoidal
   positions, pre-norm blocks with full attention, ln_post and the two output
   projections. With F32 projections the checker agrees within the f16
   rounding of the attention's operands (~1e-5 of the largest output); each
   planted mistake (post-norm blocks, positions counted over the whole input
   instead of per chunk, frequency-major features, a partial chunk not
   padded) moves it by far more.
2. Identities the checker holds bit for bit: with every block's attention
   output and FFN down projections zeroed the encoder equals the encoder
   with no blocks (pre-norm residuals add an exact zero); two identical
   chunks give identical rows (positions restart per chunk, attention is
   full).
"""

import types

import numpy as np
import pytest
from scipy.special import erf

from openasr_amd import decoders as D
from openasr_amd import ggml as g

SMALL = dict(n_mels=32, conv_channels=32, d_model=256, n_heads=4, n_layers=2, ffn=512, out_dim=96)


def _vec(w, layer, kind):
    return w.array(layer, kind).view(np.float32).astype(np.float64)


def _mat(w, layer, kind, rows, k):
    return w.array(layer, kind).view(np.float32).reshape(rows, k).astype(np.float64)


def _gelu(x):
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def _ln(x, wv, bv, eps=1e-5):
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * wv + bv


def _conv(x, kern, bias):
    """x [IC, H, W], kern [OC, IC, 3, 3]: stride 2, padding 1, then + bias"""
    ic, h, w = x.shape
    oh, ow = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    xp = np.zeros((ic, h + 2, w + 2))
    xp[:, 1:h + 1, 1:w + 1] = x
    out = np.zeros((kern.shape[0], oh, ow))
    for kh in range(3):
        for kw in range(3):
            patch = xp[:, kh:kh + 2 * oh:2, kw:kw + 2 * ow:2]
            out += np.einsum("oc,chw->ohw", kern[:, :, kh, kw], patch)
    return out + bias[:, None, None]


def textbook_encode(w, mel, mistake=None):
    c = w.cfg
    n_mels, n_frames = mel.shape
    chunks = -(-n_frames // 100)
    d, C = c.d_model, c.conv_channels
    rows_all = []
    for ch in range(chunks):
        seg = mel[:, ch * 100:(ch + 1) * 100].astype(np.float64)
        if mistake != "no_padding":
            seg = np.pad(seg, ((0, 0), (0, 100 - seg.shape[1])))
        x = seg[None]  # [1, mel (H), frames (W)]
        ic = 1
        for kk, kb in ((D.QA_CONV1_W, D.QA_CONV1_B), (D.QA_CONV2_W, D.QA_CONV2_B), (D.QA_CONV3_W, D.QA_CONV3_B)):
            kern = _vec(w, -1, kk).reshape(C, ic, 3, 3)
            x = _gelu(_conv(x, kern, _vec(w, -1, kb)))
            ic = C
        oc, fb, tt = x.shape  # channels, frequency bins, frames
        if mistake == "freq_major":
            feats = x.transpose(2, 1, 0).reshape(tt, fb * oc)
        else:
            feats = x.transpose(2, 0, 1).reshape(tt, oc * fb)
        rows_all.append(feats)
    x = np.concatenate(rows_all)
    wco = _mat(w, -1, D.QA_CONV_OUT, d, C * ((((n_mels - 1) // 2 + 1 - 1) // 2 + 1 - 1) // 2 + 1))
    x = x @ wco.T + _vec(w, -1, D.QA_CONV_OUT_B)
    inv = _vec(w, -1, D.QA_INV_TIMESCALES)
    per_chunk = x.shape[0] // chunks
    t = np.arange(x.shape[0]) if mistake == "global_positions" else np.arange(x.shape[0]) % per_chunk
    ang = t[:, None] * inv[None, :]
    x = x + np.concatenate([np.sin(ang), np.cos(ang)], axis=1)
    hd = d // c.n_heads
    for layer in range(c.n_layers):
        def lin(kind, bias, r, k, z):
            return z @ _mat(w, layer, kind, r, k).T + _vec(w, layer, bias)

        def attn(z):
            q = lin(D.QA_Q, D.QA_Q_B, d, d, z)
            k = lin(D.QA_K, D.QA_K_B, d, d, z)
            v = lin(D.QA_V, D.QA_V_B, d, d, z)
            out = np.zeros_like(q)
            for h in range(c.n_heads):
                sl = slice(h * hd, (h + 1) * hd)
                s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                out[:, sl] = (p / p.sum(axis=1, keepdims=True)) @ v[:, sl]
            return lin(D.QA_O, D.QA_O_B, d, d, out)

        def ffn(z):
            return lin(D.QA_DOWN, D.QA_DOWN_B, d, c.ffn, _gelu(lin(D.QA_UP, D.QA_UP_B, c.ffn, d, z)))

        n1 = (_vec(w, layer, D.QA_ATTN_NORM_W), _vec(w, layer, D.QA_ATTN_NORM_B))
        n2 = (_vec(w, layer, D.QA_FFN_NORM_W), _vec(w, layer, D.QA_FFN_NORM_B))
        if mistake == "post_norm":
            x = _ln(x + attn(x), *n1)
            x = _ln(x + ffn(x), *n2)
        else:
            x = x + attn(_ln(x, *n1))
            x = x + ffn(_ln(x, *n2))
    x = _ln(x, _vec(w, -1, D.QA_LN_POST_W), _vec(w, -1, D.QA_LN_POST_B))
    x = _gelu(x @ _mat(w, -1, D.QA_PROJ1, d, d).T + _vec(w, -1, D.QA_PROJ1_B))
    return x @ _mat(w, -1, D.QA_PROJ2, c.out_dim, d).T + _vec(w, -1, D.QA_PROJ2_B)


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


@pytest.fixture(scope="module")
def w32():
    w = D.QwenAudioWeights(g.F32, seed=31, **SMALL)
    yield w
    w.free()


def mel_input(n_frames, seed):
    return np.random.default_rng(seed).standard_normal((SMALL["n_mels"], n_frames)).astype(np.float32)


def test_checker_against_textbook_and_planted_mistakes(w32):
    """the checker within 1e-4 of the textbook encoder (three chunks, the
    last one partial; what is left is the f16 rounding of the attention's
    operands); every planted wiring mistake moves the textbook result by more
    than 5e-2, five hundred times that"""
    from oracle import audio_encoder as RA
    mel = mel_input(250, 5)
    want = textbook_encode(w32, mel)
    got = RA.encode(w32, mel)
    err = rel(got, want)
    print(f"checker vs textbook: {err:.2e}")
    assert err < 1e-4
    for mistake in ("post_norm", "global_positions", "freq_major", "no_padding"):
        if mistake == "no_padding":
            bad = textbook_encode(w32, mel, mistake)
            moved = rel(bad[:bad.shape[0]], want[:bad.shape[0]]) if bad.shape == want.shape else 1.0
        else:
            moved = rel(textbook_encode(w32, mel, mistake), want)
        print(f"  planted {mistake}: moves the result by {moved:.2e}")
        assert moved > 5e-2, mistake


def test_checker_zeroed_branches_equal_no_blocks(w32):
    """zero attention output and FFN down projections (weights and biases) in
    every block: the checker's encoder equals its encoder with no blocks, bit
    for bit (pre-norm residuals add an exact +0)"""
    from oracle import audio_encoder as RA
    zero = {D.QA_O, D.QA_O_B, D.QA_DOWN, D.QA_DOWN_B}

    class Zeroed:
        cfg = w32.cfg

        @staticmethod
        def array(layer, kind):
            a = w32.array(layer, kind)
            return np.zeros_like(a) if layer >= 0 and kind in zero else a

    cfg0 = types.SimpleNamespace(**{f: getattr(w32.cfg, f) for f in
                                    ("n_mels", "conv_channels", "d_model", "n_heads", "ffn", "out_dim", "wtype")},
                                 n_layers=0)

    class NoBlocks:
        cfg = cfg0

        @staticmethod
        def array(layer, kind):
            return w32.array(layer, kind)

    mel = mel_input(230, 6)
    a = RA.encode(Zeroed, mel)
    b = RA.encode(NoBlocks, mel)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert not np.array_equal(a, RA.encode(w32, mel))


def test_checker_identical_chunks_give_identical_rows(w32):
    """two identical 100-frame chunks: their 13 rows each come out equal bit
    for bit (positions restart per chunk, attention is over every row); the
    textbook with positions counted over the whole input does not"""
    from oracle import audio_encoder as RA
    m = mel_input(100, 7)
    mel = np.concatenate([m, m], axis=1)
    out = RA.encode(w32, mel)
    assert out.shape[0] == 26
    assert np.array_equal(out[:13].view(np.uint32), out[13:].view(np.uint32))
    bad = textbook_encode(w32, mel, "global_positions")
    assert rel(bad[:13], bad[13:]) > 1e-2
