"""IM2COL (the column half of ggml_conv_2d, nn/conv.rs:82-110): the oracle
pinned against convolutions computed another way, and the host constructor's
shape and op_params."""

import numpy as np
import pytest
from scipy.signal import correlate2d

from oracle import ref

RNG = np.random.default_rng(7)


def conv_scatter(x, w, s0, s1, p0, p1, d0, d1):
    """direct convolution by scattering every (input pixel, tap) product into
    the output pixel it lands on; f64"""
    n, ic, ih, iw = x.shape
    oc, _, kh, kw = w.shape
    oh = (ih + 2 * p1 - d1 * (kh - 1) - 1) // s1 + 1
    ow = (iw + 2 * p0 - d0 * (kw - 1) - 1) // s0 + 1
    y = np.zeros((n, oh, ow, oc))
    for yy in range(ih):
        for a in range(kh):
            r = yy + p1 - a * d1
            if r % s1 or not 0 <= r // s1 < oh:
                continue
            for xx in range(iw):
                for b in range(kw):
                    c = xx + p0 - b * d0
                    if c % s0 or not 0 <= c // s0 < ow:
                        continue
                    y[:, r // s1, c // s0, :] += x[:, :, yy, xx].astype(np.float64) @ w[:, :, a, b].T
    return y


@pytest.mark.parametrize("ic,ih,iw,kh,kw,s0,s1,p0,p1,d0,d1", [
    (1, 16, 12, 3, 3, 2, 2, 1, 1, 1, 1),   # the encoder stem's 3x3 stride-2 shape
    (3, 9, 11, 2, 3, 1, 2, 2, 0, 2, 1),    # every parameter different per axis
    (2, 7, 5, 3, 1, 3, 1, 0, 2, 1, 3),
])
def test_im2col_times_kernel_is_the_convolution(ic, ih, iw, kh, kw, s0, s1, p0, p1, d0, d1):
    x = RNG.standard_normal((2, ic, ih, iw)).astype(np.float32)
    w = RNG.standard_normal((4, ic, kh, kw)).astype(np.float32)
    cols = ref.im2col(x, kw, kh, s0, s1, p0, p1, d0, d1)
    y = cols.astype(np.float64) @ w.reshape(4, -1).T.astype(np.float64)
    np.testing.assert_allclose(y, conv_scatter(x, w, s0, s1, p0, p1, d0, d1), rtol=1e-12, atol=1e-12)


def test_im2col_matches_library_correlation():
    x = RNG.standard_normal((1, 2, 10, 13)).astype(np.float32)
    w = RNG.standard_normal((3, 2, 3, 3)).astype(np.float32)
    cols = ref.im2col(x, 3, 3, 1, 1, 1, 1, 1, 1)
    y = cols.astype(np.float64) @ w.reshape(3, -1).T.astype(np.float64)
    xp = np.pad(x[0].astype(np.float64), ((0, 0), (1, 1), (1, 1)))
    for o in range(3):
        want = sum(correlate2d(xp[c], w[o, c].astype(np.float64), mode="valid") for c in range(2))
        np.testing.assert_allclose(y[0, :, :, o], want, rtol=1e-12, atol=1e-12)


def test_im2col_special_cases():
    x = RNG.standard_normal((2, 5, 4, 6)).astype(np.float32)
    # a 1x1 kernel at stride 1 moves channels innermost and changes nothing else
    assert np.array_equal(ref.im2col(x, 1, 1, 1, 1, 0, 0, 1, 1), x.transpose(0, 2, 3, 1))
    # padding contributes exact zeros: with p = k-1 the corner output sees one pixel
    c = ref.im2col(x[:, :1], 2, 2, 1, 1, 1, 1, 1, 1)
    assert c.shape == (2, 5, 7, 4)
    assert np.array_equal(c[:, 0, 0], np.stack([np.zeros(2), np.zeros(2), np.zeros(2), x[:, 0, 0, 0]], 1))
    # the 1-D form is the 2-D form with one input row
    x1 = x[:, :, 0, :]
    assert np.array_equal(ref.im2col(x1, 3, 0, 2, 0, 1, 0, 1, 0, is_2d=False),
                          ref.im2col(x1[:, :, None, :], 3, 1, 2, 1, 1, 0, 1, 1)[:, 0])


def test_host_im2col_shapes_and_params(ggml):
    G = ggml.Graph()
    K = G.new(ggml.F16, 3, 3, 4, 8)        # [KW, KH, IC, OC]
    X = G.new(ggml.F32, 100, 64, 4, 2)     # [IW, IH, IC, N]
    T = G.lib.ggml_im2col(G.ctx, K, X, 2, 2, 1, 1, 1, 1, True, ggml.F16)
    t = ggml.tensor(T)
    assert list(t.ne) == [36, 50, 32, 2] and t.type == ggml.F16
    assert list(t.op_params[:7]) == [2, 2, 1, 1, 1, 1, 1]
    K1 = G.new(ggml.F32, 3, 4, 8)           # [K, IC, OC]
    X1 = G.new(ggml.F32, 50, 4, 3)          # [IW, IC, N]
    t1 = ggml.tensor(G.lib.ggml_im2col(G.ctx, K1, X1, 1, 0, 1, 0, 1, 0, False, ggml.F32))
    assert list(t1.ne) == [12, 50, 3, 1] and t1.type == ggml.F32
    G.free()
