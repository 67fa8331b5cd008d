"""Pins of the 2-D restatement (oracle/cnn_oracle.py): direct loops, closed forms and
independent library routines, so a transposed kernel, a shifted tap or a wrong stride in the
oracle fails here before it judges the device."""
import numpy as np
from scipy.signal import correlate2d

from oracle import cnn_oracle as co


def _f16(rng, shape, s=1.0):
    return (rng.standard_normal(shape) * s).astype(np.float16)


def test_conv2d_matches_scipy_correlate_and_loops():
    rng = np.random.default_rng(0)
    x = _f16(rng, (2, 3, 9, 11))
    w = _f16(rng, (4, 3, 3, 3), 0.3)
    b = _f16(rng, 4, 0.1)
    y = co.conv2d_f64(x, w, b, 1, 1)
    for f in range(2):
        for o in range(4):
            ref = sum(correlate2d(x[f, i].astype(np.float64), w[o, i].astype(np.float64),
                                  mode="same") for i in range(3)) + float(b[o])
            assert np.allclose(y[f, o], ref, rtol=1e-12, atol=1e-12)
    # stride 2: every second output of the stride-1 result
    y2 = co.conv2d_f64(x, w, b, 2, 1)
    assert np.allclose(y2, y[:, :, ::2, ::2], rtol=1e-12, atol=1e-12)
    # 1x1: a channel matmul
    w1 = _f16(rng, (5, 3, 1, 1))
    y1 = co.conv2d_f64(x, w1, None, 1, 0)
    assert np.allclose(y1, np.einsum("oc,fchw->fohw", w1[:, :, 0, 0].astype(np.float64),
                                     x.astype(np.float64)))
    # one output pixel by hand (corner: zero padding on two sides)
    v = sum(float(w[1, i, ky, kx]) * float(x[0, i, ky - 1, kx - 1])
            for i in range(3) for ky in range(1, 3) for kx in range(1, 3)) + float(b[1])
    assert abs(y[0, 1, 0, 0] - v) < 1e-12


def test_residual_and_activations():
    rng = np.random.default_rng(1)
    x = _f16(rng, (1, 2, 4, 4))
    w = _f16(rng, (2, 2, 1, 1))
    r = _f16(rng, (1, 2, 4, 4))
    base = co.conv2d_f64(x, w, None, 1, 0)
    assert np.allclose(co.conv2d_f64(x, w, None, 1, 0, "relu", r),
                       np.maximum(base, 0) + r.astype(np.float64))
    assert abs(co.act(np.array([0.0]), "sigmoid")[0] - 0.5) < 1e-15
    assert abs(co.act(np.array([1.0]), "gelu")[0] - 0.8413447460685429) < 1e-12


def test_pools_and_upsample():
    x = np.arange(2 * 1 * 4 * 6, dtype=np.float32).reshape(2, 1, 4, 6).astype(np.float16)
    m2 = co.maxpool2(x)
    assert m2.shape == (2, 1, 2, 3) and m2[0, 0, 0, 0] == x[0, 0, 1, 1] and m2[1, 0, 1, 2] == x[1, 0, 3, 5]
    m5 = co.maxpool5(x)
    # increasing ramp: the max of the clipped window is its bottom-right corner
    assert m5[0, 0, 0, 0] == x[0, 0, 2, 2] and m5[0, 0, 3, 5] == x[0, 0, 3, 5]
    assert m5[0, 0, 1, 3] == x[0, 0, 3, 5]
    u = co.upsample2(x)
    assert u.shape == (2, 1, 8, 12) and u[1, 0, 5, 7] == x[1, 0, 2, 3]


def test_upconv_is_transposed_conv():
    rng = np.random.default_rng(2)
    x = _f16(rng, (1, 3, 3, 4))
    w = _f16(rng, (2, 3, 2, 2))
    b = _f16(rng, 2)
    y = co.upconv2x2_f64(x, w, b)
    # scatter form: each input pixel adds w[:, i] * x[i] to its 2x2 output block
    ref = np.zeros((1, 2, 6, 8))
    for i in range(3):
        for yy in range(3):
            for xx in range(4):
                ref[0, :, 2 * yy:2 * yy + 2, 2 * xx:2 * xx + 2] += (
                    w[:, i].astype(np.float64) * float(x[0, i, yy, xx]))
    ref += b.astype(np.float64)[None, :, None, None]
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_layout_modes():
    a = co.Layout2D(8, 64, 2)
    assert (a.W_pad, a.single_stride, a.channel_stride) == (72, 10 * 72, 2 * 720)
    off = a.offsets(3)
    assert off[1, 2, 0, 0] == 2 * 1440 + 720 + 72 + 4
    m = co.Layout2D(5, 30)
    assert m.W_pad == 34
    tiles = (5 * 34 + 63) // 64
    assert m.single_stride == (2 * 34 + tiles * 64 + 63) & ~63
    o = m.offsets(1)
    assert o[0, 0, 4, 29] == 5 * 34 + 4 + 29  # last pixel: row H, column 4 + W - 1
    assert len(np.unique(o)) == o.size


def test_layout_token64_interleaved():
    """64-frame interleaved layout: pixel-major, 64 frames contiguous, blocks of 64 frames
    64 * single_stride apart; every pixel element distinct and inside the channel stride."""
    for H, W in ((6, 10), (8, 64)):
        L = co.Layout2D(H, W, 128, tok64=True)
        off = L.offsets(3)  # [F][C][H][W]
        assert off[0, 0, 0, 0] == (L.W_pad + 1) * 64
        assert off[63, 0, 0, 0] - off[0, 0, 0, 0] == 63
        assert off[0, 0, 0, 1] - off[0, 0, 0, 0] == 64
        assert off[0, 0, 1, 0] - off[0, 0, 0, 0] == 64 * L.W_pad
        assert off[64, 0, 0, 0] - off[0, 0, 0, 0] == 64 * L.single_stride
        assert off[0, 1, 0, 0] - off[0, 0, 0, 0] == L.channel_stride == 128 * L.single_stride
        assert len(np.unique(off)) == off.size
        assert off[:, 0].max() < L.channel_stride
