"""Pinning of the mixer-operator oracle (oracle/mixer_oracle.py), CPU only.

Every VJP is checked against f64 central differences along random directions;
the forwards against closed forms and the reference checks' structure
(crates/mixers/src/convolution_checks.rs, normalization_checks.rs).
"""
import numpy as np
import pytest

import mixer_fixtures as mf
from oracle import mixer_oracle as mo


def _fd(f, x, d, h=1e-6):
    return (f(x + h * d) - f(x - h * d)) / (2 * h)


def _conv_problem(rng, B=2, T=9, C=5, W=4):
    x = rng.normal(size=(B, T, C))
    w = rng.normal(size=(W, C)) * 0.5
    valid = np.ones((B, T))
    valid[0, 4] = 0
    valid[1, T - 1] = 0
    reset = np.zeros((B, T))
    reset[:, 0] = 1
    reset[0, 6] = 1
    reset[1, 3] = 1
    docs = np.cumsum(valid * reset, axis=1)
    return x, w, valid, docs


@pytest.mark.parametrize("silu", [False, True])
def test_conv_vjp_central_differences(silu):
    rng = np.random.default_rng(0)
    x, w, valid, docs = _conv_problem(rng)
    dy = rng.normal(size=x.shape)
    dx, dw = mo.causal_conv_vjp(x, w, valid, docs, dy, silu)
    for _ in range(3):
        u = rng.normal(size=x.shape)
        num = _fd(lambda z: (mo.causal_conv(z, w, valid, docs, silu) * dy).sum(), x, u)
        assert abs(num - (dx * u).sum()) < 1e-7 * (1 + abs(num))
        v = rng.normal(size=w.shape)
        num = _fd(lambda z: (mo.causal_conv(x, z, valid, docs, silu) * dy).sum(), w, v)
        assert abs(num - (dw * v).sum()) < 1e-7 * (1 + abs(num))


def test_conv_closed_forms():
    rng = np.random.default_rng(1)
    x, w, valid, docs = _conv_problem(rng, W=1)
    # one tap: a masked per-channel scale
    np.testing.assert_allclose(mo.causal_conv(x, w, valid, docs), x * w[0] * valid[..., None],
                               rtol=0, atol=1e-15)
    # lags never reach across a document start or from/to an invalid token
    x, w, valid, docs = _conv_problem(rng, W=4)
    y = mo.causal_conv(x, w, valid, docs)
    x2 = x.copy()
    x2[0, :6] += 1.0  # everything before the reset at t = 6 (batch 0)
    y2 = mo.causal_conv(x2, w, valid, docs)
    np.testing.assert_array_equal(y[0, 6:], y2[0, 6:])
    assert np.all(y[0, 4] == 0) and np.all(y[1, -1] == 0)


def test_conv_reference_fixture_structure():
    x, w, valid, docs, up = mf.conv_fixture(17, 128, 4, False, True)
    assert x.shape == (2, 17, 128) and not x.flags.c_contiguous
    assert w.shape == (4, 128) and not w.flags.c_contiguous
    assert np.all(np.ascontiguousarray(w.T).reshape(-1)[::7] == 0)  # every 7th stored weight
    assert docs.shape == (2, 17) and np.all(np.diff(docs, axis=1) >= 0)


@pytest.mark.parametrize("mode,eps", mf.NORM_MODES)
def test_norm_vjp_central_differences(mode, eps):
    rng = np.random.default_rng(2 + mode)
    x = rng.normal(size=(2, 3, 2, 7))
    gate = rng.normal(size=x.shape) * 2
    weight = rng.normal(size=7)
    dy = rng.normal(size=x.shape)
    dx, dg, dw = mo.row_norm_vjp(x, weight, gate, mode, eps, dy)
    f = lambda xx, gg, ww: (mo.row_norm(xx, ww, gg, mode, eps)[0] * dy).sum()  # noqa: E731
    for _ in range(3):
        u = rng.normal(size=x.shape)
        num = _fd(lambda z: f(z, gate, weight), x, u)
        assert abs(num - (dx * u).sum()) < 1e-6 * (1 + abs(num))
        if mode == 2:
            num = _fd(lambda z: f(x, z, weight), gate, u)
            assert abs(num - (dg * u).sum()) < 1e-6 * (1 + abs(num))
        if mode >= 1:
            v = rng.normal(size=7)
            num = _fd(lambda z: f(x, gate, z), weight, v)
            assert abs(num - (dw * v).sum()) < 1e-6 * (1 + abs(num))


def test_norm_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.normal(size=(1, 2, 3, 16)) * 3
    y, inv = mo.row_norm(x, None, None, 0, 1e-6)
    n = np.sqrt((x * x).sum(-1))
    np.testing.assert_allclose(np.sqrt((y * y).sum(-1)), n / np.sqrt(n * n + 1e-6), rtol=1e-14)
    w = rng.normal(size=16)
    y1, inv1 = mo.row_norm(x, w, None, 1, 1e-5)
    np.testing.assert_allclose(inv1, 1 / np.sqrt((x * x).mean(-1) + 1e-5), rtol=1e-14)
    np.testing.assert_allclose(y1, x * inv1[..., None] * w, rtol=1e-14)
    g = np.full(x.shape, 30.0)  # sigmoid(30) = 1 - 9e-14: gating is the identity
    y2, _ = mo.row_norm(x, w, g, 2, 1e-5)
    np.testing.assert_allclose(y2, y1, rtol=1e-12)


def test_decay_vjp_and_closed_forms():
    rng = np.random.default_rng(6)
    x = rng.normal(size=(2, 3, 2, 4)) * 3
    x[0, 0, 0, 0] = 25.0  # the softplus-identity branch
    bias = rng.normal(size=8)
    scale = rng.normal(size=2) * 0.3
    dy = rng.normal(size=x.shape)
    dx, db, ds = mo.decay_vjp(x, bias, scale, dy)
    f = lambda xx, bb, ss: (mo.decay(xx, bb, ss) * dy).sum()  # noqa: E731
    u = rng.normal(size=x.shape)
    u[0, 0, 0, 0] = 0.0  # keep the probe off the threshold
    num = _fd(lambda z: f(z, bias, scale), x, u)
    assert abs(num - (dx * u).sum()) < 1e-6 * (1 + abs(num))
    v = rng.normal(size=8)
    num = _fd(lambda z: f(x, z, scale), bias, v)
    assert abs(num - (db * v).sum()) < 1e-6 * (1 + abs(num))
    s = rng.normal(size=2)
    num = _fd(lambda z: f(x, bias, z), scale, s)
    assert abs(num - (ds * s).sum()) < 1e-6 * (1 + abs(num))
    # alpha = exp(-ln 2) = 1/2 at x + bias = 0, scale = 0; softplus(z) = z above 20
    half = mo.decay(np.zeros((1, 1, 1, 1)), np.zeros(1), np.zeros(1))
    assert abs(half[0, 0, 0, 0] - 0.5) < 1e-15
    big = mo.decay(np.full((1, 1, 1, 1), 30.0), np.zeros(1), np.zeros(1))
    assert abs(big[0, 0, 0, 0] - np.exp(-30.0)) < 1e-25
