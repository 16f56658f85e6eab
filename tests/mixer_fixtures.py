"""Restated procedural fixtures of the reference's operator checks (test data).

  conv_fixture    crates/mixers/src/convolution_checks.rs:57-146
  norm_fixture    crates/mixers/src/normalization_checks.rs:66-131
  decay_fixture   crates/mixers/src/normalization_checks.rs:243-275

Values follow the same formulas and storage layouts ("strided" cases store
the tensor with swapped physical axes, as the reference does); expected values
are always computed by the oracle from these same inputs, so a last-ulp
difference between numpy's and Rust's sin/cos is immaterial.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32

CONV_CASES = [(1, 3, 4), (2, 35, 4), (7, 3, 4), (17, 128, 4), (19, 256, 4), (7, 35, 1)]
NORM_WIDTHS = [3, 32, 35, 64, 256]
NORM_MODES = [(0, 1e-6), (1, 1e-6), (1, 1e-5), (2, 1e-5)]
PADDED_TOKENS = (0, 3, 6, 9, 13)  # of the 2 x 7 (batch, time) grid


def conv_fixture(t, c, width, zero, strided, b=2):
    """(x [b,t,c], w [width,c], valid [b,t], docs [b,t], upstream [b,t,c]);
    each a numpy view whose physical layout matches the reference case."""
    i = np.arange(b * t * c)
    src = np.zeros(b * t * c, F32) if zero else np.sin((i * 17 + 3) * 0.013).astype(F32)
    x = src.reshape(b, c, t).transpose(0, 2, 1) if strided else src.reshape(b, t, c)
    iw = np.arange(width * c)
    wv = np.where(iw % 7 == 0, F32(0), np.sin(F32(iw + 3) * F32(0.17)) * F32(0.1)).astype(F32)
    w = wv.reshape(c, width).T if strided else wv.reshape(width, c)
    im = np.arange(b * t)
    valid_v = np.where((im % 7 == 3) | (im % t == t - 1), F32(0), F32(1)).astype(F32)
    reset_v = np.where((im % t == 0) | (im % t == 2) | (im % t == 5), F32(1), F32(0)).astype(F32)
    meta = (lambda v: v.reshape(t, b).T) if strided else (lambda v: v.reshape(b, t))
    valid, reset = meta(valid_v), meta(reset_v)
    docs = np.cumsum(valid * reset, axis=1).astype(F32)
    if strided:
        docs = np.ascontiguousarray(docs.T).T  # genuinely strided storage
    iu = np.arange(b * t * c)
    up_v = np.where(zero | (iu % 13 == 0), F32(0),
                    np.cos((iu * 19 + 1) * 0.031).astype(F32)).astype(F32)
    up = up_v.reshape(b, c, t).transpose(0, 2, 1) if strided else up_v.reshape(b, t, c)
    return x, w, valid, docs, up


def _strided4(v, width):
    """Flat data stored as [b, w, h, t] and viewed as [b, t, h, w] (2, 7, 2, width)."""
    return v.reshape(2, width, 2, 7).transpose(0, 3, 2, 1)


def token_mask():
    m = np.ones(14, F32)
    m[list(PADDED_TOKENS)] = 0
    return m.reshape(2, 7)


def norm_fixture(width, zero):
    """(x, gate, upstream, weight, mask[2,7]) with x, gate, upstream [2,7,2,width]."""
    n = 2 * 7 * 2 * width
    i = np.arange(n)
    token = i // (width * 2 * 7) * 7 + i % 7
    xv = np.where(zero | np.isin(token, PADDED_TOKENS), F32(0),
                  np.sin((i * 17 + 3) * 0.013).astype(F32)).astype(F32)
    gv = np.cos(F32(i * 7) * F32(0.07)).astype(F32)
    gv = np.where(i % 11 == 0, F32(-30), np.where(i % 11 == 1, F32(30),
                                                 np.where(i % 11 == 2, F32(0), gv))).astype(F32)
    uv = np.where(i % 13 == 0, F32(0), np.cos((i * 19 + 1) * 0.031).astype(F32)).astype(F32)
    iw = np.arange(width)
    w = np.where(iw % 7 == 0, F32(0), np.sin(F32(iw + 3) * F32(0.17))).astype(F32)
    return _strided4(xv, width), _strided4(gv, width), _strided4(uv, width), w, token_mask()


def decay_fixture(zero):
    """(x, bias [6], scale [2], upstream, mask[2,7]) with x, upstream [2,7,2,3]."""
    n = 84
    i = np.arange(n)
    base = np.sin(F32(i * 3) * F32(0.11)).astype(F32)
    xv = np.where(i % 9 == 0, F32(-40), np.where(i % 9 == 1, F32(40),
                                                 np.where(i % 9 == 2, F32(20), base))).astype(F32)
    if zero:
        xv = np.zeros(n, F32)
    bias = np.array([0., 0.3, -4., 0., -0.7, -3.], F32)
    scale = np.array([-0.2, 0.4], F32)
    uv = np.where(i % 5 == 0, F32(0), np.cos(F32(i * 7) * F32(0.03))).astype(F32)
    return _strided4(xv, 3), bias, scale, _strided4(uv, 3), token_mask()
