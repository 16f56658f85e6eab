"""f64 restatement of the GDN mixer's prologue/epilogue operators.

TEST INFRASTRUCTURE ONLY: the checker for the HIP operators in
delta-block-lm_amd/csrc/gdn2_mixer.hip.  Nothing in the product imports it.

What it restates (read as text from the reference, never executed):
  causal_conv / _vjp   crates/mixers/src/convolution_checks.rs:156-180 (scalar-f64
                       forward and VJP), semantics of crates/kernels/src/conv.rs:11-104
                       and crates/mixers/src/lib.rs:696-725
  row_norm / _vjp      crates/mixers/src/normalization_checks.rs:137-172 (scalar-f64
                       L2 / RMS / gated RMS and VJPs), crates/kernels/src/norm.rs
  decay / _vjp         crates/mixers/src/normalization_checks.rs:276-291, with the
                       softplus threshold of crates/kernels/src/decay.rs:13-19
The optional SiLU after the convolution is the mixer's (lib.rs:463-466).

Pinned by tests/test_mixer_oracle.py: f64 central differences of every VJP,
closed forms (a one-tap convolution is a masked channel scale; the L2 norm of
a row has unit length; decay at x + bias = 0 and scale = 0 is 1/2), and the
reference fixtures' structural assertions.
"""
from __future__ import annotations

import numpy as np


def _d(x):
    return np.asarray(x, dtype=np.float64)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def conv_mask(valid, docs, b, s, d):
    return valid[b, s] * valid[b, d] if docs[b, s] == docs[b, d] else 0.0


def causal_conv(x, w, valid, docs, silu=False):
    """y[b,t,c] = sum_{l<taps, l<=t} x[b,t-l,c] w[l,c] m(b,t-l,t) (then SiLU)."""
    x, w, valid, docs = map(_d, (x, w, valid, docs))
    B, T, C = x.shape
    p = np.zeros((B, T, C))
    for b in range(B):
        for t in range(T):
            for lag in range(min(w.shape[0], t + 1)):
                m = conv_mask(valid, docs, b, t - lag, t)
                if m != 0.0:
                    p[b, t] += x[b, t - lag] * w[lag] * m
    return p * _sigmoid(p) if silu else p


def causal_conv_vjp(x, w, valid, docs, dy, silu=False):
    x, w, valid, docs, dy = map(_d, (x, w, valid, docs, dy))
    B, T, C = x.shape
    if silu:
        p = causal_conv(x, w, valid, docs, silu=False)
        s = _sigmoid(p)
        dy = dy * s * (1.0 + p * (1.0 - s))
    dx = np.zeros_like(x)
    dw = np.zeros_like(w)
    for b in range(B):
        for t in range(T):
            for lag in range(min(w.shape[0], t + 1)):
                m = conv_mask(valid, docs, b, t - lag, t)
                if m != 0.0:
                    dx[b, t - lag] += dy[b, t] * w[lag] * m
                    dw[lag] += dy[b, t] * x[b, t - lag] * m
    return dx, dw


def row_norm(x, weight, gate, mode, eps):
    """Rows over the last axis.  mode 0: x / sqrt(sum x^2 + eps); mode 1:
    w x / sqrt(mean x^2 + eps); mode 2: the same of z = x sigmoid(gate).
    Returns (y, inverse)."""
    x = _d(x)
    z = x * _sigmoid(_d(gate)) if mode == 2 else x
    div = 1.0 if mode == 0 else x.shape[-1]
    inv = 1.0 / np.sqrt((z * z).sum(-1, keepdims=True) / div + eps)
    y = z * inv
    if mode != 0:
        y = y * _d(weight)
    return y, inv[..., 0]


def row_norm_vjp(x, weight, gate, mode, eps, dy):
    """(dx, dgate, dweight) of sum(y * dy)."""
    x, dy = _d(x), _d(dy)
    s = _sigmoid(_d(gate)) if mode == 2 else np.ones_like(x)
    z = x * s
    div = 1.0 if mode == 0 else x.shape[-1]
    inv = 1.0 / np.sqrt((z * z).sum(-1, keepdims=True) / div + eps)
    w = _d(weight) if mode != 0 else np.ones(x.shape[-1])
    u = dy * w
    dot = (u * z).sum(-1, keepdims=True)
    dz = (u - z * dot * inv * inv / div) * inv
    dx = dz * s
    dgate = dz * z * (1.0 - s) if mode == 2 else None
    dweight = (dy * z * inv).reshape(-1, x.shape[-1]).sum(0) if mode != 0 else None
    return dx, dgate, dweight


def _softplus20(z):
    return np.where(z > 20.0, z, np.log1p(np.exp(np.minimum(z, 20.0))))


def decay(x, bias, scale):
    """alpha = exp(-exp(scale[h]) softplus(x + bias[h, k])) for x [B, T, H, K]."""
    x = _d(x)
    H, K = x.shape[2], x.shape[3]
    z = x + _d(bias).reshape(H, K)
    return np.exp(-_softplus20(z) * np.exp(_d(scale))[:, None])


def decay_vjp(x, bias, scale, dy):
    """(dx, dbias [H*K], dscale [H]) of sum(alpha * dy)."""
    x, dy = _d(x), _d(dy)
    H, K = x.shape[2], x.shape[3]
    z = x + _d(bias).reshape(H, K)
    sp = _softplus20(z)
    es = np.exp(_d(scale))[:, None]
    alpha = np.exp(-sp * es)
    deriv = np.where(z > 20.0, 1.0, _sigmoid(z))
    g = -dy * alpha * es
    dx = g * deriv
    dbias = dx.reshape(-1, H * K).sum(0)
    dscale = (g * sp).reshape(-1, H, K).sum((0, 2))
    return dx, dbias, dscale
