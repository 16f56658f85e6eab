"""Restatement of the training step's loss and update operators.

TEST INFRASTRUCTURE ONLY: the checker for the HIP operators in
delta-block-lm_amd/csrc/gdn2_train.hip.  Nothing in the product imports it.

What it restates (read as text from the reference, never executed):
  cross_entropy_rows / _vjp   crates/kernels/src/cross_entropy.rs:7-60 (row loss
                              (max - x[label]) + ln sum exp(x - max)) and :62-83
                              (gradient (softmax - onehot) * upstream), in f64
  adamw_f32                   crates/kernels/src/update.rs:46-82 (element update) and
                              :116-199 (per-tensor clipping coefficient, bias
                              corrections 1 - 0.9^t, 1 - 0.999^t by f32 powi, decay
                              factor 1 - lr*wd in f64), every operation rounded to
                              f32 in the reference's order
Pinned by tests/test_train_oracle.py: cross entropy against scipy's logsumexp,
the closed form ln(width) of constant rows and f64 central differences of the
VJP; AdamW against torch.optim.AdamW in float64 (same update, other rounding)
with per-tensor clip_grad_norm_, and the first-step closed form.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def cross_entropy_rows(x, target):
    """x [rows, width], target [rows] int -> (loss [rows], stats [rows, 2]) in f64."""
    x = np.asarray(x, dtype=np.float64)
    m = x.max(axis=1)
    s = np.log(np.exp(x - m[:, None]).sum(axis=1))
    loss = (m - x[np.arange(x.shape[0]), target]) + s
    return loss, np.stack([m, s], axis=1)


def cross_entropy_rows_vjp(x, target, upstream):
    """d(sum_r upstream[r] loss[r]) / dx."""
    x = np.asarray(x, dtype=np.float64)
    _, st = cross_entropy_rows(x, target)
    p = np.exp((x - st[:, :1]) - st[:, 1:])
    p[np.arange(x.shape[0]), target] -= 1.0
    return p * np.asarray(upstream, dtype=np.float64)[:, None]


def powi_f32(a, b):
    """Binary powering in f32 (compiler-rt's __powisf2, which Rust's f32::powi
    calls for a run-time exponent)."""
    a, r = F32(a), F32(1)
    while True:
        if b & 1:
            r = F32(r * a)
        b //= 2
        if b == 0:
            break
        a = F32(a * a)
    return r


def adamw_f32(param, grad, first, second, time, lr, weight_decay, clip, square=None):
    """One step of the reference's AdamW on one tensor, all f32.  first/second
    None on the first step.  square: the gradient's sum of squares (f32); by
    default np.sum in f64 rounded to f32.  Returns (param, first, second)."""
    p = np.asarray(param, F32)
    g = np.asarray(grad, F32)
    if square is None:
        square = F32(np.sum(g.astype(np.float64) ** 2))
    coef = min(F32(F32(clip) / F32(np.sqrt(F32(square)) + F32(1.17549435e-38))), F32(1))
    c1 = F32(F32(1) - powi_f32(0.9, time))
    c2 = F32(F32(1) - powi_f32(0.999, time))
    decay = F32(1.0 - float(lr) * float(F32(weight_decay)))
    lr32 = F32(lr)
    with np.errstate(over="ignore", under="ignore"):
        g = (g * coef).astype(F32)
        m = (g * F32(F32(1) - F32(0.9))).astype(F32)
        v = ((g * g).astype(F32) * F32(F32(1) - F32(0.999))).astype(F32)
        if first is not None:
            m = ((np.asarray(first, F32) * F32(0.9)).astype(F32) + m).astype(F32)
            v = ((np.asarray(second, F32) * F32(0.999)).astype(F32) + v).astype(F32)
        delta = ((m / c1).astype(F32) / (np.sqrt((v / c2).astype(F32)) + F32(1e-5)).astype(F32))
        out = ((p * decay).astype(F32) - (delta.astype(F32) * lr32).astype(F32)).astype(F32)
    return out, m, v
