"""f64 restatement of the document-limit GDN-2 scan and its VJP.

TEST INFRASTRUCTURE ONLY: the checker for gdn2_scan / gdn2_backward in
delta-block-lm_amd/csrc (the document-limit mode of the token-sequential and
chunk kernels).  Nothing in the product imports it.

What it restates (read as text from the reference, never executed):
  doc_scan       crates/mixers/src/gdn2_reference.rs:51-103 (step and scan):
                 padding where doc_end < doc_start keeps the state and emits
                 zeros; doc_start == t zeroes the state before the update
  doc_backward   crates/mixers/src/gdn2_reference.rs:107-226: reverse sweep
                 whose state adjoint is cleared at doc_end == t (before adding
                 the token's own output gradient), not at resets; padding
                 tokens pass it through
Arrays: sequences [batch, time, head, channel], limits [batch, time] int,
vectorised over batch and head, one loop over time.

Pinned by tests/test_doc_oracle.py: for documents whose tokens share their
(start, end) limits both functions equal the independently pinned
valid/reset oracle (oracle/oracle.py scan and exact VJP); the reference's own
padding test (gdn2_reference.rs:229-268) with its assertions and central
differences; and central differences of doc_backward on consistent documents.
For inconsistent limits (a reset not preceded by a document end) doc_backward
is the f64 oracle's rule, pinned by restatement only.  The reference's GPU op
(crates/kernels/src/gdn2.rs:24-65, :288-490) computes the exact VJP of the
forward instead, whose adjoint never crosses a reset: oracle.backward with the
masks of oracle.doc_limits_to_masks.  The kernels here follow the GPU op; the two rules agree
whenever each reset follows a document end.
"""
from __future__ import annotations

import numpy as np


def _f(x):
    return np.asarray(x, dtype=np.float64)


def doc_scan(q, k, v, alpha, erase, write, doc_start, doc_end):
    """Returns (output [B,T,H,V], states [B,T,H,K,V]: the state after each
    position, padding keeping the previous one)."""
    q, k, v, alpha, erase, write = map(_f, (q, k, v, alpha, erase, write))
    doc_start = np.asarray(doc_start)
    doc_end = np.asarray(doc_end)
    B, T, H, K = q.shape
    V = v.shape[3]
    S = np.zeros((B, H, K, V))
    out = np.zeros((B, T, H, V))
    states = np.zeros((B, T, H, K, V))
    for t in range(T):
        live = doc_end[:, t] >= doc_start[:, t]                   # [B]
        fresh = live & (doc_start[:, t] == t)
        S = np.where(fresh[:, None, None, None], 0.0, S)
        bar = alpha[:, t, :, :, None] * S
        read = np.einsum("bhkv,bhk->bhv", bar, erase[:, t] * k[:, t])
        delta = write[:, t] * v[:, t] - read
        new = bar + k[:, t, :, :, None] * delta[:, :, None, :]
        o = np.einsum("bhkv,bhk->bhv", new, q[:, t])
        S = np.where(live[:, None, None, None], new, S)
        out[:, t] = np.where(live[:, None, None], o, 0.0)
        states[:, t] = S
    return out, states


def doc_backward(q, k, v, alpha, erase, write, doc_start, doc_end, upstream):
    """Gradients of sum(output * upstream), by the reference's rule.  Returns a
    dict with q, k, v, alpha, erase, write."""
    q, k, v, alpha, erase, write, upstream = map(_f, (q, k, v, alpha, erase, write, upstream))
    doc_start = np.asarray(doc_start)
    doc_end = np.asarray(doc_end)
    B, T, H, K = q.shape
    V = v.shape[3]
    _, states = doc_scan(q, k, v, alpha, erase, write, doc_start, doc_end)
    g = {n: np.zeros(x.shape) for n, x in
         zip(("q", "k", "v", "alpha", "erase", "write"), (q, k, v, alpha, erase, write))}
    adj = np.zeros((B, H, K, V))
    for t in range(T - 1, -1, -1):
        live = doc_end[:, t] >= doc_start[:, t]
        m4 = live[:, None, None, None]
        clear = live & (doc_end[:, t] == t)
        adj = np.where(clear[:, None, None, None], 0.0, adj)
        fresh = doc_start[:, t] == t
        prev = states[:, t - 1] if t > 0 else np.zeros((B, H, K, V))
        prev = np.where(fresh[:, None, None, None], 0.0, prev)
        bar = alpha[:, t, :, :, None] * prev
        ek = erase[:, t] * k[:, t]
        delta = write[:, t] * v[:, t] - np.einsum("bhkv,bhk->bhv", bar, ek)
        dy = upstream[:, t]
        dq = np.einsum("bhkv,bhv->bhk", states[:, t], dy)
        a = adj + q[:, t, :, :, None] * dy[:, :, None, :]
        dk = np.einsum("bhkv,bhv->bhk", a, delta)
        dd = np.einsum("bhkv,bhk->bhv", a, k[:, t])
        dbar = a - ek[:, :, :, None] * dd[:, :, None, :]
        de = -np.einsum("bhkv,bhv->bhk", bar, dd)
        lv = live[:, None, None]
        g["q"][:, t] = np.where(lv, dq, 0.0)
        g["erase"][:, t] = np.where(lv, de * k[:, t], 0.0)
        g["k"][:, t] = np.where(lv, dk + de * erase[:, t], 0.0)
        g["alpha"][:, t] = np.where(lv, (dbar * prev).sum(-1), 0.0)
        g["write"][:, t] = np.where(lv, dd * v[:, t], 0.0)
        g["v"][:, t] = np.where(lv, dd * write[:, t], 0.0)
        adj = np.where(m4, alpha[:, t, :, :, None] * dbar, adj)
    return g
