"""Restated procedural fixtures of the reference's HOLA checks (test data).

  hola_fixture      crates/mixers/src/hola_checks.rs:76-165 (Fixture::new)
  overflow_fixture  hola_checks.rs:166-183
  cancellation      hola_checks.rs:466-486
  CASES             hola_checks.rs:561-571 (policy x (T, capacity, chunk), B 2, packed)

Arrays are [batch, time, head, width] float32 (H 4, d_k 32, d_v 64), masks and
document ids [batch, time] float32, sink [4].
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
CASES = [(7, 16, 16), (35, 16, 1), (83, 16, 16), (145, 64, 16)]


def _signal(n, phase):
    i = np.arange(n)
    return (F32(0.7) * np.sin((i * 11 + phase) * 0.09).astype(F32)).astype(F32)


def hola_fixture(b, t, capacity, chunk, recency, packed):
    h = 4
    q = _signal(b * t * h * 32, 3).reshape(-1, 32)
    k = _signal(b * t * h * 32, 7).reshape(-1, 32)
    for x in (q, k):  # per-row RMS normalisation with learned-looking scales
        rms = np.sqrt((x * x).sum(axis=1, dtype=F32) / F32(32) + F32(1e-5)).astype(F32)
        x[:] = x / rms[:, None] * (F32(0.8) + F32(0.01) * np.arange(32, dtype=F32))
    valid = np.ones((b, t), F32)
    docs = np.zeros((b, t), F32)
    if packed:
        for row in range(b):
            for p in range(t):
                if p in (8, 47):
                    valid[row, p] = 0
                if row == 1:
                    docs[row, p] = 0 if p < 37 else (1 if p < 79 else 0)
                    if 16 <= p < 32:
                        valid[row, p] = 0
                    if p == 31 or p + 1 == t:
                        valid[row, p] = 0
                        docs[row, p] = 77
    i = np.arange(b * t * h)
    p = i // h % t
    scores = np.where(valid.reshape(-1)[i // h] == 0, F32(1000),
                      np.where(p == 2, F32(8), (p % 5).astype(F32))).astype(F32)
    return {
        "q": q.reshape(b, t, h, 32), "k": k.reshape(b, t, h, 32),
        "v": _signal(b * t * h * 64, 13).reshape(b, t, h, 64),
        "scores": scores.reshape(b, t, h, 1), "valid": valid, "docs": docs,
        "sink": np.array([0.2, -0.7, 3.0, -2.0], F32),
        "upstream": _signal(b * t * h * 64, 21).reshape(b, t, h, 64),
        "capacity": capacity, "chunk": chunk, "recency": recency,
    }


def overflow_fixture():
    f = hola_fixture(1, 4, 1, 4, False, False)
    for n in ("q", "k", "v", "upstream"):
        f[n] = np.zeros_like(f[n])
    f["sink"] = np.zeros(4, F32)
    f["v"][0, :, :, 0] = F32(1e38)
    f["upstream"][0, :, :, 0] = F32(1e-36)
    return f


def cancellation_fixture():
    f = hola_fixture(1, 1, 1, 1, False, False)
    for n in ("q", "k", "v", "upstream"):
        f[n] = np.zeros_like(f[n])
    f["sink"] = np.zeros(4, F32)
    f["q"][0, 0, :, :4] = np.array([1e4, 1, 1e4, 1], F32)
    f["k"][0, 0, :, :4] = np.array([1e4, 1, -1e4, 1], F32)
    f["v"][0, 0, :, 0] = 1
    f["upstream"][0, 0, :, 0] = 1
    return f
