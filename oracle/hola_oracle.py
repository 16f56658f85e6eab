"""f64 restatement of the HOLA exact-memory cache read (scores -> cache
selection -> attention over the cache and the causal chunk) and its VJP.

TEST INFRASTRUCTURE ONLY: the checker for the HIP HOLA operators
(delta-block-lm_amd/csrc/gdn2_hola.hip).  Nothing in the product imports it.

What it restates (read as text from the reference, never executed):
  hola_read      the independent scalar oracle of crates/mixers/src/hola_checks.rs:294-391
                 (per (batch, head): chunks in order; every valid query t attends to
                 the cache plus tokens first..t of its chunk that are valid and share
                 its document, with scale 1/sqrt(d_k) and a learned zero-value sink
                 logit; then the chunk joins the cache, the cache keeps only valid
                 tokens of the document of the chunk's last physical slot, sorts by
                 score (or position, for recency) descending then position ascending,
                 and truncates to capacity).  Forward output, final positions and the
                 gradients of sum(output * upstream) in q, k, v and sink.
  hola_schedule  the positions-only schedule of crates/mixers/src/hola.rs:28-105
                 ([B, H, chunks + 1, capacity] snapshots, -1 for empty slots).
Scores select membership and take no gradient.

Pinned by tests/test_hola_oracle.py: central differences of every gradient
(membership is fixed for fixed scores), dense causal softmax attention when the
cache holds everything, the recency schedule's closed form (the last capacity
valid positions), the reference's cancellation VJP (p(1-p) forms,
hola_checks.rs:466-512) and its overflow fixture (finite output for v = 1e38).
"""
from __future__ import annotations

import numpy as np


def _cache_update(cache, first, end, valid_b, docs_b, score_of, capacity):
    cache = cache + list(range(first, end))
    last_doc = docs_b[end - 1]
    cache = [s for s in cache if valid_b[s] >= 0.5 and docs_b[s] == last_doc]
    # descending score, then ascending position (hola_checks.rs:371-382)
    cache.sort(key=lambda s: (-score_of(s), s))
    return cache[:capacity]


def hola_schedule(scores, valid, docs, capacity, chunk, recency):
    """scores [B, T, H] (or [B, T, H, 1]); valid, docs [B, T].  Returns
    [B, H, ceil(T / chunk) + 1, capacity] positions (float, -1 = empty)."""
    scores = np.asarray(scores, dtype=np.float64).reshape(np.shape(valid) + (-1,))
    B, T, H = scores.shape
    nc = -(-T // chunk)
    out = -np.ones((B, H, nc + 1, capacity))
    for b in range(B):
        for h in range(H):
            score_of = (lambda s: float(s)) if recency else (lambda s: scores[b, s, h])
            cache = []
            for c, first in enumerate(range(0, T, chunk)):
                end = min(first + chunk, T)
                cache = _cache_update(cache, first, end, valid[b], docs[b], score_of, capacity)
                out[b, h, c + 1, :len(cache)] = cache
    return out


def hola_read(q, k, v, scores, valid, docs, sink, capacity, chunk, recency, upstream=None):
    """q, k [B, T, H, dk]; v [B, T, H, dv]; scores [B, T, H(, 1)]; valid, docs
    [B, T]; sink [H].  Returns a dict: output, positions [B, H, capacity] and,
    with upstream, dq, dk, dv, dsink."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    B, T, H, dk = q.shape
    dv_w = v.shape[3]
    scores = np.asarray(scores, dtype=np.float64).reshape(B, T, H)
    valid = np.asarray(valid, dtype=np.float64)
    docs = np.asarray(docs, dtype=np.float64)
    sink = np.asarray(sink, dtype=np.float64)
    up = None if upstream is None else np.asarray(upstream, dtype=np.float64)
    scale = 1.0 / np.sqrt(dk)
    out = {"output": np.zeros((B, T, H, dv_w)), "positions": -np.ones((B, H, capacity))}
    if up is not None:
        for n, x in (("dq", q), ("dk", k), ("dv", v)):
            out[n] = np.zeros(x.shape)
        out["dsink"] = np.zeros(H)
    for b in range(B):
        for h in range(H):
            score_of = (lambda s: float(s)) if recency else (lambda s, b=b, h=h: scores[b, s, h])
            cache = []
            for first in range(0, T, chunk):
                end = min(first + chunk, T)
                for t in range(first, end):
                    if valid[b, t] < 0.5:
                        continue
                    vis = [s for s in cache + list(range(first, t + 1))
                           if valid[b, s] >= 0.5 and docs[b, s] == docs[b, t]]
                    vis = np.array(vis, dtype=np.int64)
                    logits = (k[b, vis, h] @ q[b, t, h]) * scale
                    m = max(sink[h], logits.max()) if len(vis) else sink[h]
                    den = np.exp(logits - m).sum() + np.exp(sink[h] - m)
                    p = np.exp(logits - m) / den
                    o = p @ v[b, vis, h]
                    out["output"][b, t, h] = o
                    if up is None:
                        continue
                    g = up[b, t, h]
                    delta = g @ o
                    out["dsink"][h] -= np.exp(sink[h] - m) / den * delta
                    dl = p * (v[b, vis, h] @ g - delta) * scale
                    out["dq"][b, t, h] += dl @ k[b, vis, h]
                    np.add.at(out["dk"], (b, vis, h), dl[:, None] * q[b, t, h][None, :])
                    np.add.at(out["dv"], (b, vis, h), p[:, None] * g[None, :])
                cache = _cache_update(cache, first, end, valid[b], docs[b], score_of, capacity)
            out["positions"][b, h, :len(cache)] = cache
    return out
