"""Pinning of the HOLA oracle (oracle/hola_oracle.py), CPU only."""
import numpy as np

import hola_fixtures as hf
from oracle import hola_oracle as ho


def _args(f):
    return (f["q"], f["k"], f["v"], f["scores"], f["valid"], f["docs"], f["sink"],
            f["capacity"], f["chunk"], f["recency"])


def test_gradients_central_differences():
    f = hf.hola_fixture(2, 35, 4, 8, False, True)  # small capacity: evictions happen
    rng = np.random.default_rng(0)
    r = ho.hola_read(*_args(f), upstream=f["upstream"])
    up = f["upstream"].astype(np.float64)
    base = {n: f[n].astype(np.float64) for n in ("q", "k", "v", "sink")}

    def loss(x):
        g = dict(f)
        g.update(x)
        return (ho.hola_read(*_args(g))["output"] * up).sum()

    for n, gname in (("q", "dq"), ("k", "dk"), ("v", "dv"), ("sink", "dsink")):
        d = rng.normal(size=base[n].shape)
        h = 1e-6
        plus = dict(base)
        minus = dict(base)
        plus[n] = base[n] + h * d
        minus[n] = base[n] - h * d
        num = (loss(plus) - loss(minus)) / (2 * h)
        assert abs(num - (r[gname] * d).sum()) < 1e-7 * (1 + abs(num)), n


def test_large_cache_is_dense_causal_attention():
    """Capacity >= T and one document per row (row 0: padding at 8 and 47):
    every earlier valid token stays visible.  (A document label that recurs
    after another document, as in row 1, is not: the cache keeps only the
    document of each chunk's last slot.)"""
    f = hf.hola_fixture(2, 64, 64, 4, False, True)
    r = ho.hola_read(*_args(f))
    q, k, v = (f[n].astype(np.float64) for n in ("q", "k", "v"))
    B, T, H, dk = q.shape
    want = np.zeros_like(r["output"])
    for b in range(1):
        for h in range(H):
            logits = q[b, :, h] @ k[b, :, h].T / np.sqrt(dk)
            ok = ((f["valid"][b][None, :] >= 0.5) & (f["docs"][b][None, :] == f["docs"][b][:, None])
                  & (np.arange(T)[None, :] <= np.arange(T)[:, None]))
            logits = np.where(ok, logits, -np.inf)
            m = np.maximum(logits.max(axis=1), f["sink"][h])
            e = np.exp(logits - m[:, None])
            den = e.sum(axis=1) + np.exp(f["sink"][h] - m)
            o = (e / den[:, None]) @ v[b, :, h]
            want[b, :, h] = np.where(f["valid"][b][:, None] >= 0.5, o, 0)
    np.testing.assert_allclose(r["output"][0], want[0], rtol=1e-12, atol=1e-13)


def test_recency_schedule_closed_form():
    """One document, recency: after each chunk the cache is the last `capacity`
    valid positions, newest first."""
    f = hf.hola_fixture(1, 40, 5, 6, True, False)
    f["valid"][0, [3, 17, 18]] = 0
    s = ho.hola_schedule(f["scores"], f["valid"], f["docs"], 5, 6, True)
    assert np.all(s[:, :, 0] == -1)
    for c, end in enumerate(range(6, 46, 6)):
        kept = [p for p in range(min(end, 40) - 1, -1, -1) if f["valid"][0, p] >= 0.5][:5]
        want = kept + [-1] * (5 - len(kept))
        for h in range(4):
            np.testing.assert_array_equal(s[0, h, c + 1], want)


def test_schedule_final_snapshot_equals_read_positions():
    for recency in (False, True):
        f = hf.hola_fixture(2, 83, 16, 16, recency, True)
        s = ho.hola_schedule(f["scores"], f["valid"], f["docs"], 16, 16, recency)
        r = ho.hola_read(*_args(f))
        np.testing.assert_array_equal(s[:, :, -1], r["positions"])


def test_cancellation_and_overflow_fixtures():
    f = hf.cancellation_fixture()
    r = ho.hola_read(*_args(f), upstream=f["upstream"])
    for h in range(4):
        p = r["output"][0, 0, h, 0]
        assert 0 < p < 1
        d = p * (1 - p)
        np.testing.assert_allclose(r["dv"][0, 0, h, 0], p, rtol=1e-12)
        np.testing.assert_allclose(r["dsink"][h], -d, rtol=1e-10)
        np.testing.assert_allclose(r["dq"][0, 0, h], d * f["k"][0, 0, h] / np.sqrt(32), rtol=1e-10)
    f = hf.overflow_fixture()
    r = ho.hola_read(*_args(f), upstream=f["upstream"])
    assert np.all(np.isfinite(r["output"]))
