"""Pinning of the document-limit oracle (oracle/doc_oracle.py), CPU only."""
import numpy as np

from oracle import doc_oracle as do
from oracle import oracle


def _inputs(rng, B, T, H, K, V):
    q = rng.normal(size=(B, T, H, K)) * 0.5
    k = rng.normal(size=(B, T, H, K)) * 0.5
    v = rng.normal(size=(B, T, H, V))
    alpha = rng.uniform(0.7, 1.0, size=(B, T, H, K))
    erase = rng.uniform(0.2, 0.8, size=(B, T, H, K))
    write = rng.uniform(0.2, 0.8, size=(B, T, H, V))
    return q, k, v, alpha, erase, write


def consistent_limits(B, T, docs):
    """Packed documents: docs[b] is a list of (start, end) spans (inclusive);
    positions outside every span are padding (start 1, end 0)."""
    start = np.ones((B, T), np.int32)
    end = np.zeros((B, T), np.int32)
    for b, spans in enumerate(docs):
        for s, e in spans:
            start[b, s:e + 1] = s
            end[b, s:e + 1] = e
    return start, end


def test_consistent_documents_equal_the_mask_oracle():
    rng = np.random.default_rng(0)
    B, T, H, K, V = 2, 23, 2, 5, 4
    x = _inputs(rng, B, T, H, K, V)
    start, end = consistent_limits(B, T, [[(0, 6), (7, 15), (18, 22)], [(2, 22)]])
    valid, reset = oracle.doc_limits_to_masks(start, end)
    out, states = do.doc_scan(*x, start, end)
    ref_out, ref_fin, _ = oracle.scan(*x, valid, reset)
    np.testing.assert_allclose(out, ref_out, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(states[:, -1], ref_fin, rtol=1e-12, atol=1e-13)
    up = rng.normal(size=out.shape)
    g = do.doc_backward(*x, start, end, up)
    ref = oracle.backward(*x, valid, reset, upstream=up)
    for n in ("q", "k", "v", "alpha", "erase", "write"):
        np.testing.assert_allclose(g[n], ref[n], rtol=1e-11, atol=1e-12, err_msg=n)


def test_central_differences_on_consistent_documents():
    rng = np.random.default_rng(1)
    B, T, H, K, V = 1, 9, 1, 3, 2
    x = list(_inputs(rng, B, T, H, K, V))
    start, end = consistent_limits(B, T, [[(0, 3), (5, 8)]])  # padding at 4
    up = rng.normal(size=(B, T, H, V))
    g = do.doc_backward(*x, start, end, up)
    names = ("q", "k", "v", "alpha", "erase", "write")
    f = lambda xs: (do.doc_scan(*xs, start, end)[0] * up).sum()  # noqa: E731
    for i, n in enumerate(names):
        d = rng.normal(size=x[i].shape)
        h = 1e-6
        xp = list(x)
        xm = list(x)
        xp[i] = x[i] + h * d
        xm[i] = x[i] - h * d
        num = (f(xp) - f(xm)) / (2 * h)
        assert abs(num - (g[n] * d).sum()) < 1e-7 * (1 + abs(num)), n


def test_reference_internal_padding_case():
    """crates/mixers/src/gdn2_reference.rs:229-268: three constant tokens, the
    middle one padding (start 1 > end 0); limits [0, 1, 0] / [2, 0, 2]."""
    K, V = 32, 64
    tok = lambda val: np.full((1, 3, 1, K if val[1] == "k" else V), val[0])  # noqa: E731
    q, k = tok((0.1, "k")), tok((0.1, "k"))
    v = tok((0.2, "v"))
    alpha, erase, write = tok((0.9, "k")), tok((0.3, "k")), tok((0.5, "v"))
    start = np.array([[0, 1, 0]])
    end = np.array([[2, 0, 2]])
    out, states = do.doc_scan(q, k, v, alpha, erase, write, start, end)
    np.testing.assert_array_equal(states[0, 0], states[0, 1])
    assert np.all(out[0, 1] == 0)
    up = np.zeros((1, 3, 1, V))
    up[0, 2] = 1.0
    g = do.doc_backward(q, k, v, alpha, erase, write, start, end, up)
    x = [q, k, v, alpha, erase, write]
    for field, idx in (("alpha", 3), ("erase", 4), ("k", 1)):
        xp = [a.copy() for a in x]
        xm = [a.copy() for a in x]
        xp[idx][0, 2, 0, 0] += 1e-6
        xm[idx][0, 2, 0, 0] -= 1e-6
        num = (do.doc_scan(*xp, start, end)[0][0, 2].sum()
               - do.doc_scan(*xm, start, end)[0][0, 2].sum()) / 2e-6
        assert abs(num - g[field][0, 2, 0, 0]) < 1e-7, field


def test_inconsistent_limits_follow_the_reference_rule():
    """A reset at t = 3 whose previous token does not end its document: the
    forward restarts the state, and the f64 oracle's backward
    (gdn2_reference.rs:107-226) keeps the adjoint flowing into tokens 0-2,
    unlike the exact VJP that the reference's GPU kernels compute."""
    rng = np.random.default_rng(2)
    B, T, H, K, V = 1, 6, 1, 3, 2
    x = _inputs(rng, B, T, H, K, V)
    start = np.array([[0, 0, 0, 3, 3, 3]])
    end = np.array([[5, 5, 5, 5, 5, 5]])
    valid, reset = oracle.doc_limits_to_masks(start, end)
    out, _ = do.doc_scan(*x, start, end)
    np.testing.assert_allclose(out, oracle.scan(*x, valid, reset)[0], rtol=1e-12, atol=1e-13)
    up = np.zeros((B, T, H, V))
    up[0, 4] = 1.0  # only a token after the reset has an output gradient
    g = do.doc_backward(*x, start, end, up)
    exact = oracle.backward(*x, valid, reset, upstream=up)
    assert np.all(exact["q"][0, :3] == 0) and np.all(exact["alpha"][0, :3] == 0)
    assert np.abs(g["k"][0, :3]).max() > 1e-3  # the reference leaks across the reset
    np.testing.assert_allclose(g["q"][0, 3:], exact["q"][0, 3:], rtol=1e-12, atol=1e-13)
