"""Pins the CPU oracle (oracle/gdn2_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a wrong sign, a transposed index, a mask applied at the wrong time)
fails at least one of them:
  * SplitMix64 published test values and Box-Muller moments;
  * closed forms: T=1 from the zero state, and the aligned fixture's scalar
    recurrence s_t = s_{t-1} + 0.5 (1 - s_{t-1}) (checks.rs:181-198);
  * an independent algorithm: the chunk-WY form of the whole sequence with a
    dense numpy.linalg.solve for (I + L) (chunk.rs:170-241 with a library
    solve in place of the nilpotent series), including masks and an initial
    state;
  * f64 central differences of the analytic VJP along random unit directions,
    per input group and for the initial state (tolerance of
    reuse/crates/dre-gdn2/src/tests.rs:182-216);
  * the reference fixture's own assertions (chunk_tests.rs:148-170) and the
    zero-edit subgradient cases of kron_checks.rs:132-188.
"""
import numpy as np
import pytest

import fixtures as fx
from oracle import oracle

GROUPS = ("q", "k", "v", "alpha", "erase", "write")


def rand_problem(rng, B=2, T=9, H=2, K=5, V=6, masks=True, initial=True):
    p = {
        "q": rng.normal(size=(B, T, H, K)) * 0.5,
        "k": rng.normal(size=(B, T, H, K)) * 0.45,
        "v": rng.normal(size=(B, T, H, V)),
        "alpha": rng.uniform(0.6, 0.99, size=(B, T, H, K)),
        "erase": rng.uniform(0.2, 0.8, size=(B, T, H, K)),
        "write": rng.uniform(0.3, 1.0, size=(B, T, H, V)),
    }
    valid = np.ones((B, T), np.uint8)
    reset = np.zeros((B, T), np.uint8)
    if masks:
        valid[0, 3] = 0
        valid[1, T - 2:] = 0
        reset[0, 5] = 1
        reset[1, 3] = 0
        reset[0, 3] = 1  # reset on padding: ignored
    p["valid"], p["reset"] = valid, reset
    p["initial"] = rng.normal(size=(B, H, K, V)) * 0.3 if initial else None
    return p


def wy_dense(p):
    """Whole-sequence chunk-WY forward with a dense solve (independent algorithm)."""
    q, k, v = p["q"], p["k"], p["v"]
    B, T, H, K = q.shape
    V = v.shape[3]
    out = np.zeros((B, T, H, V))
    fin = np.zeros((B, H, K, V))
    sc = np.zeros((B, T, H))
    for b in range(B):
        act = p["valid"][b].astype(float)
        rst = p["reset"][b].astype(float)
        for h in range(H):
            a = p["alpha"][b, :, h] * (1 - rst)[:, None] * act[:, None] + (1 - act)[:, None]
            qq = q[b, :, h] * act[:, None]
            kk = k[b, :, h] * act[:, None]
            vv = v[b, :, h] * act[:, None]
            ee = p["erase"][b, :, h] * act[:, None]
            ww = p["write"][b, :, h] * act[:, None]
            S0 = np.zeros((K, V)) if p["initial"] is None else p["initial"][b, h]
            D = np.ones((T, T, K))  # D[r,s] = prod_{u=s+1..r} a_u
            for r in range(T):
                for s in range(T):
                    D[r, s] = np.prod(a[s + 1:r + 1], axis=0) if s < r else (1.0 if s == r else 0.0)
            P = np.cumprod(a, axis=0)
            L = np.zeros((T, T))
            M = np.zeros((T, T))
            for r in range(T):
                for s in range(r + 1):
                    if s < r:
                        L[r, s] = np.sum(ee[r] * kk[r] * D[r, s] * kk[s])
                    M[r, s] = np.sum(qq[r] * D[r, s] * kk[s])
            rhs = ww * vv - (ee * kk * P) @ S0
            delta = np.linalg.solve(np.eye(T) + L, rhs)
            out[b, :, h] = (qq * P) @ S0 + M @ delta
            fin[b, h] = P[-1][:, None] * S0 + (D[T - 1] * kk).T @ delta
            sc[b, :, h] = np.linalg.norm(kk, axis=1) * np.linalg.norm(delta, axis=1)
    return out, fin, sc


def objective(p, U, F, G):
    out, fin, sc = oracle.scan(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                               p["valid"], p["reset"], p["initial"])
    return np.sum(out * U) + np.sum(fin * F) + np.sum(sc * G)


def test_splitmix_published_values():
    # SplitMix64 reference outputs for seed 1234567 (Vigna's splitmix64.c).
    got = oracle.splitmix(1234567, 5)
    assert [int(x) for x in got] == [6457827717110365317, 3203168211198807973,
                                     9817491932198370423, 4593380528125082431,
                                     16408922859458223821]
    py = fx.SplitMix(1234567)
    assert [py.next() for _ in range(5)] == [int(x) for x in got]


def test_box_muller_moments():
    x = oracle.normals(0, 400_000)
    assert abs(x.mean()) < 6e-3 and abs(x.var() - 1) < 1e-2
    assert abs(np.mean(x ** 3)) < 2e-2 and abs(np.mean(x ** 4) - 3) < 5e-2
    py = fx.SplitMix(0)
    assert np.allclose([py.normal() for _ in range(4)], x[:4], rtol=0, atol=1e-15)


def test_single_token_closed_form():
    rng = np.random.default_rng(1)
    p = rand_problem(rng, B=1, T=1, H=3, K=4, V=7, masks=False, initial=False)
    out, fin, sc = oracle.scan(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                               p["valid"], p["reset"], None)
    wv = p["write"] * p["v"]
    for h in range(3):
        k, q = p["k"][0, 0, h], p["q"][0, 0, h]
        assert np.allclose(fin[0, h], np.outer(k, wv[0, 0, h]), atol=1e-15)
        assert np.allclose(out[0, 0, h], (q @ k) * wv[0, 0, h], atol=1e-15)
        assert np.isclose(sc[0, 0, h], np.linalg.norm(k) * np.linalg.norm(wv[0, 0, h]))


@pytest.mark.parametrize("t", [7, 35])
def test_aligned_closed_form(t):
    f = fx.aligned_fixture(t)
    out, fin, sc = oracle.scan(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset)
    B, T, H, V = out.shape
    for b in range(B):
        s = 0.0
        for p in range(T):
            if not f.valid[b, p]:
                assert np.all(out[b, p] == 0) and np.all(sc[b, p] == 0)
                continue
            if f.reset[b, p]:
                s = 0.0
            delta = 0.5 * (1 - s)
            s = s + delta
            assert np.allclose(out[b, p, :, 0], s, rtol=0, atol=1e-15)
            assert np.all(out[b, p, :, 1:] == 0)
            assert np.allclose(sc[b, p], abs(delta), atol=1e-15)
        assert np.allclose(fin[b, :, 0, 0], s, atol=1e-15)


@pytest.mark.parametrize("masks,initial", [(False, False), (True, False), (True, True)])
def test_forward_matches_dense_wy_solve(masks, initial):
    rng = np.random.default_rng(2 + masks + 2 * initial)
    p = rand_problem(rng, masks=masks, initial=initial)
    got = oracle.scan(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                      p["valid"], p["reset"], p["initial"])
    want = wy_dense(p)
    for g, w in zip(got, want):
        assert np.allclose(g, w, rtol=1e-11, atol=1e-12)


def test_forward_zero_alpha_matches_dense():
    rng = np.random.default_rng(5)
    p = rand_problem(rng)
    p["alpha"][0, 2, 0, 1] = 0.0
    p["alpha"][1, 4, :, :] = 0.0
    got = oracle.scan(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                      p["valid"], p["reset"], p["initial"])
    for g, w in zip(got, wy_dense(p)):
        assert np.allclose(g, w, rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("masks", [False, True])
def test_backward_central_differences(masks):
    rng = np.random.default_rng(11 + masks)
    p = rand_problem(rng, B=1, T=8, H=1, K=4, V=5, masks=False, initial=True)
    if masks:
        p["valid"][0, 2] = 0
        p["reset"][0, 5] = 1
    B, T, H, K = p["q"].shape
    V = p["v"].shape[3]
    U = rng.normal(size=(B, T, H, V))
    F = rng.normal(size=(B, H, K, V))
    G = rng.normal(size=(B, T, H))
    g = oracle.backward(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                        p["valid"], p["reset"], p["initial"], U, F, G)
    for name in GROUPS + ("initial",):
        grad = g[name]
        norm = np.linalg.norm(grad)
        assert norm > 0, name
        x0 = p[name]
        step = 1e-6 * max(np.sqrt(np.mean(x0 ** 2)), 1.0)
        for _ in range(8):
            d = rng.normal(size=x0.shape)
            d /= np.linalg.norm(d)
            pp = dict(p)
            pp[name] = x0 + step * d
            fp = objective(pp, U, F, G)
            pp[name] = x0 - step * d
            fm = objective(pp, U, F, G)
            num = (fp - fm) / (2 * step)
            ana = np.sum(grad * d)
            assert abs(num - ana) <= 1e-7 * norm + 1e-6 * abs(num), (name, num, ana)


def test_backward_padding_tokens_have_exactly_zero_gradients():
    rng = np.random.default_rng(3)
    p = rand_problem(rng)
    U = rng.normal(size=p["v"].shape)
    g = oracle.backward(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                        p["valid"], p["reset"], p["initial"], U, None, None)
    pad = p["valid"] == 0
    for name in GROUPS:
        assert np.all(g[name][pad] == 0), name


def test_reference_reset_padding_fixture_assertions():
    """chunk_tests.rs:148-170 on the B2/T5/H2/K3/V4 fixture."""
    f = fx.reset_padding_fixture()
    g = oracle.backward(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                        f.initial, f.upstream, None, None)
    g0 = oracle.backward(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                         None, f.upstream, None, None)
    out, _, _ = oracle.scan(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                            f.initial)
    effect = np.max(np.abs(g["k"][0, 0] - g0["k"][0, 0]))
    assert effect > 1e-4
    H, K, V = 2, 3, 4
    assert np.any(np.abs(g["initial"][0]) > 1e-4)
    assert np.all(g["initial"][1] == 0)  # row 1 resets on its first valid token
    pad = f.valid == 0
    assert np.all(g["k"][pad] == 0) and np.all(out[pad] == 0)


@pytest.mark.parametrize("t", [1, 7, 35])
def test_gate_fixture_edge_semantics(t):
    """kron_checks.rs:132-188 edits: zero edit at p=1 scores exactly 0 and takes the
    zero subgradient; zero key at p=4; padding rows are exactly zero."""
    f = fx.gate_fixture(t, 0)
    out, fin, sc = oracle.scan(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                               f.initial)
    g = oracle.backward(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                        f.initial, f.upstream, f.final_adjoint, f.score_adjoint)
    for name in GROUPS + ("initial",):
        assert np.all(np.isfinite(g[name]))
    if t > 1:
        assert np.all(sc[:, 1][f.valid[:, 1] == 1] == 0)
    if t > 4:
        assert np.all(sc[:, 4][f.valid[:, 4] == 1] == 0)
    pad = f.valid == 0
    assert np.all(out[pad] == 0) and np.all(sc[pad] == 0)
    for name in GROUPS:
        assert np.all(g[name][pad] == 0)


def test_scalar_gate_adapter_central_differences():
    rng = np.random.default_rng(21)
    B, T, H, K, V = 1, 10, 2, 4, 3
    q = rng.normal(size=(B, T, H, K))
    k = rng.normal(size=(B, T, H, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(B, T, H, V))
    beta = 1 / (1 + np.exp(-rng.normal(size=(B, T, H))))
    gl = -np.log1p(np.exp(rng.normal(size=(B, T, H))))
    valid = np.ones((B, T), np.uint8)
    reset = np.zeros((B, T), np.uint8)
    U = rng.normal(size=(B, T, H, V))

    def f(beta_, g_):
        a, e, w = oracle.scalar_gates(beta_, g_, K, V)
        out, _, _ = oracle.scan(q, k, v, a, e, w, valid, reset)
        return np.sum(out * U)

    a, e, w = oracle.scalar_gates(beta, gl, K, V)
    grads = oracle.backward(q, k, v, a, e, w, valid, reset, None, U)
    dbeta, dg = oracle.scalar_gate_grads(gl, grads)
    h = 1e-6
    for idx in [(0, 0, 0), (0, 4, 1), (0, 9, 0)]:
        bp, bm = beta.copy(), beta.copy()
        bp[idx] += h
        bm[idx] -= h
        assert np.isclose((f(bp, gl) - f(bm, gl)) / (2 * h), dbeta[idx], rtol=1e-6, atol=1e-9)
        gp, gm = gl.copy(), gl.copy()
        gp[idx] += h
        gm[idx] -= h
        assert np.isclose((f(beta, gp) - f(beta, gm)) / (2 * h), dg[idx], rtol=1e-6, atol=1e-9)


def test_doc_limits_to_masks():
    # one row: document [0,3), padding at 3, document [4,6): gdn2_reference.rs:85-99
    starts = np.array([[0, 0, 0, 3, 4, 4]])
    ends = np.array([[2, 2, 2, 2, 5, 5]])
    valid, reset = oracle.doc_limits_to_masks(starts, ends)
    assert valid.tolist() == [[1, 1, 1, 0, 1, 1]]
    assert reset.tolist() == [[1, 0, 0, 0, 1, 0]]


def test_nonfinite_input_rejected():
    rng = np.random.default_rng(0)
    p = rand_problem(rng, masks=False)
    p["v"][0, 2, 0, 1] = np.nan
    with pytest.raises(ValueError):
        oracle.scan(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"], p["valid"],
                    p["reset"])


def test_backward_replay_checkpoint_boundary_exact():
    """T above the oracle's replay interval (64) gives the same gradients as
    splitting the sequence at the checkpoint (continuation through initial)."""
    rng = np.random.default_rng(8)
    p = rand_problem(rng, B=1, T=70, H=1, K=3, V=4, masks=False, initial=True)
    U = rng.normal(size=p["v"].shape)
    g = oracle.backward(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                        p["valid"], p["reset"], p["initial"], U)
    # second half seeded by the state after the first 64 tokens
    cut = 64
    sl = {n: p[n][:, :cut] for n in GROUPS}
    _, mid, _ = oracle.scan(*(sl[n] for n in GROUPS), p["valid"][:, :cut], p["reset"][:, :cut],
                            p["initial"])
    tl = {n: p[n][:, cut:] for n in GROUPS}
    g2 = oracle.backward(*(tl[n] for n in GROUPS), p["valid"][:, cut:], p["reset"][:, cut:],
                         mid, U[:, cut:])
    for n in GROUPS:
        assert np.allclose(g[n][:, cut:], g2[n], rtol=1e-12, atol=1e-14)
