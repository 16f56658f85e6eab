"""The f32 chunked CPU scan (oracle/chunk_cpu.c, a restatement of the
reference's CPU tensor solver crates/mixers/src/chunk.rs:129-250) against the
f64 sequential oracle: the reference's own fixtures (masks, resets on and off
padding, zero alpha on one and on all channels, exactly zero edits, zero key
and value norms, a nonzero initial state) and random bf16-style inputs, at
chunk sizes 1, 5, 16 and 64 (the solver's result must not depend on the
chunk).  Gate: the north-star f32 tolerance, rms-floored."""
import numpy as np
import pytest

from fixtures import gate_fixture, reset_padding_fixture
from oracle import oracle

TOL = 1e-4


def _close(name, got, ref, tol=TOL):
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64).reshape(ref.shape)
    scale = np.sqrt(np.mean(ref * ref)) if ref.size else 0.0
    err = np.abs(got - ref)
    assert np.all(err <= tol * (np.abs(ref) + scale) + 1e-30), (name, float(err.max()), scale)


def _check(f, chunk):
    args = (f["q"], f["k"], f["v"], f["alpha"], f["erase"], f["write"], f["valid"], f["reset"],
            f.get("initial"))
    ro, rf, rs = oracle.scan(*args)
    co, cf, cs = oracle.chunk_scan_f32(*args, chunk=chunk)
    _close("output", co, ro)
    _close("final_state", cf, rf)
    _close("scores", cs, rs)
    pad = np.asarray(f["valid"]) == 0
    assert np.all(co[pad] == 0) and np.all(cs[pad] == 0), "padding must be exactly zero"


@pytest.mark.parametrize("chunk", [1, 5, 16, 64])
def test_gate_fixture(chunk):
    _check(gate_fixture(35, 0), chunk)


@pytest.mark.parametrize("chunk", [1, 2, 16])
def test_reset_padding_fixture(chunk):
    f = reset_padding_fixture()
    _check({n: f[n] for n in ("q", "k", "v", "alpha", "erase", "write", "valid", "reset",
                              "initial")}, chunk)


@pytest.mark.parametrize("chunk", [16, 64])
def test_random_scalar_gates_long(chunk):
    rng = np.random.default_rng(3)
    B, T, H, K, V = 2, 300, 2, 32, 48
    q = rng.normal(size=(B, T, H, K))
    k = rng.normal(size=(B, T, H, K))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    beta = 1 / (1 + np.exp(-rng.normal(size=(B, T, H))))
    g = -np.log1p(np.exp(rng.normal(size=(B, T, H))))
    a, e, w = oracle.scalar_gates(beta, g, K, V)
    valid = np.ones((B, T))
    reset = np.zeros((B, T))
    valid[0, 40:44] = 0
    reset[1, 150] = 1
    f = dict(q=q, k=k, v=rng.normal(size=(B, T, H, V)), alpha=a, erase=e, write=w, valid=valid,
             reset=reset, initial=0.1 * rng.normal(size=(B, H, K, V)))
    _check(f, chunk)
