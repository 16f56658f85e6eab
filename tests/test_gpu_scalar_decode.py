"""GPU parity of the scalar-gate gated delta rule and of the decode step.

Scalar gates are the channel-wise recurrence with alpha = exp(g) and
erase = write = beta on every channel; the oracle runs the channel-wise f64
scan with those gates and the chain rule dbeta = sum derase + sum dwrite,
dg = exp(g) sum dalpha.  The decode step must agree, token by token, with the
scan carrying `initial` (the reference's T=1 scans, crates/mixers/src/sbd.rs:270-283).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from gpu_util import TOL_BF16, TOL_F32, dev, gate, host  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def scalar_problem(seed, B, T, H, K, V, masks=True):
    from delta_mixers.synthetic import NormalStream, round_bf16  # noqa: F401
    rng = np.random.default_rng(seed)
    q = rng.normal(size=(B, T, H, K))
    k = rng.normal(size=(B, T, H, K))
    q /= np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
    k /= np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    p = dict(q=q.astype(np.float32), k=k.astype(np.float32),
             v=rng.normal(size=(B, T, H, V)).astype(np.float32),
             beta=(1 / (1 + np.exp(-rng.normal(size=(B, T, H))))).astype(np.float32),
             g=(-np.log1p(np.exp(rng.normal(size=(B, T, H))))).astype(np.float32),
             valid=np.ones((B, T), np.float32), reset=np.zeros((B, T), np.float32),
             initial=(0.1 * rng.normal(size=(B, H, K, V))).astype(np.float32),
             dO=rng.normal(size=(B, T, H, V)).astype(np.float32),
             dF=(0.1 * rng.normal(size=(B, H, K, V))).astype(np.float32),
             dS=(0.1 * rng.normal(size=(B, T, H))).astype(np.float32))
    if masks:
        p["valid"][0, T // 3] = 0
        p["valid"][-1, T - 5:] = 0
        p["reset"][0, T // 2] = 1
    return p


def scalar_oracle(p):
    K, V = p["q"].shape[3], p["v"].shape[3]
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], K, V)
    out, fin, sc = oracle.scan(p["q"], p["k"], p["v"], a, e, w, p["valid"], p["reset"],
                               p["initial"])
    g = oracle.backward(p["q"], p["k"], p["v"], a, e, w, p["valid"], p["reset"], p["initial"],
                        p["dO"], p["dF"], p["dS"])
    db, dg = oracle.scalar_gate_grads(p["g"], g)
    return out, fin, sc, g, db, dg


@pytest.mark.parametrize("dtype,tol", [(torch.float32, TOL_F32), (torch.bfloat16, TOL_BF16)])
@pytest.mark.parametrize("shape", [(2, 100, 2, 32, 32), (1, 130, 3, 64, 64)])
def test_scalar_scan_matches_oracle(dk, dtype, tol, shape):
    p = scalar_problem(1, *shape)
    if dtype == torch.bfloat16:
        for n in ("q", "k", "v", "dO"):
            p[n] = torch.tensor(p[n]).to(torch.bfloat16).float().numpy()
    xs = {n: dev(p[n], dtype).requires_grad_(True) for n in ("q", "k", "v")}
    xs.update({n: dev(p[n]).requires_grad_(True) for n in ("beta", "g", "initial")})
    out, fin, sc = dk.gdn_scalar_scan(xs["q"], xs["k"], xs["v"], xs["beta"], xs["g"],
                                      dev(p["valid"]), dev(p["reset"]), xs["initial"])
    o_out, o_fin, o_sc, og, odb, odg = scalar_oracle(p)
    pad = (p["valid"] == 0)[:, :, None]
    gate("output", out, o_out, tol, exact_zero=pad[..., None])
    gate("final_state", fin, o_fin, tol)
    gate("scores", sc, o_sc, tol, exact_zero=pad)
    loss = (out.float() * dev(p["dO"])).sum() + (fin * dev(p["dF"])).sum() + \
        (sc * dev(p["dS"])).sum()
    loss.backward()
    for n in ("q", "k", "v"):
        gate(f"d{n}", xs[n].grad, og[n], tol, exact_zero=pad[..., None])
    gate("dbeta", xs["beta"].grad, odb, tol, exact_zero=pad)
    gate("dg", xs["g"].grad, odg, tol, exact_zero=pad)
    gate("d_initial", xs["initial"].grad, og["initial"], tol)


@pytest.mark.parametrize("K,V", [(64, 64), (32, 64)])
def test_decode_steps_match_scan(dk, K, V):
    """Decode step by step on a carried state matches one scan over the same
    tokens (the scan takes the f32 chunk kernels, decode the token-sequential
    kernel: equal within the f32 gate), and both match the f64 oracle."""
    rng = np.random.default_rng(3)
    B, T, H = 8, 12, 4
    q = rng.normal(size=(B, T, H, K)).astype(np.float32) * 0.3
    k = rng.normal(size=(B, T, H, K))
    k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float32)
    v = rng.normal(size=(B, T, H, V)).astype(np.float32)
    a = rng.uniform(0.7, 1.0, size=(B, T, H, K)).astype(np.float32)
    e = rng.uniform(0.2, 0.9, size=(B, T, H, K)).astype(np.float32)
    w = rng.uniform(0.2, 0.9, size=(B, T, H, V)).astype(np.float32)
    s0 = (0.02 * rng.normal(size=(B, H, K, V))).astype(np.float32)
    valid = np.ones((B, T), np.float32)
    valid[1, 4] = 0
    reset = np.zeros((B, T), np.float32)
    reset[2, 6] = 1
    r = dk.gdn_training_scan(dev(q), dev(k), dev(v), dev(a), dev(e), dev(w), dev(valid),
                             dev(reset), dev(s0), 16)
    state = dev(s0).clone()
    outs, scs = [], []
    for t in range(T):
        sl = slice(t, t + 1)
        o, s = dk.gdn_decode_step(state, dev(q[:, sl]), dev(k[:, sl]), dev(v[:, sl]),
                                  dev(a[:, sl]), dev(e[:, sl]), dev(w[:, sl]),
                                  dev(valid[:, sl]), dev(reset[:, sl]))
        outs.append(o)
        scs.append(s)
    gate("decode output vs scan", torch.cat(outs, 1), host(r.output), TOL_F32)
    gate("decode scores vs scan", torch.cat(scs, 1), host(r.scores[..., 0]), TOL_F32)
    gate("decode state vs scan", state, host(r.final_state), TOL_F32)
    out, fin, sc = oracle.scan(q, k, v, a, e, w, valid, reset, s0)
    gate("decode output", torch.cat(outs, 1), out, TOL_F32)
    gate("decode state", state, fin, TOL_F32)
