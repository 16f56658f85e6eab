"""Inputs and runners shared by the chunk-WY GPU tests: seeded scalar-gate
problems (bf16-rounded q/k/v/dO, f32 gates, optional masks and initial state),
the forward/backward through the C ABI, and the f64 oracle's gradients."""
import numpy as np
import torch

from gpu_util import dev
from oracle import oracle


def chunk_stages(D):
    """Stage-timer names of the chunk-WY path at d_k = d_v = D (64 or 128):
    prep, state scan and output forward; prep, adjoint scan and gradients
    backward."""
    assert D in (64, 128)
    return {"chunk_prep", "state_scan", "chunk_out", "chunk_bprep", "adjoint_scan", "chunk_bgrad"}


def problem(seed, B, T, H, masks=True, initial=True, K=64, V=64, reset_every=0):
    """reset_every > 0 adds a valid reset every reset_every tokens of the
    first sequence and a padded run before each (long sequences)."""
    rng = np.random.default_rng(seed)
    q = rng.normal(size=(B, T, H, K))
    k = rng.normal(size=(B, T, H, K))
    q /= np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
    k /= np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    bf = lambda x: torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).float().numpy()  # noqa
    p = dict(q=bf(q), k=bf(k), v=bf(rng.normal(size=(B, T, H, V))),
             beta=(1 / (1 + np.exp(-rng.normal(size=(B, T, H))))).astype(np.float32),
             g=(-np.log1p(np.exp(rng.normal(size=(B, T, H))))).astype(np.float32),
             valid=np.ones((B, T), np.float32), reset=np.zeros((B, T), np.float32),
             initial=(0.1 * rng.normal(size=(B, H, K, V))).astype(np.float32) if initial else None,
             dO=bf(rng.normal(size=(B, T, H, V))),
             dF=(0.1 * rng.normal(size=(B, H, K, V))).astype(np.float32),
             dS=(0.1 * rng.normal(size=(B, T, H))).astype(np.float32))
    if masks:
        p["valid"][0, 5] = 0
        p["valid"][0, min(70, T - 2):min(75, T - 1)] = 0
        p["valid"][-1, T - 9:] = 0
        p["reset"][0, 40 if T > 40 else T // 2] = 1
        p["reset"][0, min(72, T - 2)] = 1  # reset on padding: ignored
        if T > 130:
            p["reset"][-1, 129] = 1
        for t in range(reset_every, T - 1, reset_every or T):
            p["reset"][0, t] = 1
            p["valid"][0, t - 3:t - 1] = 0
    return p


def run_fwd(dk, p, chunk=64):
    x = {n: dev(p[n], torch.bfloat16) for n in ("q", "k", "v")}
    out, fin, sc, ck = dk.gdn_scalar_forward(x["q"], x["k"], x["v"], dev(p["beta"]), dev(p["g"]),
                                             dev(p["valid"]), dev(p["reset"]),
                                             dev(p["initial"]), chunk)
    return out, fin, sc


def scalar_oracle_grads(p):
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], p["q"].shape[3], p["v"].shape[3])
    g = oracle.backward(p["q"], p["k"], p["v"], a, e, w, p["valid"], p["reset"], p["initial"],
                        p["dO"], p["dF"], p["dS"])
    db, dg = oracle.scalar_gate_grads(p["g"], g)
    return g, db, dg


def run_bwd(dk, p, chunk=64, use_final=True, use_scores=True):
    x = {n: dev(p[n], torch.bfloat16) for n in ("q", "k", "v")}
    beta, g, valid, reset = (dev(p[n]) for n in ("beta", "g", "valid", "reset"))
    init = dev(p["initial"])
    out, fin, sc, ck = dk.gdn_scalar_forward(x["q"], x["k"], x["v"], beta, g, valid, reset, init,
                                             chunk)
    return dk.gdn_scalar_backward(x["q"], x["k"], x["v"], beta, g, valid, reset, ck, chunk,
                                  dev(p["dO"], torch.bfloat16),
                                  dev(p["dF"]) if use_final else None,
                                  dev(p["dS"]) if use_scores else None)


def slow_decay(p, lo, hi, seed):
    """Replace a problem's scalar log gates by g = log(alpha) with alpha drawn
    uniformly from [lo, hi] (the reference benchmark draws alpha in
    [0.90, 0.99], crates/experiment/src/kron_benchmark.rs:89)."""
    rng = np.random.default_rng(seed + 104729)
    alpha = rng.uniform(lo, hi, size=p["g"].shape)
    p["g"] = np.log(alpha).astype(np.float32)
    return p


def cw_problem(seed, B, T, H, masks=True, initial=True, alpha_lo=0.5, reset_every=0, D=64,
               alpha_hi=1.0):
    """A channel-wise gate problem: bf16-rounded q/k/v/dO (q, k unit rows),
    f32 per-channel gates alpha in (alpha_lo, alpha_hi), erase in (0, 1), write
    in (-0.5, 1), with the masks of problem()."""
    p = problem(seed, B, T, H, masks=masks, initial=initial, K=D, V=D, reset_every=reset_every)
    rng = np.random.default_rng(seed + 7919)
    p["alpha"] = rng.uniform(alpha_lo, alpha_hi, size=(B, T, H, D)).astype(np.float32)
    p["erase"] = rng.uniform(0.0, 1.0, size=(B, T, H, D)).astype(np.float32)
    p["write"] = rng.uniform(-0.5, 1.0, size=(B, T, H, D)).astype(np.float32)
    return p


def cw_oracle(p, use_final=True, use_scores=True):
    """f64 forward outputs and gradients of a cw_problem."""
    out, fin, sc = oracle.scan(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"],
                               p["valid"], p["reset"], p["initial"])
    g = oracle.backward(p["q"], p["k"], p["v"], p["alpha"], p["erase"], p["write"], p["valid"],
                        p["reset"], p["initial"], p["dO"], p["dF"] if use_final else None,
                        p["dS"] if use_scores else None)
    return (out, fin, sc), g


def fixture_problem(f, bf16=True):
    """A restated reference fixture (tests/fixtures.py) as a cw_problem-style
    dict, with q/k/v and the output adjoint rounded to bf16 when the problem
    is meant for the bf16 chunk kernels (the oracle then sees the rounded
    values)."""
    bf = (lambda x: torch.tensor(np.ascontiguousarray(x), dtype=torch.float32)
          .to(torch.bfloat16).float().numpy()) if bf16 else (lambda x: np.asarray(x, np.float32))
    return dict(q=bf(f.q), k=bf(f.k), v=bf(f.v), alpha=np.array(f.alpha, np.float32),
                erase=np.array(f.erase, np.float32), write=np.array(f.write, np.float32),
                valid=np.array(f.valid, np.float32), reset=np.array(f.reset, np.float32),
                initial=None if f.initial is None else np.array(f.initial, np.float32),
                dO=bf(f.upstream), dF=np.array(f.final_adjoint, np.float32),
                dS=np.array(f.score_adjoint, np.float32))
