"""Slow-decay parity of every chunk-WY path against the f64 oracle.

With fast decays (g = -softplus(N(0, 1)), alpha about 0.45 per token) the
state that crosses a 64-token chunk is scaled by about e^-50, so errors that
compound through the chunk-to-chunk state chain never show.  These problems
keep the chain alive over the whole sequence:

* scalar gates alpha = e^g drawn from [0.90, 0.99] (the reference
  benchmark's draw, crates/experiment/src/kron_benchmark.rs:89) and from
  [0.999, 1], at T = 8192 (128 chunks of 64) for d = 64 and d = 128, and at
  T = 32768 (512 chunks) for d = 64;
* channel-wise gates alpha in [0.90, 0.99] per channel, and the reference
  gate-fixture law alpha = 0.91 + 0.03 sin(...) (crates/mixers/src/checks.rs:138)
  with its erase/write law and masks, at K = V = 64 and T = 2048 (128 chunks of
  16).

Each problem has padding, resets (one early, so a chain of about 126 chunks
follows it), an initial state and all three adjoints (output, final state,
scores), and every gradient including d_initial is gated.  The stage timers
show that the chunk kernels produced each result.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import fixtures as fx  # noqa: E402
from chunk_util import (chunk_stages, cw_oracle, cw_problem, fixture_problem,  # noqa: E402
                        problem, scalar_oracle_grads, slow_decay)
from gpu_util import TOL_BF16, dev, gate  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu

CW_STAGES = {"chunk_prep", "state_scan", "chunk_out", "chunk_bprep", "adjoint_scan",
             "chunk_bgrad"}
GATES = ("alpha", "erase", "write")


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def _scalar_fwd_bwd(dk, p):
    x = {n: dev(p[n], torch.bfloat16) for n in ("q", "k", "v")}
    x.update({n: dev(p[n]) for n in ("beta", "g", "valid", "reset", "initial")})
    dk.stage_timing(True)
    try:
        out, fin, sc, ck = dk.gdn_scalar_forward(x["q"], x["k"], x["v"], x["beta"], x["g"],
                                                 x["valid"], x["reset"], x["initial"], 64)
        grads = dk.gdn_scalar_backward(x["q"], x["k"], x["v"], x["beta"], x["g"], x["valid"],
                                       x["reset"], ck, 64, dev(p["dO"], torch.bfloat16),
                                       dev(p["dF"]), dev(p["dS"]))
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    return (out, fin, sc), grads, ran


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("lo,hi", [(0.90, 0.99), (0.999, 1.0)])
def test_scalar_slow_decay_8192(dk, D, lo, hi):
    T = 8192
    p = slow_decay(problem(900 + D, 2, T, 2, masks=True, K=D, V=D), lo, hi, D)
    p["reset"][1] = 0  # row 1: one chain from the initial state to the final state
    print(f"slow decay scalar: D={D} alpha in [{lo}, {hi}] T={T}", flush=True)
    (out, fin, sc), grads, ran = _scalar_fwd_bwd(dk, p)
    assert chunk_stages(D) <= ran, f"chunk kernels did not all run: {sorted(ran)}"
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], D, D)
    o_out, o_fin, o_sc = oracle.scan(p["q"], p["k"], p["v"], a, e, w, p["valid"], p["reset"],
                                     p["initial"])
    pad = (p["valid"] == 0)[:, :, None]
    gate("output", out, o_out, TOL_BF16, exact_zero=pad[..., None])
    gate("final_state", fin, o_fin, TOL_BF16)
    gate("scores", sc, o_sc, TOL_BF16, exact_zero=pad)
    og, odb, odg = scalar_oracle_grads(p)
    dq, dkk, dv, db, dg, dinit = grads
    gate("dq", dq, og["q"], TOL_BF16, exact_zero=pad[..., None])
    gate("dk", dkk, og["k"], TOL_BF16, exact_zero=pad[..., None])
    gate("dv", dv, og["v"], TOL_BF16, exact_zero=pad[..., None])
    gate("dbeta", db, odb, TOL_BF16, exact_zero=pad)
    gate("dg", dg, odg, TOL_BF16, exact_zero=pad)
    gate("d_initial", dinit, og["initial"], TOL_BF16)


def test_scalar_slow_decay_32768_d64(dk):
    """512 chunks of 64 with alpha in [0.999, 1]: row 1 carries one chain from
    the initial state to the final state through every chunk, so the errors of
    the dense-map scans (maps and their f32 additive terms) compound over four
    times the 8192-token tests; the final state and d_initial are gated with
    everything else."""
    T, D = 32768, 64
    p = slow_decay(problem(777, 2, T, 1, masks=True, K=D, V=D), 0.999, 1.0, D)
    p["reset"][1] = 0
    print(f"slow decay scalar: D={D} alpha in [0.999, 1] T={T}", flush=True)
    (out, fin, sc), grads, ran = _scalar_fwd_bwd(dk, p)
    assert chunk_stages(D) <= ran, f"chunk kernels did not all run: {sorted(ran)}"
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], D, D)
    o_out, o_fin, o_sc = oracle.scan(p["q"], p["k"], p["v"], a, e, w, p["valid"], p["reset"],
                                     p["initial"])
    pad = (p["valid"] == 0)[:, :, None]
    gate("output", out, o_out, TOL_BF16, exact_zero=pad[..., None])
    gate("final_state", fin, o_fin, TOL_BF16)
    og, odb, odg = scalar_oracle_grads(p)
    dq, dkk, dv, db, dg, dinit = grads
    gate("dq", dq, og["q"], TOL_BF16, exact_zero=pad[..., None])
    gate("dk", dkk, og["k"], TOL_BF16, exact_zero=pad[..., None])
    gate("dg", dg, odg, TOL_BF16, exact_zero=pad)
    gate("d_initial", dinit, og["initial"], TOL_BF16)


def _cw_run(dk, p):
    x = {n: dev(p[n], torch.bfloat16).requires_grad_(True) for n in ("q", "k", "v")}
    x.update({n: dev(p[n]).requires_grad_(True) for n in GATES})
    init = dev(p["initial"]).requires_grad_(True)
    dk.stage_timing(True)
    try:
        r = dk.gdn_training_scan(x["q"], x["k"], x["v"], *(x[n] for n in GATES),
                                 dev(p["valid"]), dev(p["reset"]), init, 16)
        loss = ((r.output.float() * dev(p["dO"])).sum() + (r.final_state * dev(p["dF"])).sum()
                + (r.scores[..., 0] * dev(p["dS"])).sum())
        loss.backward()
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    grads = {n: x[n].grad for n in x}
    grads["initial"] = init.grad
    return r, grads, ran


def _cw_check(p, r, grads):
    (o_out, o_fin, o_sc), og = cw_oracle(p)
    pad = (p["valid"] == 0)[:, :, None]
    gate("output", r.output, o_out, TOL_BF16, exact_zero=pad[..., None])
    gate("final_state", r.final_state, o_fin, TOL_BF16)
    gate("scores", r.scores[..., 0], o_sc, TOL_BF16, exact_zero=pad)
    for n in ("q", "k", "v") + GATES:
        gate(f"d{n}", grads[n], og[n], TOL_BF16, exact_zero=pad[..., None])
    gate("d_initial", grads["initial"], og["initial"], TOL_BF16)


def test_cw_slow_decay_uniform_2048(dk):
    p = cw_problem(4242, 2, 2048, 2, masks=True, alpha_lo=0.90, alpha_hi=0.99)
    p["reset"][1] = 0
    print("slow decay channel-wise: alpha in [0.90, 0.99] T=2048", flush=True)
    r, grads, ran = _cw_run(dk, p)
    assert CW_STAGES <= ran, sorted(ran)
    _cw_check(p, r, grads)


def test_cw_fixture_law_2048(dk):
    """The gate fixture's value laws (alpha = 0.91 + 0.03 sin, erase and write
    0.45 + 0.1 sin, unit k and v rows, its valid and reset patterns, initial
    state, upstream, final and score adjoints) at K = V = 64, B = 2, H = 2,
    T = 2048, without the alpha = 0 edits (those are gated with the exact
    alpha gradient elsewhere)."""
    T = 2048
    f = fx.gate_fixture(T, 0, K=64, V=64, b=2, h=2)
    f["alpha"] = fx.gdn_fixture(T, 64, 64, 2, 2).alpha
    p = fixture_problem(f)
    print("slow decay channel-wise: gate-fixture law T=2048", flush=True)
    r, grads, ran = _cw_run(dk, p)
    assert CW_STAGES <= ran, sorted(ran)
    _cw_check(p, r, grads)
