"""The chunk-WY MFMA path on long sequences (more than 8 chunks per sequence),
against the f64 oracle, and through the split-continuation property.

T = 1000, 2048 and 8192 give 16, 32 and 128 chunks per sequence: the state and
adjoint scans' straight-line instantiation for 16 chunks and the rolled loop
that every longer sequence takes.  The checkpoint holds the chunk-start state
and the state maps in bf16, so these sizes also show whether those single
roundings stay inside the bf16 gate over 128 chained chunks.  Each test
asserts through the stage timers that the chunk kernels (not the
token-sequential fallback) produced the result.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from chunk_util import chunk_stages, problem, scalar_oracle_grads  # noqa: E402
from gpu_util import TOL_BF16, dev, gate  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def _inputs(p):
    x = {n: dev(p[n], torch.bfloat16) for n in ("q", "k", "v")}
    x.update({n: dev(p[n]) for n in ("beta", "g", "valid", "reset")})
    x["initial"] = dev(p["initial"])
    return x


def _fwd_bwd(dk, p, use_final=True, use_scores=True):
    """Forward and backward through the C ABI with the stage timers on;
    returns the forward outputs, the gradients and the stages that ran."""
    x = _inputs(p)
    dk.stage_timing(True)
    try:
        out, fin, sc, ck = dk.gdn_scalar_forward(x["q"], x["k"], x["v"], x["beta"], x["g"],
                                                 x["valid"], x["reset"], x["initial"], 64)
        grads = dk.gdn_scalar_backward(x["q"], x["k"], x["v"], x["beta"], x["g"], x["valid"],
                                       x["reset"], ck, 64, dev(p["dO"], torch.bfloat16),
                                       dev(p["dF"]) if use_final else None,
                                       dev(p["dS"]) if use_scores else None)
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    return (out, fin, sc), grads, ran


@pytest.mark.parametrize("T,H,reset_every", [(1000, 2, 300), (2048, 1, 700), (8192, 1, 2500)])
def test_long_chunk_path_matches_oracle(dk, T, H, reset_every):
    p = problem(T + H, 1, T, H, masks=True, reset_every=reset_every)
    print(f"chunk long: T={T} H={H} chunks={-(-T // 64)}", flush=True)
    (out, fin, sc), grads, ran = _fwd_bwd(dk, p)
    assert chunk_stages(64) <= ran, f"chunk kernels did not all run: {sorted(ran)}"
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], 64, 64)
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


@pytest.mark.parametrize("D", [64, 128])
def test_chunk_loops_uneven_split(dk, D):
    """336 chunks (B3 T1000 H7): the kernels that walk chunks with one workgroup
    per CU get more chunks than workgroups but not a multiple of them, so some
    workgroups walk two chunks and others one (the last chunk's stores come
    after the loop); d_k = d_v = 64 and 128, with masks and resets."""
    p = problem(77 + D, 3, 1000, 7, masks=True, K=D, V=D, reset_every=300)
    print(f"chunk loops: B3 T1000 H7 D={D}, 336 chunks", flush=True)
    (out, fin, sc), grads, ran = _fwd_bwd(dk, p)
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


@pytest.mark.parametrize("D", [64, 128])
def test_long_split_continuation(dk, D):
    """T = 8192 (128 chunks) scanned whole equals [0, 4096) then [4096, 8192)
    from the carried state; the backward of the two halves, chained through
    the state adjoint (the second half's d_initial is the first half's final
    adjoint), equals the whole sequence's backward.  d_k = d_v = 64 and 128."""
    T, half = 8192, 4096
    p = problem(11, 2, T, 2, masks=False, K=D, V=D)
    whole_fwd, whole_grads, ran = _fwd_bwd(dk, p)
    assert chunk_stages(D) <= ran
    first = {n: (x[:, :half] if x is not None and x.ndim in (2, 3, 4) and x.shape[1] == T else x)
             for n, x in p.items()}
    second = {n: (x[:, half:] if x is not None and x.ndim in (2, 3, 4) and x.shape[1] == T
                  else x) for n, x in p.items()}
    x1 = _inputs(first)
    o1, f1, s1, ck1 = dk.gdn_scalar_forward(x1["q"], x1["k"], x1["v"], x1["beta"], x1["g"],
                                            x1["valid"], x1["reset"], x1["initial"], 64)
    x2 = _inputs(second)
    o2, f2, s2, ck2 = dk.gdn_scalar_forward(x2["q"], x2["k"], x2["v"], x2["beta"], x2["g"],
                                            x2["valid"], x2["reset"], f1, 64)
    out, fin, sc = whole_fwd
    gate("output", torch.cat([o1, o2], 1), out.float().cpu().numpy(), TOL_BF16)
    gate("scores", torch.cat([s1, s2], 1), sc.cpu().numpy(), TOL_BF16)
    gate("final_state", f2, fin.cpu().numpy(), TOL_BF16)
    g2 = dk.gdn_scalar_backward(x2["q"], x2["k"], x2["v"], x2["beta"], x2["g"], x2["valid"],
                                x2["reset"], ck2, 64, dev(second["dO"], torch.bfloat16),
                                dev(p["dF"]), dev(second["dS"]))
    g1 = dk.gdn_scalar_backward(x1["q"], x1["k"], x1["v"], x1["beta"], x1["g"], x1["valid"],
                                x1["reset"], ck1, 64, dev(first["dO"], torch.bfloat16),
                                g2[5], dev(first["dS"]))
    names = ("dq", "dk", "dv", "dbeta", "dg")
    for i, name in enumerate(names):
        got = torch.cat([g1[i], g2[i]], 1)
        gate(f"{name} (split)", got, whole_grads[i].float().cpu().numpy(), TOL_BF16)
    gate("d_initial (split)", g1[5], whole_grads[5].cpu().numpy(), TOL_BF16)


def test_broadcast_upstream_from_sum(dk):
    """out.sum().backward() hands the backward an expanded (stride-0) upstream
    gradient; the chunk path takes it (as a dense copy) and matches the oracle
    with dO = 1."""
    p = problem(5, 1, 130, 1, masks=False, initial=False)
    x = {n: dev(p[n], torch.bfloat16).requires_grad_(True) for n in ("q", "k", "v")}
    beta = dev(p["beta"]).requires_grad_(True)
    g = dev(p["g"]).requires_grad_(True)
    out, fin, sc = dk.gdn_scalar_scan(x["q"], x["k"], x["v"], beta, g)
    out.sum().backward()
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], 64, 64)
    ones = np.ones((1, 130), np.uint8)
    zeros = np.zeros((1, 130), np.uint8)
    og = oracle.backward(p["q"], p["k"], p["v"], a, e, w, ones, zeros, None,
                         np.ones((1, 130, 1, 64)))
    db, dg = oracle.scalar_gate_grads(p["g"], og)
    gate("dq", x["q"].grad, og["q"], TOL_BF16)
    gate("dk", x["k"].grad, og["k"], TOL_BF16)
    gate("dv", x["v"].grad, og["v"], TOL_BF16)
    gate("dbeta", beta.grad, db, TOL_BF16)
    gate("dg", g.grad, dg, TOL_BF16)
