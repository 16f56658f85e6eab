"""GPU parity of the d_k = d_v = 128 chunk-WY MFMA path (scalar gates, bf16,
chunk 64; csrc/gdn2_chunk_wide.hip) against the f64 oracle, with masks,
resets, an initial state and every adjoint (output, final state, scores), on
ragged lengths and several heads.  The stage timers show that the chunk
kernels, not the token-sequential fallback, produced each result."""
import pytest

torch = pytest.importorskip("torch")

from chunk_util import problem, run_bwd, run_fwd, scalar_oracle_grads  # noqa: E402
from gpu_util import TOL_BF16, gate  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def _timed(dk, fn):
    dk.stage_timing(True)
    try:
        r = fn()
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    return r, ran


@pytest.mark.parametrize("B,T,H", [(1, 64, 1), (2, 200, 2), (1, 130, 3), (3, 130, 3)])
@pytest.mark.parametrize("masks", [False, True])
def test_wide_forward_matches_oracle(dk, B, T, H, masks):
    p = problem(B * 1000 + T + masks, B, T, H, masks=masks, K=D, V=D)
    (out, fin, sc), ran = _timed(dk, lambda: run_fwd(dk, p))
    assert {"chunk_prep", "state_scan", "chunk_out"} <= ran, sorted(ran)
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], D, D)
    o_out, o_fin, o_sc = oracle.scan(p["q"], p["k"], p["v"], a, e, w, p["valid"], p["reset"],
                                     p["initial"])
    pad = (p["valid"] == 0)[:, :, None]
    gate("output", out, o_out, TOL_BF16, exact_zero=pad[..., None])
    gate("final_state", fin, o_fin, TOL_BF16)
    gate("scores", sc, o_sc, TOL_BF16, exact_zero=pad)


@pytest.mark.parametrize("B,T,H", [(1, 64, 1), (2, 200, 2), (1, 130, 3), (3, 130, 3)])
@pytest.mark.parametrize("masks", [False, True])
def test_wide_backward_matches_oracle(dk, B, T, H, masks):
    p = problem(7 * B + T + masks, B, T, H, masks=masks, K=D, V=D)
    grads, ran = _timed(dk, lambda: run_bwd(dk, p))
    assert {"chunk_bprep", "adjoint_scan", "chunk_bgrad"} <= ran, sorted(ran)
    dq, dkk, dv, db, dg, dinit = grads
    og, odb, odg = scalar_oracle_grads(p)
    pad = (p["valid"] == 0)[:, :, None]
    gate("dq", dq, og["q"], TOL_BF16, exact_zero=pad[..., None])
    gate("dk", dkk, og["k"], TOL_BF16, exact_zero=pad[..., None])
    gate("dv", dv, og["v"], TOL_BF16, exact_zero=pad[..., None])
    gate("dbeta", db, odb, TOL_BF16, exact_zero=pad)
    gate("dg", dg, odg, TOL_BF16, exact_zero=pad)
    gate("d_initial", dinit, og["initial"], TOL_BF16)


def test_wide_backward_output_adjoint_only(dk):
    import numpy as np
    p = problem(3, 2, 150, 2, masks=True, K=D, V=D)
    p["dF"] = np.zeros_like(p["dF"])
    p["dS"] = np.zeros_like(p["dS"])
    dq, dkk, dv, db, dg, dinit = run_bwd(dk, p, use_final=False, use_scores=False)
    og, odb, odg = scalar_oracle_grads(p)
    for name, got, ref in (("dq", dq, og["q"]), ("dk", dkk, og["k"]), ("dv", dv, og["v"]),
                           ("dbeta", db, odb), ("dg", dg, odg), ("d_initial", dinit, og["initial"])):
        gate(name, got, ref, TOL_BF16)
