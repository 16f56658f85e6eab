"""GPU parity of the chunk-WY MFMA path (scalar gates, bf16, d_k = d_v = 64,
chunk 64) against the f64 oracle, and against the token-sequential GPU kernels
at the full BASELINE configs[1] size through size-independent properties."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from chunk_util import problem, run_bwd, run_fwd, scalar_oracle_grads  # noqa: E402
from gpu_util import TOL_BF16, dev, gate, host  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


@pytest.mark.parametrize("B,T,H", [(1, 64, 1), (2, 200, 2), (1, 130, 3)])
@pytest.mark.parametrize("masks", [False, True])
def test_chunk_forward_matches_oracle(dk, B, T, H, masks):
    p = problem(B * 1000 + T + masks, B, T, H, masks=masks)
    out, fin, sc = run_fwd(dk, p)
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], 64, 64)
    o_out, o_fin, o_sc = oracle.scan(p["q"], p["k"], p["v"], a, e, w, p["valid"], p["reset"],
                                     p["initial"])
    pad = (p["valid"] == 0)[:, :, None]
    gate("output", out, o_out, TOL_BF16, exact_zero=pad[..., None])
    gate("final_state", fin, o_fin, TOL_BF16)
    gate("scores", sc, o_sc, TOL_BF16, exact_zero=pad)


def test_chunk_forward_full_size_matches_sequential_kernel(dk):
    """BASELINE configs[1] inputs: chunk-WY MFMA forward vs the token-sequential
    GPU kernel (chunk 16 selects it) on the same bf16 inputs."""
    from delta_mixers.synthetic import CONFIGS, generate
    cfg = CONFIGS[1]
    p = generate(cfg)
    B, T, H = cfg.batch, cfg.time, cfg.heads
    p["valid"] = np.ones((B, T), np.float32)
    p["reset"] = np.zeros((B, T), np.float32)
    p["initial"] = None
    o64, f64_, s64 = run_fwd(dk, p, 64)
    o16, f16_, s16 = run_fwd(dk, p, 16)
    gate("output vs sequential", o64, host(o16), TOL_BF16)
    gate("final_state vs sequential", f64_, host(f16_), TOL_BF16)
    gate("scores vs sequential", s64, host(s16), TOL_BF16)


@pytest.mark.parametrize("B,T,H", [(1, 64, 1), (2, 200, 2), (1, 130, 3)])
@pytest.mark.parametrize("masks", [False, True])
def test_chunk_backward_matches_oracle(dk, B, T, H, masks):
    p = problem(7 * B + T + masks, B, T, H, masks=masks)
    dq, dkk, dv, db, dg, dinit = run_bwd(dk, p)
    og, odb, odg = scalar_oracle_grads(p)
    pad = (p["valid"] == 0)[:, :, None]
    gate("dq", dq, og["q"], TOL_BF16, exact_zero=pad[..., None])
    gate("dk", dkk, og["k"], TOL_BF16, exact_zero=pad[..., None])
    gate("dv", dv, og["v"], TOL_BF16, exact_zero=pad[..., None])
    gate("dbeta", db, odb, TOL_BF16, exact_zero=pad)
    gate("dg", dg, odg, TOL_BF16, exact_zero=pad)
    gate("d_initial", dinit, og["initial"], TOL_BF16)


def test_chunk_backward_output_adjoint_only(dk):
    p = problem(3, 2, 150, 2, masks=True)
    p["dF"] = np.zeros_like(p["dF"])
    p["dS"] = np.zeros_like(p["dS"])
    dq, dkk, dv, db, dg, dinit = run_bwd(dk, p, use_final=False, use_scores=False)
    og, odb, odg = scalar_oracle_grads(p)
    for name, got, ref in (("dq", dq, og["q"]), ("dk", dkk, og["k"]), ("dv", dv, og["v"]),
                           ("dbeta", db, odb), ("dg", dg, odg), ("d_initial", dinit, og["initial"])):
        gate(name, got, ref, TOL_BF16)


def test_chunk_backward_full_size_matches_sequential_kernel(dk):
    """chunk-WY MFMA backward vs the token-sequential GPU
    backward on the same bf16 inputs and upstream dO."""
    from delta_mixers.synthetic import CONFIGS, generate
    cfg = CONFIGS[1]
    p = generate(cfg)
    B, T, H = cfg.batch, cfg.time, cfg.heads
    p["valid"] = np.ones((B, T), np.float32)
    p["reset"] = np.zeros((B, T), np.float32)
    p["initial"] = None
    p["dO"] = p["d_output"]
    p["dF"] = np.zeros((B, H, 64, 64), np.float32)
    p["dS"] = np.zeros((B, T, H), np.float32)
    g64 = run_bwd(dk, p, 64, use_final=False, use_scores=False)
    g16 = run_bwd(dk, p, 16, use_final=False, use_scores=False)
    for name, a, b in zip(("dq", "dk", "dv", "dbeta", "dg"), g64[:5], g16[:5]):
        gate(f"{name} vs sequential", a, host(b), TOL_BF16)


@pytest.mark.parametrize("B,T,H", [(2, 200, 2)])
def test_autograd_passes_absent_adjoints_as_none(dk, B, T, H):
    """Only the output feeds the loss: autograd hands the backward None for the
    final-state and score adjoints (no zero tensors), and the gradients equal,
    bit for bit, the raw backward given explicit zero adjoints."""
    p = problem(21, B, T, H, masks=True)
    x = {n: dev(p[n], torch.bfloat16).requires_grad_(True) for n in ("q", "k", "v")}
    beta, g = dev(p["beta"]).requires_grad_(True), dev(p["g"]).requires_grad_(True)
    valid, reset, init = dev(p["valid"]), dev(p["reset"]), dev(p["initial"])
    dO = dev(p["dO"], torch.bfloat16)
    out, fin, sc = dk.gdn_scalar_scan(x["q"], x["k"], x["v"], beta, g, valid, reset, init)
    out.backward(dO)
    _, _, _, ck = dk.gdn_scalar_forward(x["q"].detach(), x["k"].detach(), x["v"].detach(),
                                        beta.detach(), g.detach(), valid, reset, init, 64)
    ref = dk.gdn_scalar_backward(x["q"].detach(), x["k"].detach(), x["v"].detach(),
                                 beta.detach(), g.detach(), valid, reset, ck, 64, dO,
                                 torch.zeros_like(fin), torch.zeros_like(sc))
    for name, got, want in (("dq", x["q"].grad, ref[0]), ("dk", x["k"].grad, ref[1]),
                            ("dv", x["v"].grad, ref[2]), ("dbeta", beta.grad, ref[3]),
                            ("dg", g.grad, ref[4])):
        assert torch.equal(got, want), f"{name}: None adjoints differ from zero adjoints"
