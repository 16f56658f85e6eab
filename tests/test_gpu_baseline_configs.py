"""Parity at BASELINE.json's full sizes (configs 1-3; config 0 is the golden
vector set of tests/test_gpu_golden.py).

Every (batch, head) sequence of the scan is an independent recurrence, so the
full-size GPU result is checked against the f64 oracle on whole sequences cut
out of the batch (oracle slices), and through size-independent properties:
split continuation (scanning [0, T/2) then [T/2, T) from the carried state
equals one scan) and, for the decode configuration, step-by-step equality with
the scan.  Inputs come from the BASELINE generator (SplitMix64 seed 0).
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


def _cfg(i):
    from delta_mixers.synthetic import CONFIGS, generate
    cfg = CONFIGS[i]
    return cfg, generate(cfg)


def _slice(p, b, h):
    """One sequence (b, h) as a B=1, H=1 problem."""
    return {n: (x[b:b + 1, :, h:h + 1] if x.ndim >= 3 else x[b:b + 1]) for n, x in p.items()}


def _oracle_scalar(p, K, V, initial=None, dO=None):
    a, e, w = oracle.scalar_gates(p["beta"], p["g"], K, V)
    B, T = p["q"].shape[:2]
    ones = np.ones((B, T), np.uint8)
    zeros = np.zeros((B, T), np.uint8)
    fwd = oracle.scan(p["q"], p["k"], p["v"], a, e, w, ones, zeros, initial)
    if dO is None:
        return fwd, None
    g = oracle.backward(p["q"], p["k"], p["v"], a, e, w, ones, zeros, initial, dO)
    db, dg = oracle.scalar_gate_grads(p["g"], g)
    return fwd, (g["q"], g["k"], g["v"], db, dg)


def _run_scalar(dk, p, dtype, chunk, initial=None, with_grad=True):
    xs = {n: dev(p[n], dtype).requires_grad_(with_grad) for n in ("q", "k", "v")}
    xs.update({n: dev(p[n]).requires_grad_(with_grad) for n in ("beta", "g")})
    out, fin, sc = dk.gdn_scalar_scan(xs["q"], xs["k"], xs["v"], xs["beta"], xs["g"],
                                      initial=initial, chunk_size=chunk)
    return xs, out, fin, sc


@pytest.mark.parametrize("b,h", [(0, 0), (15, 7), (9, 3)])
def test_lm512_full_size_oracle_slices(dk, b, h):
    """Config 1 at full size on the chunk-WY MFMA path (bf16, chunk 64)."""
    cfg, p = _cfg(1)
    xs, out, fin, sc = _run_scalar(dk, p, torch.bfloat16, 64)
    (out.float() * dev(p["d_output"])).sum().backward()
    s = _slice(p, b, h)
    (o, f, c), grads = _oracle_scalar(s, cfg.keys, cfg.values, dO=s["d_output"])
    gate("output", out[b:b + 1, :, h:h + 1], o, TOL_BF16)
    gate("final_state", fin[b:b + 1, h:h + 1], f, TOL_BF16)
    gate("scores", sc[b:b + 1, :, h:h + 1], c, TOL_BF16)
    for name, n, ref in zip(("dq", "dk", "dv", "dbeta", "dg"), ("q", "k", "v", "beta", "g"), grads):
        gate(name, xs[n].grad[b:b + 1, :, h:h + 1], ref, TOL_BF16)


def test_lm512_full_size_split_continuation(dk):
    """Scanning [0, 256) then [256, 512) from the carried final state equals one
    scan of [0, 512) (outputs, scores and the final state), on the MFMA path."""
    cfg, p = _cfg(1)
    _, out, fin, sc = _run_scalar(dk, p, torch.bfloat16, 64, with_grad=False)
    half = cfg.time // 2
    first = {n: x[:, :half] for n, x in p.items() if n != "d_output"}
    second = {n: x[:, half:] for n, x in p.items() if n != "d_output"}
    _, o1, f1, s1 = _run_scalar(dk, first, torch.bfloat16, 64, with_grad=False)
    _, o2, f2, s2 = _run_scalar(dk, second, torch.bfloat16, 64, initial=f1, with_grad=False)
    gate("output", torch.cat([o1, o2], 1), host(out), TOL_BF16)
    gate("scores", torch.cat([s1, s2], 1), host(sc), TOL_BF16)
    gate("final_state", f2, host(fin), TOL_BF16)


@pytest.mark.parametrize("b,h", [(0, 0), (3, 15)])
def test_long8k_full_size_oracle_slices(dk, b, h):
    """Config 2 at full size (B4 T8192 H16 d_k = d_v = 128, bf16) on the
    d = 128 chunk-WY MFMA path (128 chunks per sequence): forward and backward
    checked on whole sequences against the f64 oracle."""
    cfg, p = _cfg(2)
    dk.stage_timing(True)
    try:
        xs, out, fin, sc = _run_scalar(dk, p, torch.bfloat16, 64)
        (out.float() * dev(p["d_output"])).sum().backward()
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    assert {"chunk_prep", "state_scan", "chunk_out", "chunk_bprep", "adjoint_scan",
            "chunk_bgrad"} <= ran, f"config 2 must take the chunk-WY path: {sorted(ran)}"
    s = _slice(p, b, h)
    (o, f, c), grads = _oracle_scalar(s, cfg.keys, cfg.values, dO=s["d_output"])
    gate("output", out[b:b + 1, :, h:h + 1], o, TOL_BF16)
    gate("final_state", fin[b:b + 1, h:h + 1], f, TOL_BF16)
    gate("scores", sc[b:b + 1, :, h:h + 1], c, TOL_BF16)
    for name, n, ref in zip(("dq", "dk", "dv", "dbeta", "dg"), ("q", "k", "v", "beta", "g"), grads):
        gate(name, xs[n].grad[b:b + 1, :, h:h + 1], ref, TOL_BF16)


def test_decode_full_size_steps_match_scan(dk):
    """Config 3: 256 x 8 fp32 states, 1024 single-token steps.  Every step's
    output and score, and the final state, match the scan carrying the same
    initial state (the f32 chunk kernels; decode is token-sequential) within the
    f32 gate; one sequence of both is checked against the f64 oracle at the
    reference's gate."""
    cfg, p = _cfg(3)
    B, T, H, K, V = cfg.batch, cfg.time, cfg.heads, cfg.keys, cfg.values
    q, k, v = dev(p["q"]), dev(p["k"]), dev(p["v"])
    alpha = torch.exp(dev(p["g"]))[..., None]
    beta = dev(p["beta"])[..., None]
    a, e, w = alpha.expand(B, T, H, K), beta.expand(B, T, H, K), beta.expand(B, T, H, V)
    s0 = dev(p["state"])
    valid = torch.ones((B, T), device="cuda")
    reset = torch.zeros((B, T), device="cuda")
    r = dk.gdn_training_scan(q, k, v, a, e, w, valid, reset, s0, 16)
    state = s0.clone()
    outs, scs = [], []
    for t in range(T):
        sl = slice(t, t + 1)
        o, sc = dk.gdn_decode_step(state, q[:, sl], k[:, sl], v[:, sl], a[:, sl], e[:, sl],
                                   w[:, sl], valid[:, sl], reset[:, sl])
        outs.append(o)
        scs.append(sc)
    dec_out, dec_sc = torch.cat(outs, 1), torch.cat(scs, 1)
    gate("decode output vs scan", dec_out, host(r.output), TOL_F32)
    gate("decode scores vs scan", dec_sc, host(r.scores[..., 0]), TOL_F32)
    gate("decode state vs scan", state, host(r.final_state), TOL_F32)
    b, h = 17, 5
    s = _slice(p, b, h)
    ah, eh, wh = (host(x[b:b + 1, :, h:h + 1]) for x in (a, e, w))
    ones = np.ones((1, T), np.uint8)
    zeros = np.zeros((1, T), np.uint8)
    o, f, c = oracle.scan(s["q"], s["k"], s["v"], ah, eh, wh, ones, zeros,
                          p["state"][b:b + 1, h:h + 1])
    gate("output", r.output[b:b + 1, :, h:h + 1], o, TOL_F32, ref_gate=True)
    gate("final_state", r.final_state[b:b + 1, h:h + 1], f, TOL_F32, ref_gate=True)
    gate("scores", r.scores[b:b + 1, :, h:h + 1, 0], c, TOL_F32, ref_gate=True)
    gate("decode output", dec_out[b:b + 1, :, h:h + 1], o, TOL_F32, ref_gate=True)
    gate("decode state", state[b:b + 1, h:h + 1], f, TOL_F32, ref_gate=True)
