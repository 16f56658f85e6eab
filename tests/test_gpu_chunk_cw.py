"""GPU parity of the channel-wise chunk-WY MFMA path (the training op
gdn_training_scan with bf16 q/k/v and d_k = d_v = 64; csrc/gdn2_chunk_cw.hip)
against the f64 oracle: per-channel gates, masks, resets (on valid and on
padded tokens, at chunk starts), an initial state, every adjoint (output,
final state, scores), ragged lengths, several heads, sequences past 16 chunks
(the scan's rolled loop), broadcast gate views and strong decays.  The stage
timers show that the chunk kernels, not the token-sequential kernels,
produced each result."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from chunk_util import cw_oracle, cw_problem  # noqa: E402
from gpu_util import TOL_BF16, dev, gate  # noqa: E402

pytestmark = pytest.mark.gpu

FWD_STAGES = {"chunk_prep", "state_scan", "chunk_out"}
BWD_STAGES = {"chunk_bprep", "adjoint_scan", "chunk_bgrad"}
GATES = ("alpha", "erase", "write")


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def _inputs(p, grad=True):
    x = {n: dev(p[n], torch.bfloat16) for n in ("q", "k", "v")}
    x.update({n: dev(p[n]) for n in GATES})
    if grad:
        for t in x.values():
            t.requires_grad_(True)
    init = dev(p["initial"])
    if init is not None and grad:
        init.requires_grad_(True)
    return x, init


def _run(dk, p, use_final=True, use_scores=True, chunk=16, gates=None):
    """Forward and backward through delta_kernels.gdn_training_scan with the
    stage timers on; returns (outputs, grads, stages that ran)."""
    x, init = _inputs(p)
    g = gates(x) if gates else [x[n] for n in GATES]
    dk.stage_timing(True)
    try:
        r = dk.gdn_training_scan(x["q"], x["k"], x["v"], *g, dev(p["valid"]), dev(p["reset"]),
                                 init, chunk)
        loss = (r.output.float() * dev(p["dO"])).sum()
        if use_final:
            loss = loss + (r.final_state * dev(p["dF"])).sum()
        if use_scores:
            loss = loss + (r.scores[..., 0] * dev(p["dS"])).sum()
        loss.backward()
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    grads = {n: x[n].grad for n in x}
    if init is not None:
        grads["initial"] = init.grad
    return r, grads, ran


def _check(p, r, grads, use_final=True, use_scores=True, skip=()):
    (o_out, o_fin, o_sc), og = cw_oracle(p, use_final, use_scores)
    pad = (p["valid"] == 0)[:, :, None]
    gate("output", r.output, o_out, TOL_BF16, exact_zero=pad[..., None])
    gate("final_state", r.final_state, o_fin, TOL_BF16)
    gate("scores", r.scores[..., 0], o_sc, TOL_BF16, exact_zero=pad)
    for n in ("q", "k", "v") + GATES:
        if n not in skip:
            gate(f"d{n}", grads[n], og[n], TOL_BF16, exact_zero=pad[..., None])
    if "initial" in grads:
        gate("d_initial", grads["initial"], og["initial"], TOL_BF16)
    return og


@pytest.mark.parametrize("B,T,H", [(1, 16, 1), (2, 37, 2), (1, 200, 3), (2, 64, 1)])
@pytest.mark.parametrize("masks", [False, True])
def test_cw_matches_oracle(dk, B, T, H, masks):
    p = cw_problem(B * 100 + T + masks, B, T, H, masks=masks)
    print(f"cw: B={B} T={T} H={H} masks={masks}", flush=True)
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran, sorted(ran)
    _check(p, r, grads)


def test_cw_output_adjoint_only_no_initial(dk):
    p = cw_problem(3, 2, 150, 2, masks=True, initial=False)
    r, grads, ran = _run(dk, p, use_final=False, use_scores=False)
    assert BWD_STAGES <= ran
    _check(p, r, grads, use_final=False, use_scores=False)


def test_cw_resets_at_chunk_edges(dk):
    """Resets on the first token of a chunk, on token 0, on the last token of a
    chunk and on a padded token; a chunk that is all padding."""
    p = cw_problem(17, 2, 96, 1, masks=False)
    p["reset"][0, [0, 16, 31, 47]] = 1
    p["valid"][0, 64:80] = 0
    p["reset"][0, 70] = 1  # on padding: ignored
    p["reset"][1, [15, 17, 33]] = 1
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    _check(p, r, grads)


@pytest.mark.parametrize("T,reset_every", [(256, 0), (1000, 300), (2048, 700)])
def test_cw_long(dk, T, reset_every):
    """16, 63 and 128 chunks of 16 tokens: the scan's straight-line form and
    its rolled loop, with bf16 chunk maps chained over the whole sequence."""
    p = cw_problem(T, 1, T, 2, masks=True, reset_every=reset_every)
    print(f"cw long: T={T} chunks={-(-T // 16)}", flush=True)
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    _check(p, r, grads)


def test_cw_strong_decay(dk):
    """alpha down to 1e-3: the decays underflow the chunk within a few tokens.
    The alpha gradient itself is gated (it is formed without dividing by
    alpha)."""
    p = cw_problem(29, 1, 80, 2, masks=True, alpha_lo=1e-3)
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    _check(p, r, grads)


@pytest.mark.parametrize("tiny", [1e-4, 1e-6, 1e-20])
def test_cw_tiny_alpha_gradient(dk, tiny):
    """alpha at 1e-4, 1e-6 and 1e-20 on a scattering of tokens and channels
    (and in [1e-3, 1e-2] elsewhere on some rows): dalpha is finite and matches
    the oracle, where dividing a log-domain gradient by alpha would blow up."""
    p = cw_problem(31, 2, 70, 2, masks=True)
    rng = np.random.default_rng(7)
    pick = rng.random(p["alpha"].shape) < 0.08
    p["alpha"][pick] = tiny
    p["alpha"][0, 20:40] = rng.uniform(1e-3, 1e-2, size=p["alpha"][0, 20:40].shape).astype(np.float32)
    print(f"cw tiny alpha {tiny}", flush=True)
    r, grads, ran = _run(dk, p)
    assert BWD_STAGES <= ran
    assert torch.isfinite(grads["alpha"]).all()
    _check(p, r, grads)


def test_cw_alpha_zero_exact_gradient(dk):
    """alpha exactly 0 (an underflowed gate) on one channel of a token and on
    every channel of another: outputs, states and every gradient, dalpha
    included, match the oracle (whose dalpha there is the pre-decay state
    adjoint times the state, nonzero)."""
    p = cw_problem(78, 1, 40, 2, masks=False)
    p["alpha"][0, 10, 0, :8] = 0.0
    p["alpha"][0, 27, 1, :] = 0.0
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    og = _check(p, r, grads)
    assert np.abs(og["alpha"][0, 10, 0, :8]).max() > 0  # the exact gradient is not zero there


def test_cw_negative_alpha_fails_loudly(dk):
    """A negative alpha is outside the chunk kernels' log-domain decays: the
    sequence that holds it gets NaN outputs (never finite wrong values), the
    other sequences are untouched, and the f32 chunk kernels give the oracle's
    values for the same inputs."""
    p = cw_problem(83, 2, 40, 1, masks=False)
    p["alpha"][1, 12, 0, 5] = -0.5
    x, init = _inputs(p, grad=False)
    r = dk.gdn_training_scan(x["q"], x["k"], x["v"], x["alpha"], x["erase"], x["write"],
                             dev(p["valid"]), dev(p["reset"]), init, 16)
    torch.cuda.synchronize()
    out = r.output.float().cpu().numpy()
    assert np.isnan(out[1, 12:]).any(), "a negative alpha must not give finite outputs"
    (o_out, o_fin, _), _ = cw_oracle(p)
    gate("output of the sequence without a negative alpha", r.output[0], o_out[0], TOL_BF16)
    xf = {n: dev(p[n]) for n in ("q", "k", "v")}
    rf = dk.gdn_training_scan(xf["q"], xf["k"], xf["v"], x["alpha"], x["erase"], x["write"],
                              dev(p["valid"]), dev(p["reset"]), init, 16)
    gate("f32 (chunk kernels) output with a negative alpha", rf.output, o_out, 1e-4)
    gate("f32 (chunk kernels) final state with a negative alpha", rf.final_state, o_fin, 1e-4)


@pytest.mark.parametrize("t,mode", [(7, 0), (35, 0), (35, 1), (35, 2), (35, 3)])
def test_cw_gate_fixture_k64(dk, t, mode):
    """The reference GDN gate fixture with all its edits (crates/mixers/src/
    kron_checks.rs:124-188: reset on padding, an all-padding chunk, a zero edit,
    a negative write, zero key and value norms, alpha zero on one channel at
    p = 2 and on every channel at p = 16, a nonzero initial state, the four
    objectives) at K = V = 64 in bf16 through the channel-wise chunk kernels."""
    import fixtures as fx
    from chunk_util import fixture_problem
    p = fixture_problem(fx.gate_fixture(t, mode, K=64, V=64))
    print(f"cw gate fixture K=V=64 T={t} mode={mode}", flush=True)
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    _check(p, r, grads)


def test_cw_broadcast_gates(dk):
    """Gates handed over as stride-0 views: alpha and erase shared by the
    channels of a head ([B,T,H,1] expanded), write shared by the heads."""
    B, T, H = 1, 70, 2
    p = cw_problem(41, B, T, H, masks=True)
    p["alpha"] = np.broadcast_to(p["alpha"][..., :1], p["alpha"].shape).copy()
    p["erase"] = np.broadcast_to(p["erase"][..., :1], p["erase"].shape).copy()
    p["write"] = np.broadcast_to(p["write"][:, :, :1], p["write"].shape).copy()

    def views(x):
        return [x["alpha"][..., :1].expand(B, T, H, 64), x["erase"][..., :1].expand(B, T, H, 64),
                x["write"][:, :, :1].expand(B, T, H, 64)]
    r, grads, ran = _run(dk, p, gates=views)
    assert FWD_STAGES | BWD_STAGES <= ran
    (o_out, o_fin, o_sc), og = cw_oracle(p)
    gate("output", r.output, o_out, TOL_BF16)
    gate("final_state", r.final_state, o_fin, TOL_BF16)
    # the leaf gradients are the sums over the broadcast axes
    gate("dalpha (summed)", grads["alpha"][..., :1], og["alpha"].sum(-1, keepdims=True), TOL_BF16)
    gate("derase (summed)", grads["erase"][..., :1], og["erase"].sum(-1, keepdims=True), TOL_BF16)
    gate("dwrite (summed)", grads["write"][:, :, :1], og["write"].sum(2, keepdims=True), TOL_BF16)
    for n in ("q", "k", "v"):
        gate(f"d{n}", grads[n], og[n], TOL_BF16)


def test_cw_split_continuation(dk):
    """T = 96 scanned whole equals [0, 40) then [40, 96) from the carried state
    (a split inside a 16-token chunk); the two halves' backward, chained through
    the state adjoint, equals the whole sequence's backward."""
    T, cut = 96, 40
    p = cw_problem(53, 2, T, 2, masks=True)
    r, grads, _ = _run(dk, p)
    seq = ("q", "k", "v", "alpha", "erase", "write", "valid", "reset", "dO", "dS")
    first = {n: (p[n][:, :cut] if n in seq else p[n]) for n in p}
    second = {n: (p[n][:, cut:] if n in seq else p[n]) for n in p}
    x1, i1 = _inputs(first, grad=False)
    x2, _ = _inputs(second, grad=False)
    f = dk._training_forward(x1["q"], x1["k"], x1["v"], x1["alpha"], x1["erase"], x1["write"],
                             dev(first["valid"]), dev(first["reset"]), i1, 16)
    s = dk._training_forward(x2["q"], x2["k"], x2["v"], x2["alpha"], x2["erase"], x2["write"],
                             dev(second["valid"]), dev(second["reset"]), f[1], 16)
    gate("output (split)", torch.cat([f[0], s[0]], 1), r.output.detach().float().cpu().numpy(),
         TOL_BF16)
    gate("final_state (split)", s[1], r.final_state.detach().cpu().numpy(), TOL_BF16)
    g2 = dk.gdn_training_backward(x2["q"], x2["k"], x2["v"], x2["alpha"], x2["erase"],
                                  x2["write"], dev(second["valid"]), dev(second["reset"]), s[3],
                                  16, dev(second["dO"], torch.bfloat16), dev(p["dF"]),
                                  dev(second["dS"]))
    g1 = dk.gdn_training_backward(x1["q"], x1["k"], x1["v"], x1["alpha"], x1["erase"],
                                  x1["write"], dev(first["valid"]), dev(first["reset"]), f[3],
                                  16, dev(first["dO"], torch.bfloat16), g2[6], dev(first["dS"]))
    for i, n in enumerate(("q", "k", "v") + GATES):
        gate(f"d{n} (split)", torch.cat([g1[i], g2[i]], 1), grads[n].float().cpu().numpy(),
             TOL_BF16)
    gate("d_initial (split)", g1[6], grads["initial"].cpu().numpy(), TOL_BF16)


def test_scan_selected_reaches_mfma(dk):
    """The reference's mixer entry (scan_selected with the fused GDN-2
    backend) runs the chunk kernels for bf16 d = 64 inputs."""
    from delta_mixers import MixerKind, ScanBackend, ScanInput, scan_selected
    p = cw_problem(61, 1, 48, 2, masks=True)
    x, init = _inputs(p, grad=False)
    dk.stage_timing(True)
    try:
        r = scan_selected(ScanBackend.FUSED_GDN2, MixerKind.GDN2,
                          ScanInput(*(x[n] for n in ("q", "k", "v") + GATES)), dev(p["valid"]),
                          dev(p["reset"]), 16, init)
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    assert FWD_STAGES <= ran, sorted(ran)
    (o_out, _, _), _ = cw_oracle(p)
    gate("scan_selected output", r.output, o_out, TOL_BF16)


@pytest.mark.parametrize("T", [1, 15, 17])
def test_cw_short_sequences(dk, T):
    """Fewer tokens than one chunk, and one token past it."""
    p = cw_problem(300 + T, 2, T, 2, masks=False)
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    _check(p, r, grads)


def test_cw_all_padding_row_and_zero_keys(dk):
    """A sequence that is padding throughout keeps its initial state and gets
    zero gradients; zero key rows give zero scores (the zero subgradient of
    |k| |delta|); alpha exactly 1 (no decay) on some channels."""
    p = cw_problem(77, 2, 40, 2, masks=False)
    p["valid"][1, :] = 0
    p["k"][0, 5] = 0.0
    p["k"][0, 21, 1] = 0.0
    p["alpha"][0, 11, 1, 8:16] = 1.0
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    og = _check(p, r, grads)
    fin = r.final_state.detach().cpu().numpy()
    # the scan carries states as a bf16 hi/lo pair: 16 significant bits
    np.testing.assert_allclose(fin[1], p["initial"][1], rtol=2.0 ** -15, atol=1e-7)
    assert np.all(r.scores.detach().cpu().numpy()[0, 5] == 0)
    gate("d_initial (padded row passes dF)", grads["initial"][1], og["initial"][1], TOL_BF16)


def test_cw_many_heads(dk):
    """Twelve (batch, head) sequences: more than one group of eight heads in the
    scan's workgroup mapping, the last group partly empty."""
    p = cw_problem(91, 3, 100, 4, masks=True)
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    _check(p, r, grads)


def _cw_slice(p, b, h):
    """Sequence (b, h) of a cw_problem as a B = 1, H = 1 problem."""
    out = {}
    for n, x in p.items():
        if x is None:
            out[n] = None
        elif n in ("initial", "dF"):      # [B, H, K, V]
            out[n] = x[b:b + 1, h:h + 1]
        elif x.ndim == 2:                 # [B, T]
            out[n] = x[b:b + 1]
        else:                             # [B, T, H, ...]
            out[n] = x[b:b + 1, :, h:h + 1]
    return out


def test_cw_full_shape_oracle_slices(dk):
    """The document-scan benchmark's head shape (B16 T512 H8: 128 heads, 32
    chunks each) with masks, resets and an initial state; whole sequences cut
    out of the batch against the f64 oracle."""
    p = cw_problem(97, 16, 512, 8, masks=True)
    r, grads, ran = _run(dk, p)
    assert FWD_STAGES | BWD_STAGES <= ran
    for b, h in [(0, 0), (15, 7), (9, 3)]:
        s = _cw_slice(p, b, h)
        (o_out, o_fin, o_sc), og = cw_oracle(s)
        pad = (s["valid"] == 0)[:, :, None]
        gate(f"output ({b},{h})", r.output[b:b + 1, :, h:h + 1], o_out, TOL_BF16, exact_zero=pad[..., None])
        gate(f"final_state ({b},{h})", r.final_state[b:b + 1, h:h + 1], o_fin, TOL_BF16)
        gate(f"scores ({b},{h})", r.scores[b:b + 1, :, h:h + 1, 0], o_sc, TOL_BF16, exact_zero=pad)
        for n in ("q", "k", "v") + GATES:
            gate(f"d{n} ({b},{h})", grads[n][b:b + 1, :, h:h + 1], og[n], TOL_BF16, exact_zero=pad[..., None])
        gate(f"d_initial ({b},{h})", grads["initial"][b:b + 1, h:h + 1], og["initial"], TOL_BF16)
