"""GPU parity of the channel-wise GDN-2 training scan (C ABI via delta_kernels)
against the f64 oracle, on the reference's own fixtures and edge cases.

Mirrors the reference's GDN gate (crates/mixers/src/kron_checks.rs:89-524):
T in {1, 7, 35}, objectives 0..3, strided uploads, split continuation inside a
chunk; plus chunk_tests.rs:25-238 (reset on padding, nonzero initial state,
chunk sizes 1/2/5/16).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import fixtures as fx  # noqa: E402
from gpu_util import TOL_BF16, TOL_F32, dev, gate  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu

GROUPS = ("q", "k", "v", "alpha", "erase", "write")


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def run_scan(dk, f, chunk=16, dtype=torch.float32, initial=True, strided=False):
    def up(name):
        x = f[name]
        t = dev(x, dtype if name in ("q", "k", "v") else torch.float32)
        if strided:  # genuine noncontiguous view: physical [B,H,T,W] (kron_checks.rs:526-553)
            t = t.transpose(1, 2).contiguous().transpose(1, 2)
        return t.requires_grad_(True)
    xs = {n: up(n) for n in GROUPS}
    init = dev(f["initial"]).requires_grad_(True) if (initial and f.get("initial") is not None) \
        else None
    valid, reset = dev(f.valid), dev(f.reset)
    if strided:
        valid = valid.t().contiguous().t()
        reset = reset.t().contiguous().t()
    r = dk.gdn_training_scan(xs["q"], xs["k"], xs["v"], xs["alpha"], xs["erase"], xs["write"],
                             valid, reset, init, chunk)
    return xs, init, r


def oracle_all(f, initial=True):
    init = f.get("initial") if initial else None
    out, fin, sc = oracle.scan(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset, init)
    g = oracle.backward(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset, init,
                        f.upstream, f.final_adjoint, f.score_adjoint)
    return out, fin, sc, g


def loss_terms(r, f):
    loss = (r.output.float() * dev(f.upstream)).sum()
    if f.final_adjoint is not None:
        loss = loss + (r.final_state * dev(f.final_adjoint)).sum()
    if f.score_adjoint is not None:
        loss = loss + (r.scores[..., 0] * dev(f.score_adjoint)).sum()
    return loss


def check_all(dk, f, tol, chunk=16, dtype=torch.float32, strided=False, ref_gate=False):
    xs, init, r = run_scan(dk, f, chunk, dtype, strided=strided)
    out, fin, sc, g = oracle_all(f)
    pad = (f.valid == 0)[:, :, None, None]
    gate("output", r.output, out, tol, exact_zero=pad, ref_gate=ref_gate)
    gate("final_state", r.final_state, fin, tol, ref_gate=ref_gate)
    gate("scores", r.scores[..., 0], sc, tol, exact_zero=pad[..., 0], ref_gate=ref_gate)
    loss_terms(r, f).backward()
    for n in GROUPS:
        gate(f"d{n}", xs[n].grad, g[n], tol, exact_zero=pad, ref_gate=ref_gate)
    if init is not None:
        gate("d_initial", init.grad, g["initial"], tol, ref_gate=ref_gate)


@pytest.mark.parametrize("t", [1, 7, 35])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_gate_fixture_f32(dk, t, mode):
    check_all(dk, fx.gate_fixture(t, mode), TOL_F32, ref_gate=True)


def test_gate_fixture_strided(dk):
    check_all(dk, fx.gate_fixture(35, 0), TOL_F32, strided=True, ref_gate=True)


@pytest.mark.parametrize("chunk", [1, 2, 5, 16, 64])
def test_reset_padding_fixture(dk, chunk):
    f = fx.reset_padding_fixture()
    f["final_adjoint"] = None
    check_all(dk, f, TOL_F32, chunk=chunk, ref_gate=True)


def test_gate_fixture_bf16(dk):
    f = fx.gate_fixture(35, 0)
    for n in ("q", "k", "v"):
        f[n] = torch.tensor(f[n]).to(torch.bfloat16).float().numpy()
    check_all(dk, f, TOL_BF16, dtype=torch.bfloat16)


def test_continuation_inside_chunk(dk):
    """Split at position 3 and resume from the returned final state
    (kron_checks.rs:403-504)."""
    f = fx.gate_fixture(35, 0)
    out, fin, sc = oracle.scan(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                               f.initial)
    cut = 3
    a = {n: f[n][:, :cut] for n in GROUPS}
    b = {n: f[n][:, cut:] for n in GROUPS}
    import delta_kernels as dkk
    t = lambda x: dev(x)  # noqa: E731
    ra = dkk.gdn_training_scan(*(t(a[n]) for n in GROUPS), t(f.valid[:, :cut]),
                               t(f.reset[:, :cut]), t(f.initial), 16)
    rb = dkk.gdn_training_scan(*(t(b[n]) for n in GROUPS), t(f.valid[:, cut:]),
                               t(f.reset[:, cut:]), ra.final_state, 16)
    gate("continued output", torch.cat([ra.output, rb.output], 1), out, TOL_F32, ref_gate=True)
    gate("continued state", rb.final_state, fin, TOL_F32, ref_gate=True)
    gate("continued scores", torch.cat([ra.scores, rb.scores], 1)[..., 0], sc, TOL_F32,
         ref_gate=True)


def test_dre_tokens_long(dk):
    """reuse/crates/dre-gdn2 SplitMix tokens (K32/V64) over T=300 with no masks."""
    tok = fx.dre_tokens(300)
    rng = np.random.default_rng(0)
    f = fx.Fixture(**tok, valid=np.ones((1, 300), np.uint8), reset=np.zeros((1, 300), np.uint8),
                   initial=None, upstream=rng.normal(size=(1, 300, 1, 64)).astype(np.float32),
                   final_adjoint=rng.normal(size=(1, 1, 32, 64)).astype(np.float32) * 0.1,
                   score_adjoint=rng.normal(size=(1, 300, 1)).astype(np.float32) * 0.1)
    check_all(dk, f, TOL_F32)


@pytest.mark.parametrize("K,V", [(3, 4), (32, 32), (64, 64), (48, 80), (128, 128), (128, 32)])
def test_widths(dk, K, V):
    rng = np.random.default_rng(K * 1000 + V)
    B, T, H = 2, 40, 2
    k = rng.normal(size=(B, T, H, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    f = fx.Fixture(
        q=(rng.normal(size=(B, T, H, K)) * 0.3).astype(np.float32), k=k.astype(np.float32),
        v=rng.normal(size=(B, T, H, V)).astype(np.float32),
        alpha=rng.uniform(0.8, 1.0, size=(B, T, H, K)).astype(np.float32),
        erase=rng.uniform(0.2, 0.9, size=(B, T, H, K)).astype(np.float32),
        write=rng.uniform(0.2, 0.9, size=(B, T, H, V)).astype(np.float32),
        valid=np.ones((B, T), np.uint8), reset=np.zeros((B, T), np.uint8),
        initial=(rng.normal(size=(B, H, K, V)) * 0.1).astype(np.float32),
        upstream=rng.normal(size=(B, T, H, V)).astype(np.float32),
        final_adjoint=(rng.normal(size=(B, H, K, V)) * 0.1).astype(np.float32),
        score_adjoint=(rng.normal(size=(B, T, H)) * 0.1).astype(np.float32))
    f.valid[1, 30:] = 0
    f.reset[0, 17] = 1
    check_all(dk, f, TOL_F32)


def test_mixer_scan_selected_routes_to_hip(dk):
    from delta_mixers import MixerKind, ScanBackend, ScanInput, scan_selected
    f = fx.gate_fixture(7, 0)
    x = ScanInput(*(dev(f[n]) for n in GROUPS))
    r = scan_selected(ScanBackend.FUSED_GDN2, MixerKind.GDN2, x, dev(f.valid), dev(f.reset), 16,
                      dev(f.initial))
    out, fin, sc = oracle.scan(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                               f.initial)
    gate("scan_selected output", r.output, out, TOL_F32)
    with pytest.raises(NotImplementedError):
        scan_selected(ScanBackend.TENSOR_SOLVER, MixerKind.GDN2, x, dev(f.valid), dev(f.reset),
                      16)
    with pytest.raises(ValueError):
        scan_selected(ScanBackend.FUSED_GDN2, MixerKind.KRON_LSTM, x, dev(f.valid),
                      dev(f.reset), 16)
