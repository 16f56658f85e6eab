"""The f32 chunk kernels (csrc/gdn2_chunk_f32.hip): channel-wise GDN-2 with f32
q/k/v and d_k, d_v <= 128, in 16-token chunks, against the f64 oracle.

1. The reference's isolated-scan benchmark workload (kron_benchmark.rs:73-116:
   B8 T512 H4 K32 V64, alpha in [0.90, 0.99], erase/write in [0.1, 0.9], unit
   rows, all-ones upstream gradient) with the stage timers on: the six chunk
   stages run, and every output and gradient passes the 1e-4 gate and the
   reference's own gate 2e-5 + 3e-4|ref| (kron_checks.rs:34-35).
2. The reference's GDN gate fixture (kron_checks.rs:89-524) at T = 35, all
   four objectives, through the chunk kernels (stage timers), at both gates.
   The fixture zeroes alpha on one channel at p = 2 and on every channel at
   p = 16, so the exact alpha gradient at alpha = 0 is gated too.
3. Gates the chunk kernels handle with no special case, because they form every
   decay as a product of the gates: negative alpha, alpha = 0 on a whole
   chunk, tiny alpha; and ragged widths (d_k, d_v in 1..128: the kernels built
   for 64-wide tiles up to 64, for 128-wide tiles above, where bgrad walks the
   value axis in two blocks) with padding and resets inside chunks and sequence
   ends off the chunk grid.
4. Slow decay over 256 chunks (T = 4096) at K32/V64, and over 128 chunks
   (T = 2048) at K = V = 128, at both gates.
5. bf16 q/k/v at widths the bf16 chunk kernels do not take (d_k != d_v, below
   64 or above): the same kernels read the exact f32 values of the bf16 inputs and
   write bf16 gradients; gated at the bf16 tolerance against the oracle run on
   the bf16-rounded inputs.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import fixtures as fx  # noqa: E402
from gpu_util import TOL_BF16, TOL_F32, dev, gate  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu

GROUPS = ("q", "k", "v", "alpha", "erase", "write")
STAGES = {"chunk_prep", "state_scan", "chunk_out", "chunk_bprep", "adjoint_scan", "chunk_bgrad"}


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def run_and_check(dk, f, ref_gate=True, chunk=16, dtype=torch.float32, tol=TOL_F32):
    """Forward + backward through gdn_training_scan with the stage timers on,
    every output and gradient gated against the f64 oracle; returns the stages
    that ran.  dtype is that of q, k and v (and so of dO and dq, dk, dv)."""
    xs = {n: dev(f[n], dtype if n in ("q", "k", "v") else torch.float32).requires_grad_(True)
          for n in GROUPS}
    init = dev(f.initial).requires_grad_(True) if f.initial is not None else None
    dk.stage_timing(True)
    try:
        r = dk.gdn_training_scan(xs["q"], xs["k"], xs["v"], xs["alpha"], xs["erase"],
                                 xs["write"], dev(f.valid), dev(f.reset), init, chunk)
        loss = (r.output.float() * dev(f.upstream)).sum()
        if f.final_adjoint is not None:
            loss = loss + (r.final_state * dev(f.final_adjoint)).sum()
        if f.score_adjoint is not None:
            loss = loss + (r.scores[..., 0] * dev(f.score_adjoint)).sum()
        loss.backward()
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    out, fin, sc = oracle.scan(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset,
                               f.initial)
    g = oracle.backward(f.q, f.k, f.v, f.alpha, f.erase, f.write, f.valid, f.reset, f.initial,
                        f.upstream, f.final_adjoint, f.score_adjoint)
    pad = (f.valid == 0)[:, :, None, None]
    gate("output", r.output, out, tol, exact_zero=pad, ref_gate=ref_gate)
    gate("final_state", r.final_state, fin, tol, ref_gate=ref_gate)
    gate("scores", r.scores[..., 0], sc, tol, exact_zero=pad[..., 0], ref_gate=ref_gate)
    for n in GROUPS:
        gate(f"d{n}", xs[n].grad, g[n], tol, exact_zero=pad, ref_gate=ref_gate)
    if init is not None:
        gate("d_initial", init.grad, g["initial"], tol, ref_gate=ref_gate)
    return ran, g


def test_reference_benchmark_workload(dk):
    f = fx.kron_raw(8, 512)
    print("f32 chunk: kron_raw B8 T512 H4 K32 V64", flush=True)
    ran, _ = run_and_check(dk, f)
    assert STAGES <= ran, sorted(ran)


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_gate_fixture_runs_chunk_kernels(dk, mode):
    f = fx.gate_fixture(35, mode)
    assert (f.alpha[:, 2, :, 0] == 0).all() and (f.alpha[:, 16] == 0).all()
    ran, g = run_and_check(dk, f)
    assert STAGES <= ran, sorted(ran)
    if mode != 2:  # the final state does not depend on p = 16 (resets at 19, padding from 16)
        assert np.abs(g["alpha"][:, 16]).max() > 0  # the gradient at alpha = 0 is not zero


def _random(seed, B, T, H, K, V, alpha=(0.8, 1.0), masks=True):
    rng = np.random.default_rng(seed)
    k = rng.normal(size=(B, T, H, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    valid = np.ones((B, T), np.uint8)
    reset = np.zeros((B, T), np.uint8)
    if masks:
        valid[0, 5:9] = 0
        valid[-1, T - 3:] = 0
        reset[0, [p for p in (0, 13, 40) if p < T]] = 1
        reset[-1, [p for p in (2, 17, 18) if p < T]] = 1
        if T > 18:
            valid[-1, 18] = 0  # a reset on a padding token does nothing
    return fx.Fixture(
        q=(rng.normal(size=(B, T, H, K)) * 0.3).astype(np.float32), k=k.astype(np.float32),
        v=rng.normal(size=(B, T, H, V)).astype(np.float32),
        alpha=rng.uniform(*alpha, size=(B, T, H, K)).astype(np.float32),
        erase=rng.uniform(0.2, 0.9, size=(B, T, H, K)).astype(np.float32),
        write=rng.uniform(0.2, 0.9, size=(B, T, H, V)).astype(np.float32),
        valid=valid, reset=reset,
        initial=(rng.normal(size=(B, H, K, V)) * 0.1).astype(np.float32),
        upstream=rng.normal(size=(B, T, H, V)).astype(np.float32),
        final_adjoint=(rng.normal(size=(B, H, K, V)) * 0.1).astype(np.float32),
        score_adjoint=(rng.normal(size=(B, T, H)) * 0.1).astype(np.float32))


@pytest.mark.parametrize("K,V,T", [(1, 1, 19), (3, 4, 33), (17, 64, 50), (64, 33, 64),
                                   (64, 64, 77), (32, 64, 130), (128, 128, 70), (96, 128, 50),
                                   (128, 33, 40), (65, 64, 33), (1, 128, 20), (128, 80, 47)])
def test_ragged_widths(dk, K, V, T):
    f = _random(K * 100 + V, 2, T, 3, K, V)
    print(f"f32 chunk: widths K{K} V{V} T{T}", flush=True)
    ran, _ = run_and_check(dk, f, ref_gate=False)
    assert STAGES <= ran, sorted(ran)


def test_negative_alpha(dk):
    """alpha in [-1, 1]: the decays are signed products; the f32 chunk kernels
    take them exactly (the bf16 chunk kernels refuse them with NaN)."""
    f = _random(5, 2, 70, 2, 32, 64, alpha=(-1.0, 1.0))
    ran, _ = run_and_check(dk, f, ref_gate=False)
    assert STAGES <= ran


def test_zero_and_tiny_alpha(dk):
    """alpha = 0 over a whole chunk of one head, one channel at 1e-30 over
    another chunk, 1e-3..1e-2 elsewhere in that sequence."""
    f = _random(6, 2, 64, 2, 32, 64)
    f.alpha[0, 16:32, 0] = 0.0
    f.alpha[0, 32:48, 1, 3] = 1e-30
    f.alpha[1, :, 0] = np.random.default_rng(1).uniform(1e-3, 1e-2, size=(64, 32))
    _, g = run_and_check(dk, f, ref_gate=False)
    assert np.abs(g["alpha"][0, 16:32, 0]).max() > 0


@pytest.mark.parametrize("alpha", [(0.9, 0.99), (0.999, 1.0)])
def test_slow_decay_long(dk, alpha):
    """256 chunks of 16 tokens with slow decay (the reference benchmark's law
    and alpha >= 0.999): the state and its adjoint carry across the whole
    sequence, so errors of the f32 scans compound; every output and gradient
    stays within the 1e-4 gate, and within the reference's own gate
    2e-5 + 3e-4|ref| for alpha in [0.90, 0.99].  With alpha >= 0.999 the
    gradients grow to rms 10-12 (dalpha, dk; max 70), where that gate's absolute
    term, 2e-6 of the rms, lies at the rounding of f32 sums carried over 4096
    tokens: whether it passes depends on the order of the scan's key sums."""
    f = _random(7, 2, 4096, 2, 32, 64, alpha=alpha)
    print(f"f32 chunk: slow decay alpha {alpha} T4096", flush=True)
    ran, _ = run_and_check(dk, f, ref_gate=alpha[0] < 0.999)
    assert STAGES <= ran, sorted(ran)


@pytest.mark.parametrize("alpha", [(0.9, 0.99), (0.999, 1.0)])
def test_slow_decay_wide(dk, alpha):
    """128 chunks at K = V = 128 with slow decay: the 128-wide kernels and the
    eight-tile scans.  Both draws pass the 1e-4 gate; the reference's gate
    2e-5 + 3e-4|ref| is applied to alpha in [0.90, 0.99].  With alpha >= 0.999
    the gradients grow to rms 30 (dk; max 159) and its absolute term, 7e-7 of
    that rms, lies under the rounding of 128-term f32 sums carried over 2048
    tokens, which the 1e-4 gate (relative to |ref| + rms) allows for."""
    f = _random(8, 2, 2048, 1, 128, 128, alpha=alpha)
    print(f"f32 chunk: slow decay alpha {alpha} T2048 K128 V128", flush=True)
    ran, _ = run_and_check(dk, f, ref_gate=alpha[0] < 0.999)
    assert STAGES <= ran, sorted(ran)


def _bf16_round(f):
    """q, k, v and the output adjoint as the bf16 values the kernels receive (dO
    has q's dtype), so the oracle and the kernels see the same inputs."""
    for n in ("q", "k", "v", "upstream"):
        f[n] = torch.tensor(f[n]).to(torch.bfloat16).float().numpy()
    return f


@pytest.mark.parametrize("K,V,T", [(32, 64, 512), (17, 64, 50), (64, 33, 77), (16, 16, 40),
                                   (128, 128, 100), (80, 128, 50)])
def test_bf16_inputs(dk, K, V, T):
    f = _bf16_round(_random(K * 7 + V, 2, T, 3, K, V))
    print(f"f32 chunk: bf16 inputs K{K} V{V} T{T}", flush=True)
    ran, _ = run_and_check(dk, f, ref_gate=False, dtype=torch.bfloat16, tol=TOL_BF16)
    assert STAGES <= ran, sorted(ran)


def test_bf16_gate_fixture(dk):
    """The reference's gate fixture (K32, V64) with bf16 q/k/v."""
    f = _bf16_round(fx.gate_fixture(35, 0))
    ran, _ = run_and_check(dk, f, ref_gate=False, dtype=torch.bfloat16, tol=TOL_BF16)
    assert STAGES <= ran, sorted(ran)
