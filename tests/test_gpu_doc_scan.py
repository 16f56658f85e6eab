"""The document-limit GDN-2 scan (gdn2_scan / gdn2_backward) through the C ABI.

1. The reference's own GPU check of this op (crates/mixers/src/checks.rs:852-1010,
   custom_gdn_check), restated: its procedural fixture (checks.rs:119-180, B2
   H4 K32 V64, T 7 and 35, padding and resets), document limits derived from
   the fixture's masks exactly as the check does, and K probe tokens (identity
   queries, unit decay, zero updates) appended so that the outputs read back
   the final state.  Outputs, final state and all six gradients (with the
   check's final-state adjoint) against the f64 oracle at the check's own gate
   2e-5 + 3e-4|ref| (checks.rs:73-74).
2. Packed documents at the lm512 head shape (K = V = 64) and K = V = 128, f32
   (1e-4 rms-floored) and bf16 (2e-2) against the f64 doc-limit oracle.
3. Inconsistent limits (a reset whose previous token does not end its
   document): the backward is the exact VJP of the forward, as the reference's
   GPU kernels compute it (crates/kernels/src/gdn2.rs:24-65, :288-490); the
   reference's f64 oracle lets the adjoint cross that reset instead.
4. bf16 with K = V = 64 runs the 16-token chunk-WY MFMA kernels (stage
   timers); every other width and dtype the f32 chunk kernels (items 1 and 2,
   and bf16 at 32 x 64 and 128 x 128 with the stage timers).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from gpu_util import REF_ATOL, REF_RTOL, TOL_BF16, TOL_F32, gate  # noqa: E402
from oracle import doc_oracle as do  # noqa: E402
from oracle import oracle  # noqa: E402

pytestmark = pytest.mark.gpu
F32 = np.float32
FIELDS = ("q", "k", "v", "alpha", "erase", "write")


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def check_fixture(t):
    """checks.rs:119-180 for MixerKind::Gdn2: fields [b, t, h, width] f32,
    valid/reset [b, t] bool, upstream [b, t, h, v], final adjoint [b, h, k, v]."""
    b, h, k, v = 2, 4, 32, 64
    widths = (k, k, v, k, k, v)
    data = []
    for field, w in enumerate(widths):
        i = np.arange(b * t * h * w)
        signal = np.sin((i * 13 + field * 19 + 1) * 0.037).astype(F32)
        if field == 3:
            x = F32(0.91) + F32(0.03) * signal
        elif field >= 4:
            x = F32(0.45) + F32(0.1) * signal
        else:
            x = F32(0.1) * signal
        data.append(x.astype(F32).reshape(b, t, h, w))
    r = np.arange(b * t) // t
    p = np.arange(b * t) % t
    valid = ((p < np.maximum(t - (r + 1), 0)) & (p != 9) & (p != 11)).reshape(b, t)
    reset = ((p == 0) | (p == 5) | (p == 19)).reshape(b, t)
    up = np.cos((np.arange(b * t * h * v) * 7 + 3) * 0.051).astype(F32).reshape(b, t, h, v)
    fa = (F32(0.03) * np.sin((np.arange(b * h * k * v) * 3 + 1) * 0.04).astype(F32))
    return data, valid, reset, up, fa.astype(F32).reshape(b, h, k, v)


def check_limits(valid, reset, extended):
    """Document limits as custom_gdn_check derives them (checks.rs:862-886)."""
    b, t = valid.shape
    starts = np.ones((b, extended), np.int32)
    ends = np.zeros((b, extended), np.int32)
    for row in range(b):
        start = 0
        for p in range(t):
            if not valid[row, p]:
                continue
            if reset[row, p]:
                start = p
            starts[row, p] = start
            nxt = next((n for n in range(p + 1, t) if valid[row, n] and reset[row, n]), None)
            if nxt is None:
                ends[row, p] = extended - 1
            else:
                ends[row, p] = max(n for n in range(p, nxt) if valid[row, n])
        starts[row, t:] = start
        ends[row, t:] = extended - 1
    return starts, ends


def dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda().to(dtype)


def ref_gate(name, got, ref):
    got = got.detach().double().cpu().numpy() if torch.is_tensor(got) else got
    err = np.abs(got - ref)
    bad = ~np.isfinite(got) | (err > REF_ATOL + REF_RTOL * np.abs(ref))
    assert not bad.any(), f"{name}: {bad.sum()} outside 2e-5 + 3e-4|ref|, worst {err.max():.3e}"


@pytest.mark.parametrize("t", [7, 35])
@pytest.mark.parametrize("probes", [False, True])
def test_reference_custom_gdn_check(dk, t, probes):
    data, valid, reset, up, fa = check_fixture(t)
    b, _, h, k = data[0].shape
    v = data[2].shape[3]
    extended = t + (k if probes else 0)
    starts, ends = check_limits(valid, reset, extended)
    padded = []
    for f, x in enumerate(data):
        if probes:
            w = x.shape[3]
            probe = np.zeros((b, k, h, w), F32)
            if f == 0:
                for p in range(k):
                    probe[:, p, :, p] = 1.0
            elif f == 3:
                probe[:] = 1.0
            x = np.concatenate([x, probe], axis=1)
        padded.append(dev(x).requires_grad_(True))
    out = dk.gdn2_scan(*padded, dev(starts, torch.int32), dev(ends, torch.int32))
    ref_out, ref_fin, _ = oracle.scan(*data, valid, reset)
    ref_gate("output", out[:, :t], ref_out)
    d_out = np.zeros((b, extended, h, v), F32)
    d_out[:, :t] = up
    if probes:
        ref_gate("final state", out[:, t:].transpose(1, 2), ref_fin)
        d_out[:, t:] = fa.transpose(0, 2, 1, 3)
    out.backward(dev(d_out))
    ref = oracle.backward(*data, valid, reset, upstream=up, final_adjoint=fa if probes else None)
    for name, x in zip(FIELDS, padded):
        ref_gate(f"d{name}", x.grad[:, :t], ref[name])


def _packed_problem(B, T, H, K, V, seed):
    rng = np.random.default_rng(seed)
    q = rng.normal(size=(B, T, H, K)).astype(F32)
    k = rng.normal(size=(B, T, H, K)).astype(F32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(size=(B, T, H, V)).astype(F32)
    alpha = rng.uniform(0.8, 1.0, size=(B, T, H, K)).astype(F32)
    erase = rng.uniform(0.1, 0.9, size=(B, T, H, K)).astype(F32)
    write = rng.uniform(0.1, 0.9, size=(B, T, H, V)).astype(F32)
    up = rng.normal(size=(B, T, H, V)).astype(F32)
    start = np.ones((B, T), np.int32)
    end = np.zeros((B, T), np.int32)
    # row 0: documents crossing the 16-token staging blocks, padding between
    for s, e in ((0, 9), (10, 40), (45, 70), (71, 71), (80, T - 1)):
        start[0, s:e + 1], end[0, s:e + 1] = s, e
    if B > 1:
        start[1, 3:], end[1, 3:] = 3, T - 1  # one document after leading padding
    return [q, k, v, alpha, erase, write], start, end, up


@pytest.mark.parametrize("kv", [(64, 64), (128, 128), (32, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_packed_documents_match_doc_oracle(dk, kv, dtype):
    K, V = kv
    x, start, end, up = _packed_problem(2, 100, 3, K, V, K + V)
    xs = [dev(a, dtype if i < 3 else torch.float32).requires_grad_(True) for i, a in enumerate(x)]
    xr = [a.detach().double().cpu().numpy() for a in xs]  # inputs as stored
    out = dk.gdn2_scan(*xs, dev(start, torch.int32), dev(end, torch.int32))
    assert out.dtype == dtype
    out.backward(dev(up, dtype))
    upr = dev(up, dtype).double().cpu().numpy()
    ref_out, _ = do.doc_scan(*xr, start, end)
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    pad = np.broadcast_to((end < start)[:, :, None, None], ref_out.shape)
    gate("output", out, ref_out, tol, exact_zero=pad)
    ref = do.doc_backward(*xr, start, end, upr)
    for name, t in zip(FIELDS, xs):
        padg = np.broadcast_to((end < start)[:, :, None, None], t.shape)
        gate(f"d{name}", t.grad, ref[name], tol, exact_zero=padg)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_inconsistent_limits_follow_reference_kernels(dk, dtype):
    x, _, _, up = _packed_problem(1, 40, 2, 64, 64, 3)
    start = np.zeros((1, 40), np.int32)
    end = np.full((1, 40), 39, np.int32)
    start[0, 20:] = 20  # a reset at 20 without a document end at 19
    start[0, 33:], end[0, 25:33] = 33, 29  # an end at 29 without a reset at 30
    xs = [dev(a, dtype if i < 3 else torch.float32).requires_grad_(True) for i, a in enumerate(x)]
    xr = [a.detach().double().cpu().numpy() for a in xs]
    out = dk.gdn2_scan(*xs, dev(start, torch.int32), dev(end, torch.int32))
    out.backward(dev(up, dtype))
    upr = dev(up, dtype).double().cpu().numpy()
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    ref_out, _ = do.doc_scan(*xr, start, end)
    gate("output", out, ref_out, tol)
    valid, reset = oracle.doc_limits_to_masks(start, end)
    exact = oracle.backward(*xr, valid, reset, upstream=upr)
    for name, t in zip(FIELDS, xs):
        gate(f"d{name}", t.grad, exact[name], tol)
    # the f64 oracle's rule differs here: its adjoint crosses the reset at 20
    cpu_rule = do.doc_backward(*xr, start, end, upr)
    assert np.abs(cpu_rule["k"][0, :20] - exact["k"][0, :20]).max() > 1e-2


@pytest.mark.parametrize("kv", [(64, 64), (32, 64), (128, 128)])
def test_bf16_runs_chunk_kernels(dk, kv):
    """bf16 at 64 x 64 runs the bf16 chunk kernels, at 32 x 64 and 128 x 128
    the f32 chunk kernels; each reports the six chunk stages."""
    x, start, end, up = _packed_problem(2, 100, 3, kv[0], kv[1], 9)
    xs = [dev(a, torch.bfloat16 if i < 3 else torch.float32).requires_grad_(True)
          for i, a in enumerate(x)]
    dk.stage_timing(True)
    try:
        out = dk.gdn2_scan(*xs, dev(start, torch.int32), dev(end, torch.int32))
        out.backward(dev(up, torch.bfloat16))
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    assert {"chunk_prep", "state_scan", "chunk_out", "chunk_bprep", "adjoint_scan",
            "chunk_bgrad"} <= ran, sorted(ran)


def test_rejects_bad_limits(dk):
    x, start, end, _ = _packed_problem(2, 100, 3, 64, 64, 1)
    xs = [dev(a) for a in x]
    with pytest.raises(ValueError):
        dk.gdn2_scan(*xs, dev(start, torch.int64), dev(end, torch.int32))
    with pytest.raises(ValueError):
        dk.gdn2_scan(*xs, dev(start[:, :50], torch.int32), dev(end[:, :50], torch.int32))
