"""GPU parity of the mixer prologue/epilogue operators (include/gdn2.h) on the
reference's own check fixtures, against the f64 oracle (oracle/mixer_oracle.py),
with the reference's f32 gate 2e-5 + 3e-4|ref|
(crates/mixers/src/convolution_checks.rs:34-40, normalization_checks.rs:10-22).
Inputs keep the fixtures' strided storage; every gradient is checked.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mixer_fixtures as mf  # noqa: E402
from gpu_util import REF_ATOL, REF_RTOL, host  # noqa: E402
from oracle import mixer_oracle as mo  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def up(a, grad=False):
    """Upload keeping the physical layout: the strides of a transposed numpy view."""
    a = np.asarray(a, np.float32)
    base = np.ascontiguousarray(a.transpose(np.argsort(a.strides)[::-1]))
    order = np.argsort(a.strides)[::-1]
    t = torch.from_numpy(base).cuda().permute(*np.argsort(order).tolist())
    assert tuple(t.shape) == a.shape
    return t.requires_grad_(grad) if grad else t


def ref_gate(name, got, ref):
    got = host(got) if torch.is_tensor(got) else np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64).reshape(got.shape)
    err = np.abs(got - ref)
    bad = ~np.isfinite(got) | (err > REF_ATOL + REF_RTOL * np.abs(ref))
    assert not bad.any(), (f"{name}: {bad.sum()} outside 2e-5 + 3e-4|ref|, worst "
                           f"{err.max():.3e}")


@pytest.mark.parametrize("t,c,width", mf.CONV_CASES)
@pytest.mark.parametrize("zero", [False, True])
@pytest.mark.parametrize("strided", [False, True])
@pytest.mark.parametrize("act", [None, "silu"])
def test_causal_conv_matches_oracle(dk, t, c, width, zero, strided, act):
    x, w, valid, docs, u = mf.conv_fixture(t, c, width, zero, strided)
    xg, wg = up(x, True), up(w, True)
    y = dk.causal_conv(xg, wg, up(valid), up(docs), activation=act)
    silu = act == "silu"
    ref_gate("conv output", y, mo.causal_conv(x, w, valid, docs, silu))
    (y * up(u)).sum().backward()
    dx, dw = mo.causal_conv_vjp(x, w, valid, docs, u, silu)
    ref_gate("conv dx", xg.grad, dx)
    ref_gate("conv dw", wg.grad, dw)


@pytest.mark.parametrize("width", mf.NORM_WIDTHS)
@pytest.mark.parametrize("zero", [False, True])
@pytest.mark.parametrize("mode,eps", mf.NORM_MODES)
def test_norms_match_oracle(dk, width, zero, mode, eps):
    x, gate, u, weight, mask = mf.norm_fixture(width, zero)
    if zero:
        x = np.zeros_like(x)
    m4 = mask[:, :, None, None]
    xg, gg, wg = up(x, True), up(gate, True), up(weight, True)
    if mode == 0:
        if eps != 1e-6:
            pytest.skip("l2_norm has the reference's fixed epsilon")
        y = dk.l2_norm(xg)
    elif mode == 1:
        y = dk.rms_norm(xg, wg, None, eps)
    else:
        y = dk.rms_norm(xg, wg, gg, eps)
    yr, _ = mo.row_norm(x, weight, gate, mode, eps)
    ref_gate("norm output", y * up(m4), yr * m4)
    (y * up(m4) * up(u)).sum().backward()
    dx, dg, dw = mo.row_norm_vjp(x, weight, gate, mode, eps, u * m4)
    ref_gate("norm dx", xg.grad, dx)
    if mode >= 1:
        ref_gate("norm dweight", wg.grad, dw)
    if mode == 2:
        ref_gate("norm dgate", gg.grad, dg)


def test_rms_norm_accepts_lower_rank_inputs(dk):
    rng = np.random.default_rng(0)
    x = rng.normal(size=(5, 512)).astype(np.float32)
    w = rng.normal(size=512).astype(np.float32)
    y = dk.rms_norm(up(x), up(w), None, 1e-6)
    ref_gate("rms 2-D", y, mo.row_norm(x, w, None, 1, 1e-6)[0])


@pytest.mark.parametrize("zero", [False, True])
def test_decay_matches_oracle(dk, zero):
    x, bias, scale, u, mask = mf.decay_fixture(zero)
    m4 = mask[:, :, None, None]
    xg, bg, sg = up(x, True), up(bias, True), up(scale, True)
    y = dk.decay(xg, bg, sg)
    ref_gate("decay output", y * up(m4), mo.decay(x, bias, scale) * m4)
    (y * up(m4) * up(u)).sum().backward()
    dx, db, ds = mo.decay_vjp(x, bias, scale, u * m4)
    ref_gate("decay dx", xg.grad, dx)
    ref_gate("decay dbias", bg.grad, db)
    ref_gate("decay dscale", sg.grad, ds)


def test_operators_reject_cpu_and_wrong_dtype(dk):
    x = torch.zeros(1, 2, 1, 4)
    with pytest.raises(ValueError):
        dk.l2_norm(x)
    with pytest.raises(TypeError):
        dk.l2_norm(x.cuda().double())


def _docs_valid(rng, B, T):
    valid = np.ones((B, T), np.float32)
    valid[0, T // 3] = 0
    valid[-1, T - 2:] = 0
    reset = np.zeros((B, T), np.float32)
    reset[:, 0] = 1
    reset[0, T // 2] = 1
    reset[-1, 33] = 1  # inside the second 32-step segment
    return valid, np.cumsum(valid * reset, axis=1).astype(np.float32)


@pytest.mark.parametrize("taps", [3, 4, 8])
@pytest.mark.parametrize("act", [None, "silu"])
def test_causal_conv_long_sequences(dk, taps, act):
    """Several 32-step time segments per sequence, documents crossing them."""
    rng = np.random.default_rng(taps)
    B, T, C = 2, 130, 96  # channel count not a multiple of 64
    x = rng.normal(size=(B, T, C)).astype(np.float32)
    w = (rng.normal(size=(taps, C)) * 0.5).astype(np.float32)
    u = rng.normal(size=(B, T, C)).astype(np.float32)
    valid, docs = _docs_valid(rng, B, T)
    xg, wg = up(x, True), up(w, True)
    y = dk.causal_conv(xg, wg, up(valid), up(docs), activation=act)
    silu = act == "silu"
    ref_gate("conv output", y, mo.causal_conv(x, w, valid, docs, silu))
    (y * up(u)).sum().backward()
    dx, dw = mo.causal_conv_vjp(x, w, valid, docs, u, silu)
    ref_gate("conv dx", xg.grad, dx)
    ref_gate("conv dw", wg.grad, dw)


@pytest.mark.parametrize("width", [64, 128, 192, 256, 512, 768, 1024])
@pytest.mark.parametrize("mode,eps", mf.NORM_MODES)
@pytest.mark.parametrize("rows", [(3, 37, 5), (2, 1100, 2)])
def test_norms_contiguous_rows(dk, width, mode, eps, rows):
    """Contiguous rows (the 16-byte-access kernels): partial workgroups, and more
    rows than the backward grid holds (each group loops)."""
    if mode == 0 and eps != 1e-6:
        pytest.skip("l2_norm has the reference's fixed epsilon")
    rng = np.random.default_rng(width + mode)
    B, T, H = rows
    x = rng.normal(size=(B, T, H, width)).astype(np.float32)
    gate = (rng.normal(size=x.shape) * 2).astype(np.float32)
    weight = rng.normal(size=width).astype(np.float32)
    u = rng.normal(size=x.shape).astype(np.float32)
    xg, gg, wg = up(x, True), up(gate, True), up(weight, True)
    if mode == 0:
        y = dk.l2_norm(xg)
    elif mode == 1:
        y = dk.rms_norm(xg, wg, None, eps)
    else:
        y = dk.rms_norm(xg, wg, gg, eps)
    ref_gate("norm output", y, mo.row_norm(x, weight, gate, mode, eps)[0])
    (y * up(u)).sum().backward()
    dx, dg, dw = mo.row_norm_vjp(x, weight, gate, mode, eps, u)
    ref_gate("norm dx", xg.grad, dx)
    if mode >= 1:
        ref_gate("norm dweight", wg.grad, dw)
    if mode == 2:
        ref_gate("norm dgate", gg.grad, dg)
