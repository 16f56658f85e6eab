"""Training-step operators (cross entropy, AdamW) through the C ABI against the
oracle (oracle/train_oracle.py).

Cross entropy (reference crates/kernels/src/cross_entropy.rs): loss and stats
within 1e-5 relative of the f64 oracle for f32 logits; gradients within
1e-5 rms-floored for f32, and within bf16 rounding (2^-8 relative, rms-floored)
for bf16 logits, whose gradient is stored in bf16.  Widths cover the scalar
path (3, 1000: not a multiple of the vector width), the vector path (64,
32768) and strided logits.

AdamW (reference crates/kernels/src/update.rs): bit-exact against the f32
oracle whenever clipping is inactive (the reference's element update rounds
each operation; the kernel does the same), and within 2e-6 relative when the
clipping coefficient (a sum of squares in another order) is active; sizes cover
partial vectors and partial chunks, misaligned tensors and several tensors per
call.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from gpu_util import gate  # noqa: E402
from oracle import train_oracle as to  # noqa: E402

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _problem(rows, width, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    x = (rng.normal(size=(rows, width)) * scale).astype(np.float32)
    t = rng.integers(0, width, size=rows)
    up = rng.normal(size=rows).astype(np.float32)
    return x, t, up


@pytest.mark.parametrize("width", [3, 64, 1000, 32768])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cross_entropy_rows_forward_backward(width, dtype):
    _need_gpu()
    import delta_kernels as dk
    x, t, up = _problem(37, width, width)
    xd = torch.from_numpy(x).cuda().to(dtype).requires_grad_(True)
    xr = xd.detach().double().cpu().numpy()  # the logits as stored
    td = torch.from_numpy(t).cuda()
    loss = dk.cross_entropy_rows(xd, td)
    loss.backward(torch.from_numpy(up).cuda())
    ref_loss, _ = to.cross_entropy_rows(xr, t)
    gate("loss", loss, ref_loss, 1e-5)
    tol = 1e-5 if dtype == torch.float32 else 2.0 ** -8
    assert xd.grad.dtype == dtype
    gate("dx", xd.grad, to.cross_entropy_rows_vjp(xr, t, up), tol)


def test_cross_entropy_strided_logits_and_bad_label():
    _need_gpu()
    import delta_kernels as dk
    x, t, up = _problem(9, 40, 7)
    base = torch.from_numpy(np.ascontiguousarray(x.T)).cuda()  # stored [width, rows]
    xd = base.t().requires_grad_(True)  # [rows, width] view, column stride = rows
    assert not xd.is_contiguous()
    t_bad = t.copy()
    t_bad[4] = 40  # outside [0, width)
    loss = dk.cross_entropy_rows(xd, torch.from_numpy(t_bad).cuda())
    ref_loss, _ = to.cross_entropy_rows(x, t)
    got = loss.detach().cpu().numpy()
    assert np.isnan(got[4])
    keep = np.arange(9) != 4
    gate("loss", got[keep], ref_loss[keep], 1e-5)
    loss = dk.cross_entropy_rows(xd, torch.from_numpy(t).cuda())
    loss.backward(torch.from_numpy(up).cuda())
    gate("dx", xd.grad, to.cross_entropy_rows_vjp(x, t, up), 1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_linear_cross_entropy_fused_head(dtype):
    _need_gpu()
    import delta_kernels as dk
    rng = np.random.default_rng(3)
    rows, d, width = 70, 48, 4096
    h = torch.from_numpy(rng.normal(size=(rows, d)).astype(np.float32)).cuda().to(dtype)
    w = torch.from_numpy(rng.normal(size=(width, d)).astype(np.float32) * 0.2).cuda().to(dtype)
    t = rng.integers(0, width, size=rows)
    h.requires_grad_(True)
    w.requires_grad_(True)
    loss = dk.linear_cross_entropy(h, w, torch.from_numpy(t).cuda())
    (loss * 3.0).backward()
    logits = (h.detach() @ w.detach().t()).double().cpu().numpy()  # as the GEMM stores them
    ref_loss, _ = to.cross_entropy_rows(logits, t)
    gate("loss", loss, np.array(ref_loss.mean()), 1e-5)
    dl = to.cross_entropy_rows_vjp(logits, t, np.full(rows, 3.0 / rows))
    hh = h.detach().double().cpu().numpy()
    ww = w.detach().double().cpu().numpy()
    tol = 1e-5 if dtype == torch.float32 else 2e-2  # bf16 dlogits, bf16 GEMM outputs
    gate("dh", h.grad, dl @ ww, tol)
    gate("dw", w.grad, dl.T @ hh, tol)


def _adam_case(numel, seed, grad_scale):
    rng = np.random.default_rng(seed)
    p = rng.normal(size=numel).astype(np.float32)
    gs = [(rng.normal(size=numel) * grad_scale).astype(np.float32) for _ in range(3)]
    return p, gs


@pytest.mark.parametrize("numel", [1, 7, 4096, 16384 * 3 + 5])
def test_adamw_update_bit_exact_without_clipping(numel):
    _need_gpu()
    import delta_kernels as dk
    p, gs = _adam_case(numel, numel, 1e-3 / np.sqrt(numel))  # norm << clip
    lr, wd, clip = 3e-3, 0.01, 1.0
    x = torch.from_numpy(p).cuda()
    m = v = None
    pr, mr, vr = p, None, None
    for t, g in enumerate(gs, start=1):
        x, m, v = dk.adamw_update(x, torch.from_numpy(g).cuda(), m, v, t, lr, wd, clip)
        pr, mr, vr = to.adamw_f32(pr, g, mr, vr, t, lr, wd, clip)
        np.testing.assert_array_equal(x.cpu().numpy(), pr)
        np.testing.assert_array_equal(m.cpu().numpy(), mr)
        np.testing.assert_array_equal(v.cpu().numpy(), vr)


def test_adamw_update_with_clipping_and_misaligned_tensor():
    _need_gpu()
    import delta_kernels as dk
    numel = 16384 + 9
    p, gs = _adam_case(numel, 11, 1.0)  # norm ~ 128 >> clip
    store = torch.zeros(numel + 1, device="cuda")
    x = store[1:]  # 4-byte offset: the scalar path
    x.copy_(torch.from_numpy(p))
    gbuf = torch.zeros(numel + 1, device="cuda")
    m = v = None
    pr, mr, vr = p, None, None
    for t, g in enumerate(gs, start=1):
        gbuf[1:].copy_(torch.from_numpy(g))
        x, m, v = dk.adamw_update(x, gbuf[1:], m, v, t, 1e-2, 0.1, 0.5)
        pr, mr, vr = to.adamw_f32(pr, g, mr, vr, t, 1e-2, 0.1, 0.5)
        gate("param", x, pr, 2e-6)
        gate("first", m, mr, 2e-6)
        gate("second", v, vr, 4e-6)


def test_fused_adamw_multi_tensor_matches_per_tensor_calls():
    _need_gpu()
    import delta_kernels as dk
    rng = np.random.default_rng(5)
    shapes = [(3,), (64, 33), (16384 * 2 + 1,), (5, 7), (1,)]
    ps = [torch.nn.Parameter(torch.from_numpy(rng.normal(size=s).astype(np.float32)).cuda())
          for s in shapes]
    refs = [p.detach().clone() for p in ps]
    opt = dk.FusedAdamW(ps, lr=2e-3, weight_decay=0.05, clip=0.7)
    states = [(None, None)] * len(ps)
    for t in range(1, 4):
        gs = [torch.from_numpy((rng.normal(size=s) * (0.01 if i % 2 else 3.0))
                               .astype(np.float32)).cuda() for i, s in enumerate(shapes)]
        for p, g in zip(ps, gs):
            p.grad = g.clone() if t != 2 else g  # step 2 keeps the same grad storage
        opt.step()
        for i, (r, g) in enumerate(zip(refs, gs)):
            m, v = states[i]
            _, m, v = dk.adamw_update(r, g, m, v, t, 2e-3, 0.05, 0.7)
            states[i] = (m, v)
        for p, r in zip(ps, refs):
            assert torch.equal(p.detach(), r), "multi-tensor and per-tensor updates differ"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_cross_entropy_in_place_reads_target_before_overwrite(dtype):
    """The in-place fused kernel must read x[r, target] before any thread of
    the row writes its gradient: every label here sits in columns that the
    row's last wave reads and rewrites."""
    _need_gpu()
    import ctypes
    import delta_kernels as dk
    from delta_kernels import _ptr, _stream, _view
    rows, width = 512, 32768
    rng = np.random.default_rng(9)
    x = (rng.normal(size=(rows, width)) * 2).astype(np.float32)
    vec = 4 if dtype == torch.float32 else 8
    cols = np.arange(width)
    last_wave = cols[(cols // vec) % 256 >= 192]
    t = rng.choice(last_wave, size=rows)
    xd = torch.from_numpy(x).cuda().to(dtype)
    xr = xd.double().cpu().numpy()
    td = torch.from_numpy(t).cuda()
    loss = torch.empty(rows, device="cuda")
    rc = dk.lib().gdn2_cross_entropy_fused(rows, width, ctypes.byref(_view(xd)), _ptr(td), 1,
                                           ctypes.c_float(1.0), _ptr(loss), _ptr(xd), _stream(xd))
    assert rc == 0
    ref_loss, _ = to.cross_entropy_rows(xr, t)
    gate("loss", loss, ref_loss, 1e-5)
    tol = 1e-5 if dtype == torch.float32 else 2.0 ** -8
    gate("dx", xd, to.cross_entropy_rows_vjp(xr, t, np.ones(rows)), tol)
