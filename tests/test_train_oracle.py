"""Pinning of the training-operator oracle (oracle/train_oracle.py), CPU only."""
import numpy as np
import pytest
from scipy.special import logsumexp

from oracle import train_oracle as to


def test_cross_entropy_matches_logsumexp_and_closed_forms():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(5, 37)) * 4
    t = rng.integers(0, 37, size=5)
    loss, st = to.cross_entropy_rows(x, t)
    np.testing.assert_allclose(loss, logsumexp(x, axis=1) - x[np.arange(5), t], rtol=1e-13)
    np.testing.assert_allclose(st[:, 0] + st[:, 1], logsumexp(x, axis=1), rtol=1e-13)
    # constant rows: uniform softmax, loss ln(width), gradient 1/width - onehot
    c = np.full((2, 64), 3.5)
    l2, _ = to.cross_entropy_rows(c, np.array([0, 63]))
    np.testing.assert_allclose(l2, np.log(64.0), rtol=1e-15)
    d = to.cross_entropy_rows_vjp(c, np.array([0, 63]), np.ones(2))
    assert abs(d[0, 0] - (1 / 64 - 1)) < 1e-15 and abs(d[1, 5] - 1 / 64) < 1e-15


def test_cross_entropy_vjp_central_differences():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(4, 11)) * 2
    t = rng.integers(0, 11, size=4)
    up = rng.normal(size=4)
    dx = to.cross_entropy_rows_vjp(x, t, up)
    f = lambda z: (to.cross_entropy_rows(z, t)[0] * up).sum()  # noqa: E731
    for _ in range(3):
        u = rng.normal(size=x.shape)
        h = 1e-6
        num = (f(x + h * u) - f(x - h * u)) / (2 * h)
        assert abs(num - (dx * u).sum()) < 1e-7 * (1 + abs(num))


def test_powi_matches_exact_powers_for_small_exponents():
    assert to.powi_f32(0.9, 1) == np.float32(0.9)
    assert to.powi_f32(0.9, 2) == np.float32(np.float32(0.9) * np.float32(0.9))
    assert abs(float(to.powi_f32(0.999, 1000)) - 0.999 ** 1000) < 1e-5


@pytest.mark.parametrize("clip", [1e3, 0.05])
def test_adamw_matches_torch_adamw_in_float64(clip):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    p0 = rng.normal(size=(7, 9)).astype(np.float32)
    grads = [rng.normal(size=(7, 9)).astype(np.float32) * s for s in (1.0, 0.3, 2.0)]
    lr, wd = 1e-2, 0.01
    # torch in float64, clipping each gradient by its own norm first
    tp = torch.nn.Parameter(torch.tensor(p0, dtype=torch.float64))
    opt = torch.optim.AdamW([tp], lr=lr, betas=(0.9, 0.999), eps=1e-5, weight_decay=wd)
    p, m, v = p0, None, None
    for t, g in enumerate(grads, start=1):
        tp.grad = torch.tensor(g, dtype=torch.float64)
        torch.nn.utils.clip_grad_norm_([tp], clip)
        opt.step()
        p, m, v = to.adamw_f32(p, g, m, v, t, lr, wd, clip)
    # same update up to f32 rounding (torch divides sqrt(v) by sqrt(c2), the
    # reference takes sqrt(v / c2); both add epsilon outside the root)
    np.testing.assert_allclose(p, tp.detach().numpy(), rtol=0, atol=2e-6)


def test_adamw_first_step_closed_form():
    g = np.array([3.0, -0.5, 1e-3, 0.0], np.float32)
    p = np.array([1.0, -2.0, 0.5, 0.25], np.float32)
    out, m, v = to.adamw_f32(p, g, None, None, 1, 1e-3, 0.0, 1e9)
    # m/c1 = g and sqrt(v/c2) = |g| (up to rounding): step = lr * g / (|g| + 1e-5)
    want = p - 1e-3 * g / (np.abs(g) + 1e-5)
    np.testing.assert_allclose(out, want, rtol=0, atol=1e-7)
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-6)
