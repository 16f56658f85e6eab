"""The GDN-2 mixer module (delta_mixers.mixer) on the HIP operators against a
float64 CPU composition of the same block from plain torch operations
(reference crates/mixers/src/lib.rs:434-693): the convolution as masked lags,
the norms and decay from their formulas, and the recurrence of
crates/mixers/src/reference.rs:41-119 as a differentiable token loop.
Output, input gradient and every parameter gradient are compared with the
north-star fp32 gate (1e-4, rms-floored).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from gpu_util import TOL_F32, gate  # noqa: E402

pytestmark = pytest.mark.gpu


def reference_mixer(p, x, valid, reset, cfg):
    """p: dict of float64 CPU parameter tensors (requires_grad)."""
    F = torch.nn.functional
    B, T, _ = x.shape
    H, K, V = cfg.heads, cfg.key_dim, cfg.value_dim
    x = x * valid[..., None]
    docs = torch.cumsum(reset * valid, dim=1)

    def conv(z, w):
        out = torch.zeros_like(z)
        for lag in range(w.shape[0]):
            if lag >= T:
                break
            same = (docs[:, lag:] == docs[:, :T - lag]).double()
            m = same * valid[:, :T - lag] * valid[:, lag:]
            out = out + F.pad(z[:, :T - lag] * w[lag] * m[..., None], (0, 0, lag, 0))
        return out

    def l2(z):
        return z / torch.sqrt((z * z).sum(-1, keepdim=True) + 1e-6)

    q = l2(F.silu(conv(x @ p["q"].T, p["q_conv"])).view(B, T, H, K))
    k = l2(F.silu(conv(x @ p["k"].T, p["k_conv"])).view(B, T, H, K))
    v = F.silu(conv(x @ p["v"].T, p["v_conv"])).view(B, T, H, V)
    z = (x @ p["decay"].T).view(B, T, H, K) + p["decay_bias"].view(H, K)
    alpha = torch.exp(-F.softplus(z, beta=1, threshold=20) * torch.exp(p["decay_scale"])[:, None])
    erase = torch.sigmoid(x @ p["erase"].T).view(B, T, H, K)
    write = torch.sigmoid(x @ p["write"].T).view(B, T, H, V)
    S = torch.zeros(B, H, K, V, dtype=torch.float64)
    outs = []
    for t in range(T):
        on = valid[:, t].view(B, 1, 1, 1)
        keep = 1 - reset[:, t].view(B, 1, 1, 1) * on
        bar = alpha[:, t, :, :, None] * (S * keep)
        delta = write[:, t] * v[:, t] - ((erase[:, t] * k[:, t])[..., None] * bar).sum(2)
        new = bar + k[:, t, :, :, None] * delta[:, :, None, :]
        outs.append((new * q[:, t, :, :, None]).sum(2) * on[..., 0])
        S = on * new + (1 - on) * S
    out = torch.stack(outs, 1)
    g = (x @ p["output_gate"].T).view(B, T, H, V)
    zz = out * torch.sigmoid(g)
    y = zz / torch.sqrt((zz * zz).mean(-1, keepdim=True) + cfg.norm_epsilon) * p["norm_weight"]
    return (y.reshape(B, T, H * V) @ p["output"].T) * valid[..., None]


def test_mixer_matches_float64_composition():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from delta_mixers.mixer import GdnMixer, GdnMixerConfig
    torch.manual_seed(0)
    cfg = GdnMixerConfig(d_model=32, heads=2, key_dim=8, value_dim=8, chunk_size=16)
    m = GdnMixer(cfg, device="cuda")
    with torch.no_grad():  # nonzero decay parameters and a non-unit norm weight
        m.decay_bias.uniform_(-3, 1)
        m.decay_scale.uniform_(-0.5, 0.5)
        m.norm_weight.uniform_(0.5, 1.5)
    B, T = 2, 21
    x = torch.randn(B, T, cfg.d_model, device="cuda", requires_grad=True)
    valid = torch.ones(B, T, device="cuda")
    valid[0, 5] = 0
    valid[1, T - 3:] = 0
    reset = torch.zeros(B, T, device="cuda")
    reset[0, 9] = 1
    reset[1, 4] = 1
    reset[0, 5] = 1  # on a padding token: ignored
    y = m(x, valid, reset)
    up = torch.randn_like(y)
    (y * up).sum().backward()

    p = {n: t.detach().double().cpu().requires_grad_(True) for n, t in m.named_parameters()}
    xr = x.detach().double().cpu().requires_grad_(True)
    yr = reference_mixer(p, xr, valid.double().cpu(), reset.double().cpu(), cfg)
    (yr * up.double().cpu()).sum().backward()

    gate("output", y, yr.detach().numpy(), TOL_F32)
    gate("dx", x.grad, xr.grad.numpy(), TOL_F32)
    for n, t in m.named_parameters():
        gate(f"d{n}", t.grad, p[n].grad.numpy(), TOL_F32)
    assert np.all(y.detach().cpu().numpy()[1, T - 3:] == 0)
