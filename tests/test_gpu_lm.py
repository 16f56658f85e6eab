"""The configuration-4 language model (delta_mixers.model) on the HIP operators
against a float64 CPU composition of the same network from plain torch
operations: block structure of crates/experiment/src/model.rs:300-364
(pre-norm residual mixer and MLP, final RMSNorm, head), the convolution as
masked lags, the norms from their formulas, and the scalar-gate recurrence of
crates/mixers/src/reference.rs:68-111 (alpha = exp(g) on every key channel,
erase = write = beta) as a differentiable token loop.

float32 model (token-sequential scan, float32 GEMMs) against the exact
float64 composition: the loss within the north-star fp32 gate (1e-4); each
parameter gradient within 1e-4 normwise and 5e-4 elementwise (rms-floored).
The model composes two scans, each within 1e-4 of its oracle, and ~30 other
f32 operators; measured on two initialisations: worst normwise 2.2e-5,
worst elementwise 1.1e-4.  This pins the model's semantics.

bfloat16 model (the chunk-WY MFMA scan, bf16 GEMMs): compared with the same
composition rounded to bfloat16 wherever the model holds bfloat16 values
(reference_loss(bf16=True)).  These gradients are sensitive to rounding: bf16
rounding alone moves them 2-10% (normwise) away from exact float64 (the
"spread", computed per parameter in the test).  The gates, per gradient:
distance to the bf16-rounded reference at most the spread (measured: 0.22-0.78
of it), distance to exact float64 at most 1.5 x the spread (measured: up to
1.14 x); the loss within 1e-4 relative of the bf16-rounded reference.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from gpu_util import TOL_F32, gate  # noqa: E402

pytestmark = pytest.mark.gpu

F = torch.nn.functional


def _rms(x, w, eps):
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * w


def _conv(z, w):
    T = z.shape[1]
    out = torch.zeros_like(z)
    for lag in range(min(w.shape[0], T)):
        out = out + F.pad(z[:, :T - lag] * w[lag], (0, 0, lag, 0))
    return out


def _l2(z):
    return z / torch.sqrt((z * z).sum(-1, keepdim=True) + 1e-6)


def _scan(q, k, v, beta, g):
    B, T, H, K = q.shape
    S = torch.zeros(B, H, K, v.shape[3], dtype=q.dtype)
    outs = []
    for t in range(T):
        bar = torch.exp(g[:, t])[..., None, None] * S
        delta = beta[:, t, :, None] * (v[:, t] - (k[:, t, :, :, None] * bar).sum(2))
        S = bar + k[:, t, :, :, None] * delta[:, :, None, :]
        outs.append((S * q[:, t, :, :, None]).sum(2))
    return torch.stack(outs, 1)


def _r(x):
    """Round to the nearest bfloat16 value (kept in float64)."""
    return x.to(torch.bfloat16).to(x.dtype)


class _Bf16(torch.autograd.Function):
    """A tensor the model holds in bfloat16: rounded value, rounded gradient."""

    @staticmethod
    def forward(ctx, x):
        return _r(x)

    @staticmethod
    def backward(ctx, g):
        return _r(g)


class _Bf16Linear(torch.autograd.Function):
    """F.linear(a, W.to(bf16)) on a bf16 input: bf16 product of rounded
    operands; gradients of the bf16 output rounded first, bf16 dA and dW."""

    @staticmethod
    def forward(ctx, a, w):
        ctx.save_for_backward(a, w)
        return _r(a @ _r(w).T)

    @staticmethod
    def backward(ctx, g):
        a, w = ctx.saved_tensors
        g = _r(g)
        return _r(g @ _r(w)), _r(g.reshape(-1, g.shape[-1]).T @ a.reshape(-1, a.shape[-1]))


class _Bf16Silu(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a):
        ctx.save_for_backward(a)
        return _r(F.silu(a))

    @staticmethod
    def backward(ctx, g):
        (a,) = ctx.saved_tensors
        s = torch.sigmoid(a)
        return _r(_r(g) * s * (1 + a * (1 - s)))


class _Bf16Mul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return _r(a * b)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        g = _r(g)
        return _r(g * b), _r(g * a)


def reference_loss(p, tokens, cfg, bf16=False):
    """p: dict name -> float64 CPU tensor (requires_grad).  With bf16, every
    value the bfloat16 model holds in bfloat16 is rounded to it, forward and
    backward; everything else is exact float64."""
    eps = cfg.norm_epsilon
    H, K, V = cfg.heads, cfg.key_dim, cfg.value_dim
    cast = _Bf16.apply if bf16 else (lambda x: x)
    lin = _Bf16Linear.apply if bf16 else (lambda a, w: a @ w.T)
    silu = _Bf16Silu.apply if bf16 else F.silu
    mul = _Bf16Mul.apply if bf16 else (lambda a, b: a * b)
    inp, tgt = tokens[:, :-1], tokens[:, 1:]
    B, T = inp.shape
    x = p["embed"][inp]
    HK, HV = H * K, H * V
    for i in range(cfg.layers):
        m = f"blocks.{i}.mixer."
        h = cast(_rms(x, p[f"blocks.{i}.norm1"], eps))
        z = lin(h, p[m + "in_proj"])
        cw = p[m + "qkv_conv"]
        q = cast(_l2(F.silu(_conv(z[..., :HK], cw[:, :HK])).view(B, T, H, K)))
        k = cast(_l2(F.silu(_conv(z[..., HK:2 * HK], cw[:, HK:2 * HK])).view(B, T, H, K)))
        v = cast(F.silu(_conv(z[..., 2 * HK:2 * HK + HV], cw[:, 2 * HK:])).view(B, T, H, V))
        gate = z[..., 2 * HK + HV:2 * HK + 2 * HV]
        beta = torch.sigmoid(z[..., 2 * HK + 2 * HV:2 * HK + 2 * HV + H])
        g = -torch.exp(p[m + "decay_scale"]) * F.softplus(z[..., 2 * HK + 2 * HV + H:] +
                                                          p[m + "decay_bias"])
        o = _rms(cast(_scan(q, k, v, beta, g)), p[m + "norm_weight"], eps)
        y = o.reshape(B, T, HV) * F.silu(gate)
        x = x + lin(cast(y), p[m + "out"])
        h = cast(_rms(x, p[f"blocks.{i}.norm2"], eps))
        f = f"blocks.{i}.mlp."
        a = lin(h, p[f + "w13"])
        M = cfg.mlp_width
        x = x + lin(mul(silu(a[..., :M]), a[..., M:]), p[f + "w2"])
    logits = lin(cast(_rms(x, p["norm"], eps)), p["embed"])
    return F.cross_entropy(logits.reshape(-1, cfg.vocab), tgt.reshape(-1))


def _small(dtype):
    from delta_mixers.model import GdnLMConfig
    return GdnLMConfig(vocab=512, d_model=128, layers=2, heads=2, key_dim=64, value_dim=64,
                       mlp_width=256, chunk=64, compute_dtype=dtype)


def _perturbed_model(cfg):
    from delta_mixers.model import GdnLM
    torch.manual_seed(0)
    model = GdnLM(cfg, device="cuda")
    with torch.no_grad():  # move gates and norms off their initial constants
        for n, t in model.named_parameters():
            if n.endswith("decay_bias"):
                t.uniform_(-3, 1)
            elif n.endswith("decay_scale"):
                t.uniform_(-0.5, 0.5)
            elif "norm" in n:
                t.uniform_(0.5, 1.5)
    return model


def _reference_grads(model, tokens, cfg, bf16):
    p = {n: t.detach().double().cpu().requires_grad_(True) for n, t in model.named_parameters()}
    ref = reference_loss(p, tokens, cfg, bf16)
    ref.backward()
    return ref.item(), {n: t.grad.numpy() for n, t in p.items()}


def _run(dtype, B=2, T=131):
    cfg = _small(dtype)
    model = _perturbed_model(cfg)
    gen = torch.Generator().manual_seed(1)
    tokens = torch.randint(0, cfg.vocab, (B, T), generator=gen)
    loss = model.loss(tokens.cuda())
    loss.backward()
    return model, loss, tokens, cfg


def _normwise(a, b):
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_lm_float32_matches_float64_composition():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    model, loss, tokens, cfg = _run(torch.float32)
    ref, grads = _reference_grads(model, tokens, cfg, False)
    gate("loss", loss, np.array(ref), TOL_F32)
    for n, t in model.named_parameters():
        gate(f"d{n}", t.grad, grads[n], 5e-4)
        err = _normwise(t.grad.double().cpu().numpy(), grads[n])
        assert err <= 1e-4, f"d{n}: normwise relative error {err:.3e}"


def test_lm_bfloat16_chunk_path_matches_bf16_rounded_composition():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels as dk
    dk.stage_timing(True)  # the chunk-path kernels record events only when they run
    try:
        model, loss, tokens, cfg = _run(torch.bfloat16)
        torch.cuda.synchronize()
        ran = set(dk.stage_times())
    finally:
        dk.stage_timing(False)
    assert {"chunk_prep", "chunk_bgrad"} <= ran, "the bf16 model must take the chunk-WY path"
    ref16, g16 = _reference_grads(model, tokens, cfg, True)
    _, g64 = _reference_grads(model, tokens, cfg, False)
    assert abs(loss.item() - ref16) <= 1e-4 * abs(ref16)
    for n, t in model.named_parameters():
        got = t.grad.double().cpu().numpy()
        assert np.all(np.isfinite(got)), f"d{n}: nonfinite values"
        spread = _normwise(g16[n], g64[n])
        near = np.linalg.norm(got - g16[n]) / np.linalg.norm(g64[n])
        far = _normwise(got, g64[n])
        assert near <= spread, f"d{n}: {near:.3e} from the bf16 reference, spread {spread:.3e}"
        assert far <= 1.5 * spread, f"d{n}: {far:.3e} from float64, spread {spread:.3e}"


def test_lm_fused_matches_unfused_within_bf16_spread():
    """The fused bf16 model (delta_kernels.lm_ops, one autograd node per block)
    against the unfused bf16 composition of the reference-mirrored operators,
    same weights and tokens.  Both hold the same bf16 values but sum in
    different orders (and the fused weight gradients stay float32), so they
    differ by bf16 rounding flips: per gradient, their distance must be at most
    the bf16 spread against exact float64; the losses within 2e-4 relative."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from dataclasses import replace

    from delta_mixers.model import GdnLM
    cfg = _small(torch.bfloat16)
    fused = _perturbed_model(cfg)
    assert fused._fused()
    plain = GdnLM(replace(cfg, fused=False), device="cuda")
    plain.load_state_dict(fused.state_dict())
    assert not plain._fused()
    tokens = torch.randint(0, cfg.vocab, (2, 131), generator=torch.Generator().manual_seed(1))
    lf = fused.loss(tokens.cuda())
    lf.backward()
    lp = plain.loss(tokens.cuda())
    lp.backward()
    assert abs(lf.item() - lp.item()) <= 2e-4 * abs(lp.item())
    _, g16 = _reference_grads(fused, tokens, cfg, True)
    _, g64 = _reference_grads(fused, tokens, cfg, False)
    for (n, a), (_, b) in zip(fused.named_parameters(), plain.named_parameters()):
        ga, gb = a.grad.double().cpu().numpy(), b.grad.double().cpu().numpy()
        assert np.all(np.isfinite(ga)), f"d{n}: nonfinite values"
        spread = _normwise(g16[n], g64[n])
        dist = np.linalg.norm(ga - gb) / np.linalg.norm(g64[n])
        assert dist <= spread, f"d{n}: fused vs unfused {dist:.3e}, spread {spread:.3e}"


def test_lm_training_steps_reduce_loss():
    """AdamW steps on one fixed batch drive its loss down (the update wiring)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from delta_mixers.model import GdnLM, make_optimizer, train_step
    cfg = _small(torch.bfloat16)
    torch.manual_seed(0)
    model = GdnLM(cfg, device="cuda")
    opt = make_optimizer(model, lr=3e-3)
    tokens = torch.randint(0, cfg.vocab, (4, 129), device="cuda")
    losses = [train_step(model, opt, tokens).item() for _ in range(12)]
    assert all(np.isfinite(losses))
    assert losses[-1] < losses[0] - 0.5, losses
