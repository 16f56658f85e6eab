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


def reference_hola(cq, ck, v, scores, valid, docs, sink, cfg):
    """The cache read as differentiable float64 torch code: membership from the
    oracle's schedule (selection is discrete), then, per valid query, softmax
    over the cache snapshot of its chunk plus its chunk's causal tokens in its
    document, next to the sink logit (crates/mixers/src/hola_checks.rs:294-364)."""
    from oracle import hola_oracle as ho
    B, T, H, K = cq.shape
    sched = ho.hola_schedule(scores.detach().numpy(), valid.numpy(), docs.numpy(),
                             cfg.cache_capacity, cfg.chunk_size, cfg.cache_policy == "recency")
    rows = []
    for b in range(B):
        per_t = []
        for t in range(T):
            per_h = []
            for h in range(H):
                if valid[b, t] < 0.5:
                    per_h.append(torch.zeros(v.shape[3], dtype=v.dtype))
                    continue
                c = t // cfg.chunk_size
                cache = [int(p) for p in sched[b, h, c] if p >= 0]
                vis = [s for s in cache + list(range(c * cfg.chunk_size, t + 1))
                       if valid[b, s] >= 0.5 and docs[b, s] == docs[b, t]]
                logits = (ck[b, vis, h] @ cq[b, t, h]) / K ** 0.5
                w = torch.softmax(torch.cat([logits, sink[h:h + 1]]), 0)
                per_h.append(w[:-1] @ v[b, vis, h])
            per_t.append(torch.stack(per_h))
        rows.append(torch.stack(per_t))
    return torch.stack(rows)


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

    raw_q = F.silu(conv(x @ p["q"].T, p["q_conv"])).view(B, T, H, K)
    raw_k = F.silu(conv(x @ p["k"].T, p["k_conv"])).view(B, T, H, K)
    q, k = l2(raw_q), l2(raw_k)
    v = F.silu(conv(x @ p["v"].T, p["v_conv"])).view(B, T, H, V)
    z = (x @ p["decay"].T).view(B, T, H, K) + p["decay_bias"].view(H, K)
    alpha = torch.exp(-F.softplus(z, beta=1, threshold=20) * torch.exp(p["decay_scale"])[:, None])
    erase = torch.sigmoid(x @ p["erase"].T).view(B, T, H, K)
    write = torch.sigmoid(x @ p["write"].T).view(B, T, H, V)
    S = torch.zeros(B, H, K, V, dtype=torch.float64)
    outs, scores = [], []
    for t in range(T):
        on = valid[:, t].view(B, 1, 1, 1)
        keep = 1 - reset[:, t].view(B, 1, 1, 1) * on
        bar = alpha[:, t, :, :, None] * (S * keep)
        delta = write[:, t] * v[:, t] - ((erase[:, t] * k[:, t])[..., None] * bar).sum(2)
        new = bar + k[:, t, :, :, None] * delta[:, :, None, :]
        outs.append((new * q[:, t, :, :, None]).sum(2) * on[..., 0])
        scores.append((k[:, t].norm(dim=-1) * delta.norm(dim=-1)) * on[:, 0, 0])
        S = on * new + (1 - on) * S
    out = torch.stack(outs, 1)
    if cfg.cache_policy != "none":
        rms = lambda z, w: z / torch.sqrt((z * z).mean(-1, keepdim=True) + cfg.norm_epsilon) * w  # noqa: E731
        exact = reference_hola(rms(raw_q, p["cache_q_norm"]), rms(raw_k, p["cache_k_norm"]), v,
                               torch.stack(scores, 1), valid, docs, p["cache_sink"], cfg)
        out = out + exact * torch.sigmoid(p["cache_gate"]).view(1, 1, H, 1)
    g = (x @ p["output_gate"].T).view(B, T, H, V)
    zz = out * torch.sigmoid(g)
    y = zz / torch.sqrt((zz * zz).mean(-1, keepdim=True) + cfg.norm_epsilon) * p["norm_weight"]
    return (y.reshape(B, T, H * V) @ p["output"].T) * valid[..., None]


# (policy, capacity, chunk): no eviction under the score policy (membership then
# cannot depend on near-ties between f32 and f64 scores); evictions under recency.
CASES = [("none", 16, 16), ("surprise", 16, 16), ("recency", 4, 4)]


@pytest.mark.parametrize("policy,capacity,chunk", CASES)
def test_mixer_matches_float64_composition(policy, capacity, chunk):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from delta_mixers.mixer import GdnMixer, GdnMixerConfig
    torch.manual_seed(0)
    cfg = GdnMixerConfig(d_model=32, heads=2, key_dim=8, value_dim=8, chunk_size=chunk,
                         cache_policy=policy, cache_capacity=capacity)
    m = GdnMixer(cfg, device="cuda")
    with torch.no_grad():  # nonzero decay parameters and a non-unit norm weight
        m.decay_bias.uniform_(-3, 1)
        m.decay_scale.uniform_(-0.5, 0.5)
        m.norm_weight.uniform_(0.5, 1.5)
        if policy != "none":  # an open cache gate and non-unit cache norms
            m.cache_gate.uniform_(-1, 1)
            m.cache_sink.uniform_(-1, 1)
            m.cache_q_norm.uniform_(0.5, 1.5)
            m.cache_k_norm.uniform_(0.5, 1.5)
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
