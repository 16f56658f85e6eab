"""The fused operators of the lm512 training step (delta_kernels.lm_ops) against
float64 compositions of the same formulas on the CPU.

These operators have no counterpart in the reference; their contract is the
unfused bf16 composition they replace (delta_mixers.model with fused=False):
every value computed in f32 and rounded to bf16 only where that composition
holds bf16.  So bf16 outputs must lie within one bf16 rounding of the float64
value (|got - ref| <= 2^-8 |ref| + tiny: the f32 arithmetic may land on the
other side of a rounding boundary, never further), and f32 outputs and
parameter gradients (fixed-order sums) within 1e-5 normwise.  Also: the two
mixer VJPs write complementary column sets of dz (every column exactly once),
ragged sizes (rows not a multiple of the workgroup's, T not a multiple of the
32-step segment), masks with padding and document boundaries.  The fused
model against the unfused one is in test_gpu_lm.py (it needs that file's
float64 reference for its gate).
"""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

F = torch.nn.functional
BF = torch.bfloat16


def _lm():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels as dk
    return dk.lm_ops


def _bf16_close(name, got, ref, slack=1e-6, loose=None):
    """got (bf16, any device) within one bf16 rounding of ref (float64): a
    relative half-ulp 2^-8 |ref| (widened 0.1 % for the f32 arithmetic) plus
    slack * max |ref| for cancellation.  Entries flagged in `loose` may be off
    by two roundings (an intermediate bf16 value on a rounding boundary)."""
    g = got.double().cpu()
    r = ref.double().cpu()
    bound = 2.0 ** -8 * 1.001 * r.abs() + slack * float(r.abs().max())
    if loose is not None:
        bound = torch.where(loose, 2 * bound + 2.0 ** -7 * r.abs(), bound)
    bad = (g - r).abs() > bound
    assert not bool(bad.any()), (
        f"{name}: {int(bad.sum())} of {g.numel()} values off by more than one bf16 rounding; "
        f"worst {float(((g - r).abs() - bound).max()):.3e}")


def _ambiguous(x):
    """Entries of x (float64) within 1e-5 relative of a bf16 rounding boundary
    (the kernels' f32 pointwise ops are accurate to about 1e-6 relative)."""
    return (x * (1 + 1e-5)).to(BF) != (x * (1 - 1e-5)).to(BF)


def _zstride(H):
    """A z row stride for H heads: the packed width, a multiple of 4, plus padding."""
    return (4 * H * 64 + 2 * H + 3) // 4 * 4 + 4


def _normwise(name, got, ref, tol):
    g = got.double().cpu()
    r = ref.double().cpu()
    err = float((g - r).norm() / max(float(r.norm()), 1e-30))
    assert err <= tol, f"{name}: normwise error {err:.3e} > {tol:.1e}"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ---- RMSNorm with residual ------------------------------------------------------------


@pytest.mark.parametrize("rows,width", [(1, 128), (1003, 128), (1001, 256), (997, 512),
                                        (513, 768), (258, 1024)])
def test_norm_forward_backward(rows, width):
    lm = _lm()
    gen = _gen(rows + width)
    x = torch.randn(rows, width, generator=gen)
    r = torch.randn(rows, width, generator=gen).to(BF)
    w = torch.rand(width, generator=gen) + 0.5
    dy = torch.randn(rows, width, generator=gen).to(BF)
    dres = torch.randn(rows, width, generator=gen)
    eps = 1e-6
    for with_r in (True, False):
        rr = r.cuda() if with_r else None
        u, y, inv = lm.norm_forward(x.cuda(), rr, w.cuda(), eps)
        # reference, float64 from the f32 sum (exact in f64 for these inputs)
        uf = x + r.float() if with_r else x
        assert torch.equal(u.cpu(), uf), "u = x + r must be the f32 sum"
        ud = uf.double().requires_grad_(True)
        invd = 1.0 / torch.sqrt((ud * ud).mean(-1, keepdim=True) + eps)
        yd = ud * invd * w.double()
        _normwise("inverse", inv, invd[:, 0].detach(), 1e-6)
        _bf16_close("y", y, yd.detach())
        for with_res in (True, False):
            dx, dxb, dw = lm.norm_backward(u, w.cuda(), inv, dy.cuda(),
                                           dres.cuda() if with_res else None, True)
            wd = w.double().requires_grad_(True)
            ud2 = uf.double().requires_grad_(True)
            inv2 = 1.0 / torch.sqrt((ud2 * ud2).mean(-1, keepdim=True) + eps)
            (ud2 * inv2 * wd * dy.double()).sum().backward()
            ref_dx = ud2.grad + (dres.double() if with_res else 0)
            _normwise("dx", dx, ref_dx, 1e-5)
            assert torch.equal(dxb.cpu(), dx.cpu().to(BF)), "dx_bf16 must be dx rounded"
            _normwise("dweight", dw, wd.grad, 1e-5)


def test_norm_rejects_bad_width():
    lm = _lm()
    from delta_kernels._lib import Gdn2Error
    x = torch.randn(4, 192, device="cuda")
    with pytest.raises(Gdn2Error, match="width"):
        lm.norm_forward(x, None, torch.ones(192, device="cuda"), 1e-6)


# ---- mixer prologue / epilogue --------------------------------------------------------


def _masks(B, T, gen):
    valid = torch.ones(B, T)
    docs = torch.zeros(B, T)
    if T > 40:
        valid[0, 5] = 0.0
        valid[-1, T - 3:] = 0.0  # trailing padding
        docs[0, T // 3:] = 1.0
        docs[-1, 17:] = 1.0
        docs[-1, 60 % T:] = 2.0
    return valid, docs


def _conv_ref(zc, w, valid, docs):
    """Depthwise causal conv with the lag mask of gdn2_conv_forward (float64)."""
    B, T, C = zc.shape
    out = torch.zeros_like(zc)
    for lag in range(w.shape[0]):
        if lag >= T:
            break
        src = zc[:, :T - lag]
        m = (valid[:, :T - lag] * valid[:, lag:] *
             (docs[:, :T - lag] == docs[:, lag:]).double())
        out[:, lag:] = out[:, lag:] + src * w[lag] * m[..., None]
    return out


def _in_ref(z, conv_w, valid, docs, ds, db, B, T, H):
    """Float64 composition of mixer_in_forward from z (float64, requires grad ok)."""
    C = 3 * H * 64
    zz = z.view(B, T, -1)
    s = F.silu(_conv_ref(zz[..., :C], conv_w, valid.double(), docs.double()))
    qk = s[..., :2 * H * 64].reshape(B, T, 2 * H, 64)
    qk = qk / torch.sqrt((qk * qk).sum(-1, keepdim=True) + 1e-6)
    v = s[..., 2 * H * 64:].reshape(B, T, H, 64)
    cb = C + H * 64
    beta = torch.sigmoid(zz[..., cb:cb + H])
    g = -torch.exp(ds) * F.softplus(zz[..., cb + H:cb + 2 * H] + db)
    return torch.cat([qk, v], 2), beta, g


@pytest.mark.parametrize("B,T,H,taps", [(2, 131, 2, 4), (1, 64, 8, 4), (2, 45, 4, 3),
                                        (1, 7, 1, 8)])
def test_mixer_in_forward_backward(B, T, H, taps):
    lm = _lm()
    gen = _gen(B * 1000 + T + H)
    Z = _zstride(H)
    z = (torch.randn(B * T, Z, generator=gen) * 1.5).to(BF)
    conv_w = torch.rand(taps, 3 * H * 64, generator=gen) - 0.5
    valid, docs = _masks(B, T, gen)
    ds = torch.rand(H, generator=gen) - 0.5
    db = torch.rand(H, generator=gen) * 4 - 3
    zc = z.cuda()
    qkv, beta, g = lm.mixer_in_forward(zc, conv_w.cuda(), valid.cuda(), docs.cuda(), ds.cuda(),
                                       db.cuda(), B, T, H)
    zd = z.double().requires_grad_(True)
    cwd = conv_w.double().requires_grad_(True)
    dsd = ds.double().requires_grad_(True)
    dbd = db.double().requires_grad_(True)
    rq, rb, rg = _in_ref(zd, cwd, valid, docs, dsd, dbd, B, T, H)
    _bf16_close("qkv", qkv, rq.detach())
    _normwise("beta", beta, rb.detach(), 1e-6)
    _normwise("g", g, rg.detach(), 1e-6)
    # VJP, with the gate columns left to mixer_out_backward
    dq = torch.randn(B, T, H, 64, generator=gen).to(BF)
    dk_ = torch.randn(B, T, H, 64, generator=gen).to(BF)
    dv = torch.randn(B, T, H, 64, generator=gen).to(BF)
    dbeta = torch.randn(B, T, H, generator=gen)
    dg = torch.randn(B, T, H, generator=gen)
    sentinel = torch.full((B * T, Z), 7.0, dtype=BF, device="cuda")
    dz = sentinel.clone()
    dconv, dds, ddb = lm.mixer_in_backward(zc, conv_w.cuda(), valid.cuda(), docs.cuda(), ds.cuda(),
                                           db.cuda(), dq.cuda(), dk_.cuda(), dv.cuda(),
                                           dbeta.cuda(), dg.cuda(), dz, B, T, H)
    up = torch.cat([dq, dk_, dv], 2).double()
    (rq * up).sum().backward(retain_graph=True)
    ((rb * dbeta.double()).sum() + (rg * dg.double()).sum()).backward()
    C, cb = 3 * H * 64, 4 * H * 64
    cols = list(range(C)) + list(range(cb, cb + 2 * H))
    _bf16_close("dz", dz[:, cols], zd.grad[:, cols], slack=1e-5)
    untouched = [c for c in range(Z) if c not in set(cols)]
    assert torch.equal(dz[:, untouched], sentinel[:, untouched]), "wrote outside its columns"
    _normwise("dconv", dconv, cwd.grad, 1e-5)
    _normwise("ddecay_scale", dds, dsd.grad, 1e-5)
    _normwise("ddecay_bias", ddb, dbd.grad, 1e-5)


@pytest.mark.parametrize("B,T,H", [(2, 131, 2), (3, 33, 8), (1, 1, 1)])
def test_mixer_out_forward_backward(B, T, H):
    lm = _lm()
    gen = _gen(7 * B + T + H)
    Z = _zstride(H)
    z = (torch.randn(B * T, Z, generator=gen) * 2).to(BF)
    o = torch.randn(B, T, H, 64, generator=gen).to(BF)
    w = torch.rand(64, generator=gen) + 0.5
    eps = 1e-6
    y, inv = lm.mixer_out_forward(o.cuda(), z.cuda(), w.cuda(), eps, B, T, H)
    od = o.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    zd = z.double().requires_grad_(True)
    gc = 3 * H * 64
    gate = zd[:, gc:gc + H * 64].reshape(B, T, H, 64)
    invd = 1.0 / torch.sqrt((od * od).mean(-1, keepdim=True) + eps)
    yd = (od * invd * wd) * F.silu(gate)
    _bf16_close("y", y, yd.detach().reshape(B * T, H * 64))
    _normwise("inverse", inv, invd.detach().reshape(-1), 1e-6)
    dy = torch.randn(B * T, H * 64, generator=gen).to(BF)
    sentinel = torch.full((B * T, Z), 7.0, dtype=BF, device="cuda")
    dz = sentinel.clone()
    d_o, dw = lm.mixer_out_backward(o.cuda(), z.cuda(), w.cuda(), inv, dy.cuda(), dz, B, T, H)
    (yd.reshape(B * T, H * 64) * dy.double()).sum().backward()
    _bf16_close("d_o", d_o, od.grad, slack=1e-5)
    _bf16_close("dgate", dz[:, gc:gc + H * 64], zd.grad[:, gc:gc + H * 64], slack=1e-5)
    others = list(range(gc)) + list(range(gc + H * 64, Z))
    assert torch.equal(dz[:, others], sentinel[:, others]), "wrote outside the gate columns"
    _normwise("dnorm_w", dw, wd.grad, 1e-5)


@pytest.mark.parametrize("rows,M", [(1, 8), (517, 1408), (64, 256)])
def test_swiglu_matches_bf16_composition(rows, M):
    lm = _lm()
    gen = _gen(rows + M)
    h = (torch.randn(rows, 2 * M, generator=gen) * 3).to(BF)
    a = lm.swiglu_forward(h.cuda())
    hd = h.double()
    s64 = F.silu(hd[:, :M])
    s = s64.to(BF).double()  # the composition rounds silu to bf16
    amb = _ambiguous(s64)
    _bf16_close("a", a, s * hd[:, M:], loose=amb)
    da = torch.randn(rows, M, generator=gen).to(BF)
    dh = lm.swiglu_backward(h.cuda(), da.cuda())
    g, u, d = hd[:, :M], hd[:, M:], da.double()
    sg = torch.sigmoid(g)
    ds = (d * u).to(BF).double()  # the product's gradient is held in bf16
    _bf16_close("dgate", dh[:, :M], ds * sg * (1 + g * (1 - sg)), slack=1e-5)
    _bf16_close("dup", dh[:, M:], d * s, slack=1e-5, loose=amb)
