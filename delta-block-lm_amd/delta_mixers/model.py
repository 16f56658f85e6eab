"""The lm512 GDN language model and its training step.

Each of the `layers` blocks is pre-norm residual
    x += mixer(rms_norm(x));  x += swiglu(rms_norm(x))
followed by a final RMSNorm and the tied embedding as output head, with AdamW
(block structure: crates/experiment/src/model.rs:300-364; train step:
crates/experiment/src/train.rs:335-357; optimizer: update.rs:43-96).  Widths
follow configuration 4, which is not the reference's own lm512 (d_model 512,
8 layers, H8 K64 V64, SwiGLU 1408, vocab 32768, tied head).  The mixer is the scalar-gate gated delta rule:
    q = l2(silu(conv(x Wq)))   k = l2(silu(conv(x Wk)))   v = silu(conv(x Wv))
    beta = sigmoid(x Wb)       g = -exp(decay_scale) * softplus(x Wg + decay_bias)
    o = scan(q, k, v, beta, g)                       chunk-WY HIP kernels
    y = (rms_norm(o) * silu(x Wgate)) Wout           SiLU output gate
The convolution and every norm are the library's HIP operators (float32, as the
reference's); projections and the MLP are GEMMs in `compute_dtype` (bfloat16 by
default, float32 master weights).  In bfloat16, q/k/v enter the scan as bf16 and
take the chunk-WY MFMA path (d_k = d_v = 64, chunk 64); in float32 the scan runs
the token-sequential kernels.

With `fused` (the default for bfloat16) each block is one autograd node whose
backward is written out: the GEMMs stay torch (hipBLASLt) calls and everything
between them runs in the library's fused step operators (delta_kernels.lm_ops):
residual add + RMSNorm to bf16, convolution + SiLU + L2 + gates from the packed
projection, the output gate, SwiGLU, and their VJPs writing bf16 gradients in
place.  The rounding points are those of the unfused bf16 composition, except
that the weight-gradient GEMMs write float32 (the unfused path rounds them to
bf16 first).  The residual stream is carried as (u, r) pairs, u float32 and r
the bf16 branch output, added inside the next norm.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

import delta_kernels as dk


@dataclass
class GdnLMConfig:
    vocab: int = 32768
    d_model: int = 512
    layers: int = 8
    heads: int = 8
    key_dim: int = 64
    value_dim: int = 64
    conv_taps: int = 4
    mlp_width: int = 1408
    chunk: int = 64
    norm_epsilon: float = 1e-6  # the reference model's RMSNorm epsilon (model.rs:108-111)
    decay_bias: float = -4.0  # the reference mixer's initial bias (alpha close to 1)
    compute_dtype: torch.dtype = torch.bfloat16
    fused: bool = True  # bfloat16 only: the fused step operators (module docstring)


def _linear(i, o, device):
    w = torch.empty(o, i, device=device)
    torch.nn.init.normal_(w, std=i ** -0.5)
    return torch.nn.Parameter(w)


def _mm(x, w):
    return F.linear(x, w.to(x.dtype))


class ScalarGdnMixer(torch.nn.Module):
    """Input projections packed in one weight, rows [q | k | v | gate | beta |
    decay] (one GEMM per direction; the reference packs its seven projections
    the same way at execution time, crates/mixers/src/projections.rs:31-44),
    and one depthwise convolution over the q | k | v channels."""

    def __init__(self, cfg: GdnLMConfig, device=None):
        super().__init__()
        self.cfg = cfg
        D, H, K, V = cfg.d_model, cfg.heads, cfg.key_dim, cfg.value_dim
        self.widths = (H * K, H * K, H * V, H * V, H, H)  # q, k, v, gate, beta, decay
        self.in_proj = _linear(D, sum(self.widths), device)
        self.out = _linear(H * V, D, device)
        self.qkv_conv = torch.nn.Parameter(
            torch.empty(cfg.conv_taps, 2 * H * K + H * V, device=device).uniform_(-0.1, 0.1))
        self.decay_scale = torch.nn.Parameter(torch.zeros(H, device=device))
        self.decay_bias = torch.nn.Parameter(torch.full((H,), cfg.decay_bias, device=device))
        self.norm_weight = torch.nn.Parameter(torch.ones(V, device=device))

    def forward(self, x, valid, docs):
        """x [B, T, d_model] in compute_dtype; valid/docs [B, T] float32."""
        cfg = self.cfg
        B, T, _ = x.shape
        H, K, V = cfg.heads, cfg.key_dim, cfg.value_dim
        cd = cfg.compute_dtype
        z = _mm(x, self.in_proj)
        qkv_w = 2 * H * K + H * V
        qkv = dk.causal_conv(z[..., :qkv_w].float(), self.qkv_conv, valid, docs,
                             activation="silu")
        qk = dk.l2_norm(qkv[..., :2 * H * K].view(B, T, 2 * H, K)).to(cd)
        q, k = qk[:, :, :H], qk[:, :, H:]
        v = qkv[..., 2 * H * K:].to(cd).view(B, T, H, V)
        rest = z[..., qkv_w:].float()
        gate, beta, dec = rest[..., :H * V], rest[..., H * V:H * V + H], rest[..., H * V + H:]
        beta = torch.sigmoid(beta)
        g = -torch.exp(self.decay_scale) * F.softplus(dec + self.decay_bias)
        o, _, _ = dk.gdn_scalar_scan(q, k, v, beta, g, valid, None, None, cfg.chunk)
        o = dk.rms_norm(o.float(), self.norm_weight, None, cfg.norm_epsilon)
        y = o.reshape(B, T, H * V) * F.silu(gate)
        return _mm(y.to(cd), self.out)


class SwiGLU(torch.nn.Module):
    """w13 packs the gate and up projections ([w1 | w3] rows): one GEMM."""

    def __init__(self, cfg: GdnLMConfig, device=None):
        super().__init__()
        D, M = cfg.d_model, cfg.mlp_width
        self.M = M
        self.w13 = _linear(D, 2 * M, device)
        self.w2 = _linear(M, D, device)

    def forward(self, x):
        h = _mm(x, self.w13)
        return _mm(F.silu(h[..., :self.M]) * h[..., self.M:], self.w2)


class Block(torch.nn.Module):
    def __init__(self, cfg: GdnLMConfig, device=None):
        super().__init__()
        self.cfg = cfg
        self.norm1 = torch.nn.Parameter(torch.ones(cfg.d_model, device=device))
        self.norm2 = torch.nn.Parameter(torch.ones(cfg.d_model, device=device))
        self.mixer = ScalarGdnMixer(cfg, device)
        self.mlp = SwiGLU(cfg, device)

    def forward(self, x, valid, docs):
        """x [B, T, d_model] float32 residual stream."""
        eps, cd = self.cfg.norm_epsilon, self.cfg.compute_dtype
        x = x + self.mixer(dk.rms_norm(x, self.norm1, None, eps).to(cd), valid, docs).float()
        return x + self.mlp(dk.rms_norm(x, self.norm2, None, eps).to(cd)).float()


def _wgrad(g, x):
    """Weight gradient g^T x in float32 for g [R, N], x [R, D] (bf16, R = batch *
    time).  These outputs are small (N x D <= 2816 x 512) and the reduction long
    (R = 8192 at lm512): one GEMM gives too few output tiles for 256 CUs, so the
    rows are split into 2 or 4 slices, one batched GEMM computes the slices'
    products and a fixed-order sum adds them (split-K; 1.3-2x faster here)."""
    R, N = g.shape
    splits = 4 if N * x.shape[1] <= 1_200_000 else 2
    if R % splits or R < 1024 * splits:
        return torch.mm(g.t(), x, out_dtype=torch.float32)
    gv = g.view(splits, R // splits, N).transpose(1, 2)
    return torch.bmm(gv, x.view(splits, R // splits, -1), out_dtype=torch.float32).sum(0)


class _FusedBlock(torch.autograd.Function):
    """One block on the fused operators: (u, r) -> (u', r') with the block input
    x = u + r (r bf16 or None), u' = x + mixer(norm1(x)), r' = mlp(norm2(u'))."""

    @staticmethod
    def forward(ctx, u_prev, r_prev, norm1, in_proj, conv_w, decay_scale, decay_bias, onorm,
                out_w, norm2, w13, w2, valid, docs, reset, cfg):
        B, T, D = u_prev.shape
        H, R, cd, eps = cfg.heads, B * T, cfg.compute_dtype, cfg.norm_epsilon
        lm = dk.lm_ops
        w_in, w_out, w_13, w_2 = (w.to(cd) for w in (in_proj, out_w, w13, w2))
        x, n1, inv1 = lm.norm_forward(u_prev.reshape(R, D),
                                      None if r_prev is None else r_prev.reshape(R, D), norm1, eps)
        z = torch.mm(n1, w_in.t())
        qkv, beta, g = lm.mixer_in_forward(z, conv_w, valid, docs, decay_scale, decay_bias, B, T, H)
        q, k, v = qkv[:, :, :H], qkv[:, :, H:2 * H], qkv[:, :, 2 * H:]
        o, _, _, ck = dk.gdn_scalar_forward(q, k, v, beta, g, valid, reset, None, cfg.chunk)
        yg, inv_o = lm.mixer_out_forward(o, z, onorm, eps, B, T, H)
        m = torch.mm(yg, w_out.t())
        u, n2, inv2 = lm.norm_forward(x, m, norm2, eps)
        h = torch.mm(n2, w_13.t())
        a = lm.swiglu_forward(h)
        r = torch.mm(a, w_2.t())
        ctx.save_for_backward(x, n1, inv1, z, qkv, beta, g, o, yg, inv_o, u, n2, inv2, h, a,
                              norm1, conv_w, decay_scale, decay_bias, onorm, norm2, valid, docs,
                              reset, w_in, w_out, w_13, w_2)
        ctx.ck, ctx.cfg, ctx.has_r = ck, cfg, r_prev is not None
        return u.view(B, T, D), r.view(B, T, D)

    @staticmethod
    def backward(ctx, du, dr):
        (x, n1, inv1, z, qkv, beta, g, o, yg, inv_o, u, n2, inv2, h, a, norm1, conv_w,
         decay_scale, decay_bias, onorm, norm2, valid, docs, reset, w_in, w_out, w_13,
         w_2) = ctx.saved_tensors
        cfg, ck = ctx.cfg, ctx.ck
        ctx.ck = None
        B, T, D = du.shape
        H, R = cfg.heads, B * T
        lm = dk.lm_ops
        du = du.reshape(R, D).float().contiguous()
        dr = dr.reshape(R, D).to(cfg.compute_dtype).contiguous()
        # MLP branch
        da = torch.mm(dr, w_2)
        dw2 = _wgrad(dr, a)
        dh = lm.swiglu_backward(h, da)
        dw13 = _wgrad(dh, n2)
        dn2 = torch.mm(dh, w_13)
        du_in, dm, dnorm2 = lm.norm_backward(u, norm2, inv2, dn2, du, True)
        # mixer branch
        dyg = torch.mm(dm, w_out)
        dwout = _wgrad(dm, yg)
        dz = torch.empty_like(z)
        d_o, donorm = lm.mixer_out_backward(o, z, onorm, inv_o, dyg, dz, B, T, H)
        q, k, v = qkv[:, :, :H], qkv[:, :, H:2 * H], qkv[:, :, 2 * H:]
        dq, dkk, dv, dbeta, dg, _ = dk.gdn_scalar_backward(q, k, v, beta, g, valid, reset, ck,
                                                           cfg.chunk, d_o)
        dconv, dds, ddb = lm.mixer_in_backward(z, conv_w, valid, docs, decay_scale, decay_bias,
                                               dq, dkk, dv, dbeta, dg, dz, B, T, H)
        dwin = _wgrad(dz, n1)
        dn1 = torch.mm(dz, w_in)
        dx, dxb, dnorm1 = lm.norm_backward(x, norm1, inv1, dn1, du_in, ctx.has_r)
        return (dx.view(B, T, D), None if dxb is None else dxb.view(B, T, D), dnorm1,
                dwin, dconv, dds, ddb, donorm, dwout, dnorm2, dw13, dw2, None, None, None, None)


class _FusedFinalNorm(torch.autograd.Function):
    """The final RMSNorm of the (u, r) stream, to bf16 [B T, D]."""

    @staticmethod
    def forward(ctx, u, r, weight, eps):
        B, T, D = u.shape
        x, y, inv = dk.lm_ops.norm_forward(u.reshape(B * T, D),
                                           None if r is None else r.reshape(B * T, D), weight, eps)
        ctx.save_for_backward(x, weight, inv)
        ctx.shape, ctx.has_r = (B, T, D), r is not None
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, inv = ctx.saved_tensors
        dx, dxb, dw = dk.lm_ops.norm_backward(x, weight, inv, dy.to(torch.bfloat16).contiguous(),
                                              None, ctx.has_r)
        return dx.view(ctx.shape), None if dxb is None else dxb.view(ctx.shape), dw, None


class GdnLM(torch.nn.Module):
    def __init__(self, cfg: GdnLMConfig, device=None):
        super().__init__()
        self.cfg = cfg
        self.embed = torch.nn.Parameter(torch.randn(cfg.vocab, cfg.d_model, device=device) * 0.02)
        self.blocks = torch.nn.ModuleList(Block(cfg, device) for _ in range(cfg.layers))
        self.norm = torch.nn.Parameter(torch.ones(cfg.d_model, device=device))

    def features(self, tokens):
        """tokens [B, T] int64 -> final-norm features [B, T, d_model] float32."""
        B, T = tokens.shape
        valid = torch.ones(B, T, device=tokens.device)
        docs = torch.zeros(B, T, device=tokens.device)
        x = self.embed[tokens]
        for blk in self.blocks:
            x = blk(x, valid, docs)
        return dk.rms_norm(x, self.norm, None, self.cfg.norm_epsilon)

    def _fused(self) -> bool:
        """The fused operators cover bf16 models with K = V = 64, an even power-of-two
        head count up to 32, d_model 128 or a multiple of 256 up to 1024, and an
        MLP width that is a multiple of 8; other shapes take the unfused path."""
        c = self.cfg
        H = c.heads
        return (c.fused and c.compute_dtype == torch.bfloat16 and c.key_dim == 64 and
                c.value_dim == 64 and 2 <= H <= 32 and H & (H - 1) == 0 and
                (c.d_model == 128 or (c.d_model % 256 == 0 and c.d_model <= 1024)) and
                c.mlp_width % 8 == 0 and 1 <= c.conv_taps <= 8)

    def features_bf16(self, tokens):
        """tokens [B, T] -> final-norm features [B T, d_model] bf16 on the
        fused step operators."""
        cfg = self.cfg
        B, T = tokens.shape
        dev = tokens.device
        valid = torch.ones(B, T, device=dev)
        docs = torch.zeros(B, T, device=dev)
        reset = torch.zeros(B, T, device=dev)
        u, r = self.embed[tokens], None
        for blk in self.blocks:
            mx, mlp = blk.mixer, blk.mlp
            u, r = _FusedBlock.apply(u, r, blk.norm1, mx.in_proj, mx.qkv_conv, mx.decay_scale,
                                     mx.decay_bias, mx.norm_weight, mx.out, blk.norm2, mlp.w13,
                                     mlp.w2, valid, docs, reset, cfg)
        return _FusedFinalNorm.apply(u, r, self.norm, cfg.norm_epsilon)

    def forward(self, tokens):
        """tokens [B, T] int64 -> logits [B, T, vocab] in compute_dtype."""
        if self._fused():
            B, T = tokens.shape
            return _mm(self.features_bf16(tokens), self.embed).view(B, T, -1)
        return _mm(self.features(tokens).to(self.cfg.compute_dtype), self.embed)

    def loss(self, tokens):
        """Mean next-token cross entropy over positions 0..T-2: the tied head and
        the loss in one operator (logits computed once, replaced in place by
        their gradient)."""
        cd = self.cfg.compute_dtype
        if self._fused():
            h = self.features_bf16(tokens[:, :-1])
        else:
            h = self.features(tokens[:, :-1]).to(cd)
        return dk.linear_cross_entropy(h.reshape(-1, self.cfg.d_model), self.embed.to(cd),
                                       tokens[:, 1:].reshape(-1))


def make_optimizer(model: GdnLM, lr: float = 1e-3, weight_decay: float = 0.01,
                   clip: float = 1.0):
    """The reference's optimizer (FusedAdamW: per-parameter gradient clipping,
    then AdamW; crates/experiment/src/train.rs:20-38) over float32 master
    weights, with its default hyperparameters (config.rs:442-444)."""
    return dk.FusedAdamW(model.parameters(), lr=lr, weight_decay=weight_decay, clip=clip)


def train_step(model: GdnLM, opt: torch.optim.Optimizer, tokens: torch.Tensor) -> torch.Tensor:
    """One forward, backward and AdamW update; returns the detached loss."""
    opt.zero_grad(set_to_none=True)
    loss = model.loss(tokens)
    loss.backward()
    opt.step()
    return loss.detach()
