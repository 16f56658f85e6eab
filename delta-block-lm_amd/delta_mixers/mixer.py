"""The GDN-2 mixer around the scan (reference crates/mixers/src/lib.rs:205-262
construction, :434-693 forward), on the MI355X operators.

Per block input x [B, T, d_model] with masks valid/reset [B, T]:
  x <- x * valid;  documents = cumsum(reset * valid) over time       (lib.rs:447-455)
  q = l2(silu(conv(x Wq)))   k = l2(silu(conv(x Wk)))   v = silu(conv(x Wv))
  alpha = decay(x Wdecay, decay_bias, decay_scale)                    (lib.rs:460-503)
  erase = sigmoid(x Werase)   write = sigmoid(x Wwrite)              (lib.rs:504-523)
  out = scan(q, k, v, alpha, erase, write; valid, reset)             (lib.rs:524-565)
  y = rms_norm(out, norm_weight, gate = x Wgate, eps 1e-5) Wout * valid (lib.rs:661-693)
With cache_policy "surprise" or "recency" the mixer also reads the HOLA exact
cache (lib.rs:570-660): RMS-normed raw q and k (cache norms, eps 1e-5) attend to
the top-capacity tokens chosen by the scan's scores (or recency), and the read
joins the scan output scaled by sigmoid(cache gate) per head:
  out += hola_read(rms(q_raw), rms(k_raw), v, scores, ...) * sigmoid(gate)
The convolution fuses its SiLU (one pass over the projection), the gated RMSNorm
is one pass, and the recurrence is the HIP scan (channel-wise gates: the
16-token chunk kernels).  Projections are plain GEMMs (torch, hipBLASLt).
The reference's SBD block is not part of this module.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

import delta_kernels as dk


@dataclass
class GdnMixerConfig:
    d_model: int = 512
    heads: int = 8
    key_dim: int = 64
    value_dim: int = 64
    chunk_size: int = 16
    conv_taps: int = 4
    norm_epsilon: float = 1e-5  # burn RmsNormConfig default, the mixer's output norm
    cache_policy: str = "none"  # "none", "surprise" (scan scores) or "recency" (lib.rs:131-158)
    cache_capacity: int = 16


class GdnMixer(torch.nn.Module):
    """Parameters and initialisation follow lib.rs:216-235: bias-free linear
    projections, conv weights U(-0.1, 0.1) [taps, channels], decay_scale 0,
    decay_bias -4, output RMSNorm weight 1."""

    def __init__(self, cfg: GdnMixerConfig, device=None):
        super().__init__()
        self.cfg = cfg
        H, K, V, D = cfg.heads, cfg.key_dim, cfg.value_dim, cfg.d_model
        kw, vw = H * K, H * V

        def linear(i, o):
            w = torch.empty(o, i, device=device)
            torch.nn.init.kaiming_uniform_(w, a=5 ** 0.5)  # burn LinearConfig default init
            return torch.nn.Parameter(w)

        self.q = linear(D, kw)
        self.k = linear(D, kw)
        self.v = linear(D, vw)
        self.decay = linear(D, kw)
        self.erase = linear(D, kw)
        self.write = linear(D, vw)
        self.output_gate = linear(D, vw)
        self.output = linear(vw, D)
        conv = lambda c: torch.nn.Parameter(  # noqa: E731
            torch.empty(cfg.conv_taps, c, device=device).uniform_(-0.1, 0.1))
        self.q_conv, self.k_conv, self.v_conv = conv(kw), conv(kw), conv(vw)
        self.decay_scale = torch.nn.Parameter(torch.zeros(H, device=device))
        self.decay_bias = torch.nn.Parameter(torch.full((kw,), -4.0, device=device))
        self.norm_weight = torch.nn.Parameter(torch.ones(V, device=device))
        if cfg.cache_policy not in ("none", "surprise", "recency"):
            raise ValueError(f"unknown cache policy {cfg.cache_policy!r}")
        if cfg.cache_policy != "none":  # lib.rs:236-243
            self.cache_q_norm = torch.nn.Parameter(torch.ones(K, device=device))
            self.cache_k_norm = torch.nn.Parameter(torch.ones(K, device=device))
            self.cache_gate = torch.nn.Parameter(torch.full((H,), -4.0, device=device))
            self.cache_sink = torch.nn.Parameter(torch.zeros(H, device=device))

    def forward(self, x: torch.Tensor, valid: torch.Tensor = None,
                reset: torch.Tensor = None) -> torch.Tensor:
        cfg = self.cfg
        B, T, _ = x.shape
        H, K, V = cfg.heads, cfg.key_dim, cfg.value_dim
        if valid is None:
            valid = torch.ones(B, T, device=x.device)
        if reset is None:
            reset = torch.zeros(B, T, device=x.device)
        valid, reset = valid.float(), reset.float()
        x = x * valid[..., None]
        docs = torch.cumsum(reset * valid, dim=1)

        def branch(w, conv, width):
            return dk.causal_conv(F.linear(x, w), conv, valid, docs, activation="silu").view(
                B, T, H, width)

        raw_q = branch(self.q, self.q_conv, K)
        raw_k = branch(self.k, self.k_conv, K)
        q = dk.l2_norm(raw_q)
        k = dk.l2_norm(raw_k)
        v = branch(self.v, self.v_conv, V)
        alpha = dk.decay(F.linear(x, self.decay).view(B, T, H, K), self.decay_bias,
                         self.decay_scale)
        erase = torch.sigmoid(F.linear(x, self.erase)).view(B, T, H, K)
        write = torch.sigmoid(F.linear(x, self.write)).view(B, T, H, V)
        scan = dk.gdn_training_scan(q, k, v, alpha, erase, write, valid, reset, None,
                                    cfg.chunk_size)
        out = scan.output
        if cfg.cache_policy != "none":
            exact = dk.hola_read(dk.rms_norm(raw_q, self.cache_q_norm, None, cfg.norm_epsilon),
                                 dk.rms_norm(raw_k, self.cache_k_norm, None, cfg.norm_epsilon),
                                 v, scan.scores, valid, docs, self.cache_sink,
                                 cfg.cache_capacity, cfg.chunk_size,
                                 cfg.cache_policy == "recency").output
            out = out + exact * torch.sigmoid(self.cache_gate).view(1, 1, H, 1)
        gate = F.linear(x, self.output_gate).view(B, T, H, V)
        mixed = dk.rms_norm(out, self.norm_weight, gate, cfg.norm_epsilon).reshape(B, T, H * V)
        return F.linear(mixed, self.output) * valid[..., None]
