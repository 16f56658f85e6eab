"""Fused operators of the lm512 training step on the HIP library (include/gdn2.h,
"Fused operators of the lm512 training step").

They have no counterpart in the reference, whose model composes the f32
custom ops one by one (crates/mixers/src/lib.rs:456-525; block
crates/experiment/src/model.rs:300-364).  Each call here is one forward or one
VJP without autograd: delta_mixers.model's fused block calls them from its own
backward.  bf16 tensors are torch.bfloat16; all tensors live on the GPU and
must be contiguous.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from ._lib import Gdn2LmMixerShape, check, lib, on_device, raw_stream

__all__ = ["norm_forward", "norm_backward", "mixer_in_forward", "mixer_in_backward",
           "mixer_out_forward", "mixer_out_backward", "swiglu_forward", "swiglu_backward"]

BF16 = torch.bfloat16
F32 = torch.float32


def _stream(t: torch.Tensor):
    return raw_stream(t.device)


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t: torch.Tensor, name: str, dtype, shape=None):
    if not t.is_cuda:
        raise ValueError(f"{name} must live on the GPU; there is no CPU fallback")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)} (got {tuple(t.shape)})")
    return t


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=device)


# ---- RMSNorm with residual ------------------------------------------------------------


def norm_forward(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor,
                 eps: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """x f32 [rows, W], residual bf16 [rows, W] or None, weight f32 [W] ->
    (u = x + residual (x itself when residual is None), y bf16, inverse f32 [rows])."""
    rows, W = x.shape
    _need(x, "x", F32)
    _need(weight, "weight", F32, (W,))
    u = x
    if residual is not None:
        _need(residual, "residual", BF16, (rows, W))
        u = torch.empty_like(x)
    y = torch.empty((rows, W), dtype=BF16, device=x.device)
    inv = torch.empty((rows,), dtype=F32, device=x.device)
    with on_device(x.device):
        rc = lib().gdn2_lm_norm_forward(rows, W, ctypes.c_float(eps), _p(x), _p(residual),
                                        _p(weight), _p(u) if residual is not None else None,
                                        _p(y), _p(inv), _stream(x))
    check("gdn2_lm_norm_forward", rc)
    return u, y, inv


def norm_backward(x: torch.Tensor, weight: torch.Tensor, inv: torch.Tensor, dy: torch.Tensor,
                  dres: Optional[torch.Tensor], want_bf16: bool):
    """VJP of norm_forward at its input u (= x here): dx = dres + J^T dy.
    Returns (dx f32, dx bf16 or None, dweight f32 [W])."""
    rows, W = x.shape
    _need(x, "x", F32)
    _need(weight, "weight", F32, (W,))
    _need(inv, "inverse", F32, (rows,))
    _need(dy, "dy", BF16, (rows, W))
    if dres is not None:
        _need(dres, "dres", F32, (rows, W))
    dx = torch.empty_like(x)
    dxb = torch.empty((rows, W), dtype=BF16, device=x.device) if want_bf16 else None
    dw = torch.empty((W,), dtype=F32, device=x.device)
    L = lib()
    nws = L.gdn2_lm_norm_workspace_bytes(rows, W)
    ws = _ws(nws, x.device)
    with on_device(x.device):
        rc = L.gdn2_lm_norm_backward(rows, W, _p(x), _p(weight), _p(inv), _p(dy), _p(dres),
                                     _p(dx), _p(dxb), _p(dw), _p(ws), ws.numel(), _stream(x))
    check("gdn2_lm_norm_backward", rc)
    return dx, dxb, dw


# ---- GDN mixer around the scan ----------------------------------------------------------


def _mixer_shape(z: torch.Tensor, B: int, T: int, H: int, taps: int) -> Gdn2LmMixerShape:
    _need(z, "z", BF16)
    if z.dim() != 2 or z.shape[0] != B * T:
        raise ValueError("z must be [batch * time, z_stride]")
    return Gdn2LmMixerShape(B, T, H, 64, 64, taps, z.shape[1])


def mixer_in_forward(z, conv_w, valid, docs, decay_scale, decay_bias, B: int, T: int, H: int):
    """z bf16 [B T, Z] -> (qkv bf16 [B, T, 3 H, 64], beta f32 [B, T, H], g f32 [B, T, H])."""
    taps = conv_w.shape[0]
    shape = _mixer_shape(z, B, T, H, taps)
    _need(conv_w, "conv_w", F32, (taps, 3 * H * 64))
    _need(valid, "valid", F32, (B, T))
    _need(docs, "docs", F32, (B, T))
    _need(decay_scale, "decay_scale", F32, (H,))
    _need(decay_bias, "decay_bias", F32, (H,))
    qkv = torch.empty((B, T, 3 * H, 64), dtype=BF16, device=z.device)
    beta = torch.empty((B, T, H), dtype=F32, device=z.device)
    g = torch.empty((B, T, H), dtype=F32, device=z.device)
    with on_device(z.device):
        rc = lib().gdn2_lm_mixer_in_forward(ctypes.byref(shape), _p(z), _p(conv_w), _p(valid),
                                            _p(docs), _p(decay_scale), _p(decay_bias), _p(qkv),
                                            _p(beta), _p(g), _stream(z))
    check("gdn2_lm_mixer_in_forward", rc)
    return qkv, beta, g


def mixer_in_backward(z, conv_w, valid, docs, decay_scale, decay_bias, dq, dk, dv, dbeta, dg,
                      dz, B: int, T: int, H: int):
    """Writes the q, k, v, beta and decay columns of dz (bf16, z's layout);
    returns (dconv_w, ddecay_scale, ddecay_bias)."""
    taps = conv_w.shape[0]
    shape = _mixer_shape(z, B, T, H, taps)
    for t, n in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        _need(t, n, BF16, (B, T, H, 64))
    _need(dbeta, "dbeta", F32, (B, T, H))
    _need(dg, "dg", F32, (B, T, H))
    _need(dz, "dz", BF16, tuple(z.shape))
    dconv = torch.empty_like(conv_w)
    dds = torch.empty((H,), dtype=F32, device=z.device)
    ddb = torch.empty((H,), dtype=F32, device=z.device)
    L = lib()
    nws = L.gdn2_lm_mixer_in_workspace_bytes(ctypes.byref(shape))
    ws = _ws(nws, z.device)
    with on_device(z.device):
        rc = L.gdn2_lm_mixer_in_backward(ctypes.byref(shape), _p(z), _p(conv_w), _p(valid),
                                         _p(docs), _p(decay_scale), _p(decay_bias), _p(dq), _p(dk),
                                         _p(dv), _p(dbeta), _p(dg), _p(dz), _p(dconv), _p(dds),
                                         _p(ddb), _p(ws), ws.numel(), _stream(z))
    check("gdn2_lm_mixer_in_backward", rc)
    return dconv, dds, ddb


def mixer_out_forward(o, z, norm_w, eps: float, B: int, T: int, H: int):
    """o bf16 [B, T, H, 64] -> (y bf16 [B T, H 64], inverse f32 [B T H])."""
    shape = _mixer_shape(z, B, T, H, 1)
    _need(o, "o", BF16, (B, T, H, 64))
    _need(norm_w, "norm_w", F32, (64,))
    y = torch.empty((B * T, H * 64), dtype=BF16, device=z.device)
    inv = torch.empty((B * T * H,), dtype=F32, device=z.device)
    with on_device(z.device):
        rc = lib().gdn2_lm_mixer_out_forward(ctypes.byref(shape), _p(o), _p(z), _p(norm_w),
                                             ctypes.c_float(eps), _p(y), _p(inv), _stream(z))
    check("gdn2_lm_mixer_out_forward", rc)
    return y, inv


def mixer_out_backward(o, z, norm_w, inv, dy, dz, B: int, T: int, H: int):
    """Writes the gate columns of dz; returns (d_o bf16 [B, T, H, 64], dnorm_w)."""
    shape = _mixer_shape(z, B, T, H, 1)
    _need(o, "o", BF16, (B, T, H, 64))
    _need(norm_w, "norm_w", F32, (64,))
    _need(inv, "inverse", F32, (B * T * H,))
    _need(dy, "dy", BF16, (B * T, H * 64))
    _need(dz, "dz", BF16, tuple(z.shape))
    d_o = torch.empty_like(o)
    dw = torch.empty((64,), dtype=F32, device=z.device)
    L = lib()
    nws = L.gdn2_lm_mixer_out_workspace_bytes(ctypes.byref(shape))
    ws = _ws(nws, z.device)
    with on_device(z.device):
        rc = L.gdn2_lm_mixer_out_backward(ctypes.byref(shape), _p(o), _p(z), _p(norm_w), _p(inv),
                                          _p(dy), _p(d_o), _p(dz), _p(dw), _p(ws), ws.numel(),
                                          _stream(z))
    check("gdn2_lm_mixer_out_backward", rc)
    return d_o, dw


# ---- SwiGLU ---------------------------------------------------------------------------------


def swiglu_forward(h: torch.Tensor) -> torch.Tensor:
    """h bf16 [rows, 2 M] = [gate | up] -> bf16(bf16(silu(gate)) * up) [rows, M]."""
    _need(h, "h", BF16)
    rows, M2 = h.shape
    a = torch.empty((rows, M2 // 2), dtype=BF16, device=h.device)
    with on_device(h.device):
        rc = lib().gdn2_lm_swiglu_forward(rows, M2 // 2, _p(h), _p(a), _stream(h))
    check("gdn2_lm_swiglu_forward", rc)
    return a


def swiglu_backward(h: torch.Tensor, da: torch.Tensor) -> torch.Tensor:
    _need(h, "h", BF16)
    rows, M2 = h.shape
    _need(da, "da", BF16, (rows, M2 // 2))
    dh = torch.empty_like(h)
    with on_device(h.device):
        rc = lib().gdn2_lm_swiglu_backward(rows, M2 // 2, _p(h), _p(da), _p(dh), _stream(h))
    check("gdn2_lm_swiglu_backward", rc)
    return dh
