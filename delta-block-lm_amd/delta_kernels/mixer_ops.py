"""Mixer prologue/epilogue operators on the HIP library (include/gdn2.h).

Mirrors the reference's custom ops, with the same names and argument order:
  causal_conv(x, w, valid, documents)   crates/kernels/src/conv_ops.rs:119-136
  l2_norm(x)                            crates/kernels/src/norm_ops.rs:148-153
  rms_norm(x, weight, gate, epsilon)    crates/kernels/src/norm_ops.rs:154-174
  decay(x, bias, scale)                 crates/kernels/src/decay_ops.rs:123
All are float32, differentiable in their tensor inputs (masks and document ids
are metadata without a gradient), and run only on the GPU: there is no CPU
fallback.  causal_conv(..., activation="silu") fuses the SiLU the mixer
applies right after the convolution (crates/mixers/src/lib.rs:463-466).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from ._lib import Gdn2ConvShape, Gdn2RowsShape, check, lib, on_device

__all__ = ["causal_conv", "l2_norm", "rms_norm", "decay"]


def _helpers():
    from . import _ptr, _stream, _view  # the package's view/pointer/stream adapters
    return _view, _ptr, _stream


def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 (the reference's operators are f32 only)")
    if not t.is_cuda:
        raise ValueError(f"{name} must live on the GPU; there is no CPU fallback")
    return t


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty((max(nbytes, 4),), dtype=torch.uint8, device=device)


# ---- causal convolution --------------------------------------------------------


class _CausalConv(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, valid, docs, act):
        _view, _ptr, _stream = _helpers()
        B, T, C = x.shape
        shape = Gdn2ConvShape(B, T, C, w.shape[0])
        y = torch.empty((B, T, C), dtype=torch.float32, device=x.device)
        views = [_view(t) for t in (x, w, valid, docs)]
        with on_device(x.device):
            rc = lib().gdn2_conv_forward(ctypes.byref(shape), *[ctypes.byref(v) for v in views],
                                         act, _ptr(y), _stream(x))
        check("gdn2_conv_forward", rc)
        ctx.save_for_backward(x, w, valid, docs)
        ctx.act = act
        return y

    @staticmethod
    def backward(ctx, dy):
        _view, _ptr, _stream = _helpers()
        x, w, valid, docs = ctx.saved_tensors
        B, T, C = x.shape
        shape = Gdn2ConvShape(B, T, C, w.shape[0])
        L = lib()
        dy = dy.float()
        dx = torch.empty((B, T, C), dtype=torch.float32, device=x.device) \
            if ctx.needs_input_grad[0] else None
        dw = torch.empty(tuple(w.shape), dtype=torch.float32, device=x.device) \
            if ctx.needs_input_grad[1] else None
        nws = L.gdn2_conv_workspace_bytes(ctypes.byref(shape))
        ws = _workspace(nws, x.device)
        views = [_view(t) for t in (x, w, valid, docs, dy)]
        with on_device(x.device):
            rc = L.gdn2_conv_backward(ctypes.byref(shape), *[ctypes.byref(v) for v in views[:4]],
                                      ctx.act, ctypes.byref(views[4]), _ptr(dx), _ptr(dw),
                                      _ptr(ws), nws, _stream(x))
        check("gdn2_conv_backward", rc)
        return dx, dw, None, None, None


def causal_conv(x: torch.Tensor, w: torch.Tensor, valid: torch.Tensor, documents: torch.Tensor,
                activation: Optional[str] = None) -> torch.Tensor:
    """Depthwise causal convolution of x [B, T, C] with w [taps, C]; a lag never
    crosses a document boundary or touches an invalid token."""
    for t, n in ((x, "x"), (w, "w"), (valid, "valid"), (documents, "documents")):
        _f32(t, n)
    if x.dim() != 3 or w.dim() != 2 or w.shape[1] != x.shape[2]:
        raise ValueError("x must be [B, T, C] and w [taps, C]")
    if tuple(valid.shape) != tuple(x.shape[:2]) or tuple(documents.shape) != tuple(x.shape[:2]):
        raise ValueError("valid and documents must be [B, T]")
    if valid.requires_grad or documents.requires_grad:
        raise ValueError("convolution masks are nondifferentiable metadata")
    act = {None: 0, "silu": 1}[activation]
    return _CausalConv.apply(x, w, valid, documents, act)


# ---- row normalization -----------------------------------------------------------


def _rows4(x: torch.Tensor) -> torch.Tensor:
    while x.dim() < 4:
        x = x.unsqueeze(0)
    return x


class _RowNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x4, weight, gate4, mode, eps):
        _view, _ptr, _stream = _helpers()
        B, T, H, W = x4.shape
        shape = Gdn2RowsShape(B, T, H, W)
        y = torch.empty((B, T, H, W), dtype=torch.float32, device=x4.device)
        inv = torch.empty((B * T * H,), dtype=torch.float32, device=x4.device)
        vx, vw, vg = _view(x4), _view(weight), _view(gate4)
        with on_device(x4.device):
            rc = lib().gdn2_norm_forward(ctypes.byref(shape), mode, ctypes.c_float(eps),
                                         ctypes.byref(vx), ctypes.byref(vw), ctypes.byref(vg),
                                         _ptr(y), _ptr(inv), _stream(x4))
        check("gdn2_norm_forward", rc)
        ctx.save_for_backward(x4, weight, gate4, inv)
        ctx.mode = mode
        return y

    @staticmethod
    def backward(ctx, dy):
        _view, _ptr, _stream = _helpers()
        x4, weight, gate4, inv = ctx.saved_tensors
        mode = ctx.mode
        B, T, H, W = x4.shape
        shape = Gdn2RowsShape(B, T, H, W)
        L = lib()
        dy = dy.float()
        dx = torch.empty((B, T, H, W), dtype=torch.float32, device=x4.device) \
            if ctx.needs_input_grad[0] else None
        dw = torch.empty((W,), dtype=torch.float32, device=x4.device) \
            if mode >= 1 and ctx.needs_input_grad[1] else None
        dg = torch.empty((B, T, H, W), dtype=torch.float32, device=x4.device) \
            if mode == 2 and ctx.needs_input_grad[2] else None
        nws = L.gdn2_norm_workspace_bytes(ctypes.byref(shape))
        ws = _workspace(nws, x4.device)
        vx, vw, vg, vd = _view(x4), _view(weight), _view(gate4), _view(dy)
        with on_device(x4.device):
            rc = L.gdn2_norm_backward(ctypes.byref(shape), mode, ctypes.byref(vx),
                                      ctypes.byref(vw), ctypes.byref(vg), _ptr(inv),
                                      ctypes.byref(vd), _ptr(dx), _ptr(dg), _ptr(dw), _ptr(ws),
                                      nws, _stream(x4))
        check("gdn2_norm_backward", rc)
        return dx, dw, dg, None, None


def l2_norm(x: torch.Tensor) -> torch.Tensor:
    """x / sqrt(sum(x^2) + 1e-6) over the last axis of a [B, T, H, W] tensor."""
    _f32(x, "x")
    if x.dim() != 4:
        raise ValueError("l2_norm expects [B, T, H, W]")
    return _RowNorm.apply(x, x, x, 0, 1e-6)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, gate: Optional[torch.Tensor] = None,
             epsilon: float = 1e-6) -> torch.Tensor:
    """Learned RMSNorm over the last axis (optionally of x * sigmoid(gate)),
    for tensors of 1 to 4 dimensions."""
    _f32(x, "x")
    _f32(weight, "weight")
    if not 1 <= x.dim() <= 4 or weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError("rms_norm expects x [..., W] (at most 4-D) and weight [W]")
    if gate is not None:
        _f32(gate, "gate")
        if gate.shape != x.shape:
            raise ValueError("gate must match x")
    dims = x.shape
    x4 = _rows4(x)
    g4 = _rows4(gate) if gate is not None else x4
    y = _RowNorm.apply(x4, weight, g4, 2 if gate is not None else 1, float(epsilon))
    return y.reshape(dims)


# ---- decay -----------------------------------------------------------------------


class _Decay(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, bias, scale):
        _view, _ptr, _stream = _helpers()
        B, T, H, W = x.shape
        shape = Gdn2RowsShape(B, T, H, W)
        y = torch.empty((B, T, H, W), dtype=torch.float32, device=x.device)
        vx, vb, vs = _view(x), _view(bias), _view(scale)
        with on_device(x.device):
            rc = lib().gdn2_decay_forward(ctypes.byref(shape), ctypes.byref(vx), ctypes.byref(vb),
                                          ctypes.byref(vs), _ptr(y), _stream(x))
        check("gdn2_decay_forward", rc)
        ctx.save_for_backward(x, bias, scale)
        return y

    @staticmethod
    def backward(ctx, dy):
        _view, _ptr, _stream = _helpers()
        x, bias, scale = ctx.saved_tensors
        B, T, H, W = x.shape
        shape = Gdn2RowsShape(B, T, H, W)
        L = lib()
        dy = dy.float()
        dx = torch.empty((B, T, H, W), dtype=torch.float32, device=x.device) \
            if ctx.needs_input_grad[0] else None
        db = torch.empty((H * W,), dtype=torch.float32, device=x.device)
        ds = torch.empty((H,), dtype=torch.float32, device=x.device)
        nws = L.gdn2_decay_workspace_bytes(ctypes.byref(shape))
        ws = _workspace(nws, x.device)
        vx, vb, vs, vd = _view(x), _view(bias), _view(scale), _view(dy)
        with on_device(x.device):
            rc = L.gdn2_decay_backward(ctypes.byref(shape), ctypes.byref(vx), ctypes.byref(vb),
                                       ctypes.byref(vs), ctypes.byref(vd), _ptr(dx), _ptr(db),
                                       _ptr(ds), _ptr(ws), nws, _stream(x))
        check("gdn2_decay_backward", rc)
        return dx, db, ds


def decay(x: torch.Tensor, bias: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """exp(-exp(scale[h]) * softplus(x + bias[h, k])) for x [B, T, H, K],
    bias [H * K], scale [H] (softplus is the identity above 20)."""
    for t, n in ((x, "x"), (bias, "bias"), (scale, "scale")):
        _f32(t, n)
    if x.dim() != 4:
        raise ValueError("decay expects x [B, T, H, K]")
    H, K = x.shape[2], x.shape[3]
    if tuple(bias.shape) != (H * K,) or tuple(scale.shape) != (H,):
        raise ValueError("bias must be [H * K] and scale [H]")
    return _Decay.apply(x, bias, scale)
