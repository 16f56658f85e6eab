"""Training-step operators on the HIP library (include/gdn2.h).

  cross_entropy_rows(x, target)        crates/kernels/src/cross_entropy_ops.rs:108-117
  adamw_update(x, g, m, v, time, ...)  crates/kernels/src/update_ops.rs:90-117
  FusedAdamW                           crates/experiment/src/update.rs:43-96 (its
                                       optimizer), one launch pair per parameter set
  linear_cross_entropy(h, w, target)   the tied-head loss of a training step: the
                                       logits are computed once (torch GEMM), then
                                       one kernel turns them into the mean loss and
                                       their own gradient, in place
All run only on the GPU: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from ._lib import Gdn2AdamwTensor, check, lib, on_device

__all__ = ["cross_entropy_rows", "linear_cross_entropy", "adamw_update", "FusedAdamW"]


def _helpers():
    from . import _ptr, _stream, _view
    return _view, _ptr, _stream


def _targets(target: torch.Tensor, rows: int, device) -> torch.Tensor:
    if target.dtype != torch.int64:
        raise TypeError("target must hold int64 class ids")
    if target.dim() != 1 or target.shape[0] != rows:
        raise ValueError(f"target must be [{rows}]")
    if target.device != device:
        raise ValueError("target must live on the logits' device")
    return target


# ---- cross entropy -----------------------------------------------------------------


class _CrossEntropyRows(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, target):
        _view, _ptr, _stream = _helpers()
        rows, width = x.shape
        loss = torch.empty((rows,), dtype=torch.float32, device=x.device)
        stats = torch.empty((rows, 2), dtype=torch.float32, device=x.device)
        with on_device(x.device):
            rc = lib().gdn2_cross_entropy_forward(rows, width, ctypes.byref(_view(x)), _ptr(target),
                                                  target.stride(0), _ptr(loss), _ptr(stats),
                                                  _stream(x))
        check("gdn2_cross_entropy_forward", rc)
        ctx.save_for_backward(x, target, stats)
        return loss

    @staticmethod
    def backward(ctx, d_loss):
        _view, _ptr, _stream = _helpers()
        x, target, stats = ctx.saved_tensors
        rows, width = x.shape
        up = d_loss.float()
        dx = torch.empty((rows, width), dtype=x.dtype, device=x.device)
        with on_device(x.device):
            rc = lib().gdn2_cross_entropy_backward(rows, width, ctypes.byref(_view(x)),
                                                   _ptr(target), target.stride(0), _ptr(stats),
                                                   _ptr(up), up.stride(0), _ptr(dx), _stream(x))
        check("gdn2_cross_entropy_backward", rc)
        return dx, None


def cross_entropy_rows(x: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """Per-row negative log probability of target under softmax(x): x [rows,
    width] float32 or bfloat16, target [rows] int64.  Returns [rows] float32,
    differentiable in x (gradient in x's dtype)."""
    if x.dim() != 2 or x.dtype not in (torch.float32, torch.bfloat16) or not x.is_cuda:
        raise ValueError("x must be a [rows, width] float32/bfloat16 GPU tensor")
    return _CrossEntropyRows.apply(x, _targets(target, x.shape[0], x.device))


class _LinearCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, w, target):
        _view, _ptr, _stream = _helpers()
        rows = h.shape[0]
        width = w.shape[0]
        logits = torch.mm(h, w.t())
        loss = torch.empty((rows,), dtype=torch.float32, device=h.device)
        with on_device(h.device):
            rc = lib().gdn2_cross_entropy_fused(rows, width, ctypes.byref(_view(logits)),
                                                _ptr(target), target.stride(0),
                                                ctypes.c_float(1.0 / rows), _ptr(loss),
                                                _ptr(logits), _stream(h))
        check("gdn2_cross_entropy_fused", rc)
        ctx.save_for_backward(h, w)
        ctx.dlogits = logits  # now d(mean loss)/d(logits)
        return loss.mean()

    @staticmethod
    def backward(ctx, g):
        h, w = ctx.saved_tensors
        dl = ctx.dlogits
        ctx.dlogits = None
        dh = torch.mm(dl, w).mul_(g) if ctx.needs_input_grad[0] else None
        dw = torch.mm(dl.t(), h).mul_(g) if ctx.needs_input_grad[1] else None
        return dh, dw, None


def linear_cross_entropy(h: torch.Tensor, w: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """Mean over rows of cross_entropy_rows(h @ w^T, target), for h [rows, d]
    and w [width, d] of one dtype (float32 or bfloat16).  The logits buffer is
    overwritten by its gradient in the forward pass; the backward scales the
    two GEMM results by the upstream gradient."""
    if h.dim() != 2 or w.dim() != 2 or h.shape[1] != w.shape[1] or h.dtype != w.dtype:
        raise ValueError("h must be [rows, d] and w [width, d] of one dtype")
    if h.dtype not in (torch.float32, torch.bfloat16) or not h.is_cuda:
        raise ValueError("h and w must be float32/bfloat16 GPU tensors")
    return _LinearCrossEntropy.apply(h, w, _targets(target, h.shape[0], h.device))


# ---- AdamW ---------------------------------------------------------------------------


def _adamw_call(entries, initialized, time, lr, weight_decay, clip, workspace, reuse, stream,
                device):
    n = len(entries)
    arr = (Gdn2AdamwTensor * max(n, 1))(*entries)
    nbytes = lib().gdn2_adamw_workspace_bytes(n, arr)
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=device)
        reuse = False
    with on_device(device):
        rc = lib().gdn2_adamw_update(n, arr, 1 if initialized else 0, time, float(lr),
                                     float(weight_decay), float(clip), 1 if reuse else 0,
                                     ctypes.c_void_p(workspace.data_ptr()), workspace.numel(),
                                     stream)
    check("gdn2_adamw_update", rc)
    return workspace


def _f32_contig(t: torch.Tensor, name: str):
    if t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
        raise ValueError(f"{name} must be a contiguous float32 GPU tensor")


def adamw_update(x: torch.Tensor, g: torch.Tensor, m: Optional[torch.Tensor],
                 v: Optional[torch.Tensor], time: int, lr: float, decay: float, clip: float):
    """One AdamW step of one parameter tensor with its own clipping norm
    (crates/kernels/src/update_ops.rs:90-117).  m and v are both None on the
    first step.  x is updated in place; returns (x, m, v)."""
    if (m is None) != (v is None):
        raise ValueError("m and v must both be given or both be None")
    initialized = m is not None
    if m is None:
        m = torch.empty_like(x)
        v = torch.empty_like(x)
    for t, n in ((x, "x"), (g, "g"), (m, "m"), (v, "v")):
        _f32_contig(t, n)
        if t.shape != x.shape:
            raise ValueError(f"{n} must match x's shape")
    _view, _ptr, _stream = _helpers()
    e = Gdn2AdamwTensor(x.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), x.numel())
    _adamw_call([e], initialized, time, lr, decay, clip, None, False, _stream(x), x.device)
    return x, m, v


class FusedAdamW(torch.optim.Optimizer):
    """AdamW with per-parameter gradient-norm clipping, the reference's
    training optimizer (crates/experiment/src/update.rs:43-96 with Burn 0.22's
    AdamW constants: betas 0.9 / 0.999, epsilon 1e-5 outside the square root;
    crates/experiment/src/config.rs:442-444 defaults lr 1e-3, weight decay 0.01,
    clip 1.0).  One gdn2_adamw_update call per parameter group updates every
    parameter that has a gradient; parameters must be contiguous float32."""

    def __init__(self, params, lr: float = 1e-3, weight_decay: float = 0.01, clip: float = 1.0):
        super().__init__(params, dict(lr=lr, weight_decay=weight_decay, clip=clip))
        self._ws = {}

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        _view, _ptr, _stream = _helpers()
        for gi, group in enumerate(self.param_groups):
            batches = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                _f32_contig(p, "parameter")
                _f32_contig(p.grad, "gradient")
                st = self.state[p]
                if not st:
                    st["step"] = 0
                    st["first"] = torch.empty_like(p)
                    st["second"] = torch.empty_like(p)
                st["step"] += 1
                batches.setdefault(st["step"], []).append(p)
            for time, ps in sorted(batches.items()):
                entries = [Gdn2AdamwTensor(p.data_ptr(), p.grad.data_ptr(),
                                           self.state[p]["first"].data_ptr(),
                                           self.state[p]["second"].data_ptr(), p.numel())
                           for p in ps]
                key = (gi, time > 1)
                sig = tuple((e.param, e.grad, e.first, e.second, e.numel) for e in entries)
                ws, prev = self._ws.get(key, (None, None))
                ws = _adamw_call(entries, time > 1, time, group["lr"], group["weight_decay"],
                                 group["clip"], ws, prev == sig, _stream(ps[0]), ps[0].device)
                self._ws[key] = (ws, sig)
        return loss
