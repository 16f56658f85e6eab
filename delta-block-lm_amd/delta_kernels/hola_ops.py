"""HOLA exact-memory cache read on the HIP library (include/gdn2.h).

Mirrors the reference's ops (crates/kernels/src/hola_ops.rs):
  hola_schedule(scores, valid, documents, capacity, chunk, recency)   :358-385
  hola_read(q, k, v, scores, valid, documents, sink, capacity, chunk,
            recency, return_final_positions)                           :387-425
float32 only, as the reference's; q, k, v and sink receive gradients, the
scores choose cache membership only.  GPU only: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from ._lib import Gdn2HolaShape, check, lib, on_device

__all__ = ["HolaReadOutput", "hola_schedule", "hola_read"]


class HolaReadOutput(NamedTuple):
    """crates/kernels/src/hola_ops.rs (HolaReadOutput)."""
    output: torch.Tensor                      # [B, T, H, V] f32
    final_positions: Optional[torch.Tensor]   # [B, H, capacity] f32, -1 = empty


def _helpers():
    from . import _ptr, _stream, _view
    return _view, _ptr, _stream


def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float32 or not t.is_cuda:
        raise ValueError(f"{name} must be a float32 GPU tensor (the reference's HOLA is f32)")
    return t


def _scores3(scores: torch.Tensor) -> torch.Tensor:
    return scores[..., 0] if scores.dim() == 4 else scores


def _shape(B, T, H, K, V, capacity, chunk):
    return Gdn2HolaShape(B, T, H, K, V, capacity, chunk)


def hola_schedule(scores, valid, documents, capacity: int, chunk: int,
                  recency: bool = False) -> torch.Tensor:
    """Cache positions before the first chunk and after each chunk:
    [B, H, ceil(T / chunk) + 1, capacity] float32 (-1 = empty)."""
    _view, _ptr, _stream = _helpers()
    sc = _scores3(_f32(scores, "scores"))
    B, T, H = sc.shape
    for t, n in ((valid, "valid"), (documents, "documents")):
        _f32(t, n)
        if tuple(t.shape) != (B, T):
            raise ValueError(f"{n} must be [batch, time]")
    nc = -(-T // chunk)
    out = torch.empty((B, H, nc + 1, capacity), dtype=torch.float32, device=sc.device)
    shape = _shape(B, T, H, 1, 1, capacity, chunk)
    with on_device(sc.device):
        rc = lib().gdn2_hola_schedule(ctypes.byref(shape), 1 if recency else 0,
                                      ctypes.byref(_view(sc)), ctypes.byref(_view(valid)),
                                      ctypes.byref(_view(documents)), _ptr(out), _stream(sc))
    check("gdn2_hola_schedule", rc)
    return out


class _HolaRead(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, sink, scores, valid, documents, capacity, chunk, recency):
        _view, _ptr, _stream = _helpers()
        B, T, H, K = q.shape
        V = v.shape[3]
        shape = _shape(B, T, H, K, V, capacity, chunk)
        L = lib()
        out = torch.empty((B, T, H, V), dtype=torch.float32, device=q.device)
        fin = torch.empty((B, H, capacity), dtype=torch.float32, device=q.device)
        nck = L.gdn2_hola_checkpoint_bytes(ctypes.byref(shape))
        if nck == 0:
            check("gdn2_hola_checkpoint_bytes", 1)
        ck = torch.empty((nck,), dtype=torch.uint8, device=q.device)
        views = [_view(x) for x in (q, k, v, scores, valid, documents, sink)]
        with on_device(q.device):
            rc = L.gdn2_hola_read(ctypes.byref(shape), 1 if recency else 0,
                                  *[ctypes.byref(x) for x in views], _ptr(out), _ptr(fin),
                                  _ptr(ck), nck, _stream(q))
        check("gdn2_hola_read", rc)
        ctx.save_for_backward(q, k, v, sink, valid, documents, out)
        ctx.checkpoint = ck
        ctx.shape = (B, T, H, K, V, capacity, chunk)
        ctx.mark_non_differentiable(fin)
        return out, fin

    @staticmethod
    def backward(ctx, d_out, _d_fin):
        _view, _ptr, _stream = _helpers()
        q, k, v, sink, valid, documents, out = ctx.saved_tensors
        shape = _shape(*ctx.shape)
        L = lib()
        dq = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        dk = torch.empty(k.shape, dtype=torch.float32, device=q.device)
        dv = torch.empty(v.shape, dtype=torch.float32, device=q.device)
        ds = torch.empty((q.shape[2],), dtype=torch.float32, device=q.device)
        nws = L.gdn2_hola_workspace_bytes(ctypes.byref(shape))
        ws = torch.empty((nws,), dtype=torch.uint8, device=q.device)
        d_out = d_out.float() if d_out is not None else None  # held until the launch
        dov = _view(d_out)
        views = [_view(x) for x in (q, k, v, valid, documents, sink)]
        with on_device(q.device):
            rc = L.gdn2_hola_backward(ctypes.byref(shape), *[ctypes.byref(x) for x in views],
                                      _ptr(ctx.checkpoint), ctx.checkpoint.numel(), _ptr(out),
                                      ctypes.byref(dov) if d_out is not None else None,
                                      _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ds), _ptr(ws), nws,
                                      _stream(q))
        check("gdn2_hola_backward", rc)
        return dq, dk, dv, ds, None, None, None, None, None, None


def hola_read(q, k, v, scores, valid, documents, sink, capacity: int, chunk: int,
              recency: bool = False, return_final_positions: bool = False) -> HolaReadOutput:
    """Attention of every valid query over the score-selected cache of earlier
    chunks plus its own chunk's causal tokens, within its document, with a
    zero-value sink logit per head.  q, k [B,T,H,K], v [B,T,H,V], scores
    [B,T,H(,1)], valid/documents [B,T], sink [H]; all float32."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (scores, "scores"), (valid, "valid"),
                 (documents, "documents"), (sink, "sink")):
        _f32(t, n)
    if q.dim() != 4 or k.shape != q.shape or v.shape[:3] != q.shape[:3]:
        raise ValueError("q, k must be [B,T,H,K] and v [B,T,H,V]")
    B, T, H, _ = q.shape
    sc = _scores3(scores)
    if tuple(sc.shape) != (B, T, H) or tuple(valid.shape) != (B, T) or \
            tuple(documents.shape) != (B, T) or tuple(sink.shape) != (H,):
        raise ValueError("scores [B,T,H], valid/documents [B,T] and sink [H] required")
    out, fin = _HolaRead.apply(q, k, v, sink, sc.detach(), valid, documents, capacity, chunk,
                               bool(recency))
    return HolaReadOutput(out, fin if return_final_positions else None)
