"""GDN-2 scan operators on MI355X, behind the reference's kernel-level surface.

Python mirror of delta-block-lm's `delta_kernels` GDN-2 training op
(crates/kernels/src/gdn_training_ops.rs:17-333): `gdn_training_scan` returns
`GdnTrainingOutput(output, final_state, scores)` and is differentiable in
q, k, v, alpha, erase, write and the initial state, with float 0/1 masks
`valid`/`reset` [batch, time] that carry no gradient.  The compute runs in
libgdn2_amd.so (hand-written HIP for gfx950) through its C ABI
(include/gdn2.h); PyTorch only supplies device memory and the stream.

Also exposed: the scalar-gate gated delta rule (`gdn_scalar_scan`, beta and
log-decay g per token and head) and a decode step on a carried state.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from ._lib import (GDN2_BF16, GDN2_F32, GDN2_I32, Gdn2Shape, Gdn2View, check, lib, on_device,
                   raw_stream)

__all__ = ["GdnTrainingOutput", "gdn_training_scan", "gdn_training_forward",
           "gdn_training_backward", "gdn2_scan", "gdn2_scan_forward", "gdn2_backward",
           "gdn_scalar_scan", "gdn_scalar_forward", "gdn_scalar_backward", "gdn_decode_step",
           "stage_timing", "stage_times", "lib"]


class GdnTrainingOutput(NamedTuple):
    """crates/kernels/src/gdn_training_ops.rs:275-282."""
    output: torch.Tensor        # [batch, time, head, value]
    final_state: torch.Tensor   # [batch, head, key, value] f32
    scores: torch.Tensor        # [batch, time, head, 1] f32: ||k|| * ||delta||


_CODES = {torch.float32: GDN2_F32, torch.bfloat16: GDN2_BF16, torch.int32: GDN2_I32}
_STRIDES = ctypes.c_int64 * 4


def _code(t: torch.Tensor) -> int:
    c = _CODES.get(t.dtype)
    if c is None:
        raise TypeError(f"GDN-2 tensors must be float32 or bfloat16, got {t.dtype}")
    return c


def _view(t: Optional[torch.Tensor]) -> Gdn2View:
    if t is None:
        return Gdn2View(None, GDN2_F32)
    if not t.is_cuda:
        raise ValueError("GDN-2 tensors must live on the GPU; there is no CPU fallback")
    st = t.stride()
    if len(st) < 4:
        st = st + (0,) * (4 - len(st))
    return Gdn2View(t.data_ptr(), _code(t), 0, _STRIDES(*st))


def _shape(q: torch.Tensor, v: torch.Tensor) -> Gdn2Shape:
    B, T, H, K = q.shape
    return Gdn2Shape(B, T, H, K, v.shape[3])


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return raw_stream(t.device)


_SIZES: dict = {}


def _size(query, shape: Gdn2Shape, *extra) -> int:
    """A checkpoint or workspace size query, remembered per shape (the sizes
    depend on nothing else)."""
    key = (query, shape.batch, shape.time, shape.heads, shape.keys, shape.values) + extra
    n = _SIZES.get(key)
    if n is None:
        n = getattr(lib(), query)(ctypes.byref(shape), *extra)
        if n:
            _SIZES[key] = n
    return n


def _rows_aligned(t: torch.Tensor) -> bool:
    """True when every token row of t is a 16-byte aligned run of unit-stride
    channels: the form in which the chunk kernels read sequence rows."""
    el = t.element_size()
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all((s * el) % 16 == 0 for s in t.stride()[:-1]))


def _mask(m: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    if m.dtype != torch.float32:
        m = m.to(torch.float32)
    return m


def _check_shapes(q, k, v, gates, valid, reset, initial):
    if q.dim() != 4:
        raise ValueError("q must be [batch, time, head, key]")
    B, T, H, K = q.shape
    V = v.shape[3]
    if k.shape != q.shape or v.shape[:3] != q.shape[:3]:
        raise ValueError("q, k, v must share [batch, time, head]")
    for name, g, w in gates:
        if tuple(g.shape) != (B, T, H) + ((w,) if w else ()):
            raise ValueError(f"{name} must have shape {(B, T, H) + ((w,) if w else ())}")
    if tuple(valid.shape) != (B, T) or tuple(reset.shape) != (B, T):
        raise ValueError("valid/reset must be [batch, time]")
    if initial is not None and tuple(initial.shape) != (B, H, K, V):
        raise ValueError("initial must be [batch, head, key, value]")
    devs = {t.device for t in (q, k, v, valid, reset) + tuple(g for _, g, _ in gates)}
    if initial is not None:
        devs.add(initial.device)
    if len(devs) != 1:
        raise ValueError("GDN-2 inputs must share a device")


# ---- channel-wise training scan ---------------------------------------------------


def gdn_training_forward(q, k, v, alpha, erase, write, valid, reset, initial, chunk):
    """Raw forward (crates/kernels/src/gdn_training_ops.rs:27-48).  Returns
    (output, final_state, scores, checkpoint); the checkpoint feeds
    gdn_training_backward."""
    return _training_forward(q, k, v, alpha, erase, write, valid, reset, initial, chunk)


def _training_forward(q, k, v, alpha, erase, write, valid, reset, initial, chunk):
    L = lib()
    shape = _shape(q, v)
    B, T, H, K = q.shape
    V = v.shape[3]
    dev = q.device
    out = torch.empty((B, T, H, V), dtype=q.dtype, device=dev)
    final = torch.empty((B, H, K, V), dtype=torch.float32, device=dev)
    scores = torch.empty((B, T, H, 1), dtype=torch.float32, device=dev)
    nck = _size("gdn2_training_checkpoint_bytes", shape, chunk)
    if nck == 0:
        check("gdn2_training_checkpoint_bytes", 1)
    ck = torch.empty((nck,), dtype=torch.uint8, device=dev)
    views = [_view(x) for x in (q, k, v, alpha, erase, write, valid, reset, initial)]
    with on_device(dev):
        rc = L.gdn2_training_scan(ctypes.byref(shape), chunk, *[ctypes.byref(x) for x in views],
                                  _ptr(out), _code(out), _ptr(final), _ptr(scores), _ptr(ck), nck,
                                  _stream(q))
    check("gdn2_training_scan", rc)
    return out, final, scores, ck


def gdn_training_backward(q, k, v, alpha, erase, write, valid, reset, checkpoint, chunk,
                          d_output=None, d_final_state=None, d_scores=None):
    """Raw VJP (crates/kernels/src/gdn_training_ops.rs:47-68).  Returns
    (dq, dk, dv, dalpha, derase, dwrite, d_initial)."""
    L = lib()
    shape = _shape(q, v)
    B, T, H, K = q.shape
    V = v.shape[3]
    dev = q.device
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    da = torch.empty((B, T, H, K), dtype=torch.float32, device=dev)
    de = torch.empty((B, T, H, K), dtype=torch.float32, device=dev)
    dw = torch.empty((B, T, H, V), dtype=torch.float32, device=dev)
    dinit = torch.empty((B, H, K, V), dtype=torch.float32, device=dev)
    nws = _size("gdn2_training_workspace_bytes", shape, chunk)
    ws = torch.empty((nws,), dtype=torch.uint8, device=dev)
    if d_output is not None:
        if d_output.dtype != q.dtype:
            d_output = d_output.to(q.dtype)
        if not _rows_aligned(d_output):
            # The chunk kernels read 16-byte row pieces of the upstream gradient.
            d_output = d_output.contiguous()
    dfin = None if d_final_state is None else d_final_state.to(torch.float32).contiguous()
    dsc = None if d_scores is None else d_scores.to(torch.float32).contiguous()
    views = [_view(x) for x in (q, k, v, alpha, erase, write, valid, reset)]
    dov = _view(d_output)
    with on_device(dev):
        rc = L.gdn2_training_backward(
            ctypes.byref(shape), chunk, *[ctypes.byref(x) for x in views], _ptr(checkpoint),
            checkpoint.numel(), ctypes.byref(dov) if d_output is not None else None, _ptr(dfin),
            _ptr(dsc), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(da), _ptr(de), _ptr(dw), _ptr(dinit),
            _ptr(ws), nws, _stream(q))
    check("gdn2_training_backward", rc)
    return dq, dk, dv, da, de, dw, dinit


class _TrainingScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, alpha, erase, write, valid, reset, initial, chunk):
        out, final, scores, ck = _training_forward(q, k, v, alpha, erase, write, valid, reset,
                                                   initial, chunk)
        # Unused outputs reach backward as None (not zero tensors), so the
        # kernels skip the work of adjoints that are absent.
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(q, k, v, alpha, erase, write, valid, reset)
        ctx.checkpoint = ck
        ctx.chunk = chunk
        ctx.has_initial = initial is not None
        return out, final, scores

    @staticmethod
    def backward(ctx, d_out, d_final, d_scores):
        q, k, v, alpha, erase, write, valid, reset = ctx.saved_tensors
        dq, dk, dv, da, de, dw, dinit = gdn_training_backward(
            q, k, v, alpha, erase, write, valid, reset, ctx.checkpoint, ctx.chunk, d_out,
            d_final, d_scores)
        return (dq, dk, dv, da, de, dw, None, None, dinit if ctx.has_initial else None, None)


def gdn_training_scan(q, k, v, alpha, erase, write, valid, reset, initial=None,
                      chunk_size: int = 16) -> GdnTrainingOutput:
    """Fused GDN-2 scan (crates/kernels/src/gdn_training_ops.rs:284-333).

    q, k: [B,T,H,K]; v: [B,T,H,V] (float32 or bfloat16, same dtype);
    alpha, erase: [B,T,H,K] and write: [B,T,H,V] float32 channel-wise gates;
    valid, reset: [B,T] float 0/1; initial: [B,H,K,V] float32 or None (zero).
    Padding freezes the state; a reset on a valid token discards it before
    the update.  Binary masks are nondifferentiable.  chunk_size (1..64) is
    the checkpoint interval; results do not depend on it."""
    _check_shapes(q, k, v, [("alpha", alpha, q.shape[3]), ("erase", erase, q.shape[3]),
                            ("write", write, v.shape[3])], valid, reset, initial)
    valid = _mask(valid, q)
    reset = _mask(reset, q)
    gates = [g if g.dtype == torch.float32 else g.float() for g in (alpha, erase, write)]
    if initial is not None and initial.dtype != torch.float32:
        initial = initial.float()
    out, final, scores = _TrainingScan.apply(q, k, v, *gates, valid, reset, initial, chunk_size)
    return GdnTrainingOutput(out, final, scores)


# ---- document-limit scan ----------------------------------------------------------


def _doc_limits(doc_start, doc_end, B, T, device):
    for name, t in (("doc_start", doc_start), ("doc_end", doc_end)):
        if t.dtype != torch.int32 or tuple(t.shape) != (B, T) or t.device != device:
            raise ValueError(f"{name} must be an int32 [batch, time] tensor on the inputs' device")


def gdn2_scan_forward(q, k, v, alpha, erase, write, doc_start, doc_end):
    """Raw forward of the document-limit scan (crates/kernels/src/ops.rs:19-31):
    returns (output, checkpoint)."""
    L = lib()
    shape = _shape(q, v)
    B, T, H, K = q.shape
    V = v.shape[3]
    out = torch.empty((B, T, H, V), dtype=q.dtype, device=q.device)
    nck = L.gdn2_scan_checkpoint_bytes(ctypes.byref(shape))
    if nck == 0:
        check("gdn2_scan_checkpoint_bytes", 1)
    ck = torch.empty((nck,), dtype=torch.uint8, device=q.device)
    views = [_view(x) for x in (q, k, v, alpha, erase, write, doc_start, doc_end)]
    with on_device(q.device):
        rc = L.gdn2_scan(ctypes.byref(shape), *[ctypes.byref(x) for x in views], _ptr(out),
                         _code(out), _ptr(ck), nck, _stream(q))
    check("gdn2_scan", rc)
    return out, ck


def gdn2_backward(q, k, v, alpha, erase, write, d_output, checkpoint, doc_start, doc_end):
    """Raw VJP of the document-limit scan (crates/kernels/src/ops.rs:33-55):
    returns (dq, dk, dv, dalpha, derase, dwrite)."""
    L = lib()
    shape = _shape(q, v)
    B, T, H, K = q.shape
    V = v.shape[3]
    dev = q.device
    dq = torch.empty((B, T, H, K), dtype=q.dtype, device=dev)
    dk = torch.empty((B, T, H, K), dtype=q.dtype, device=dev)
    dv = torch.empty((B, T, H, V), dtype=q.dtype, device=dev)
    da = torch.empty((B, T, H, K), dtype=torch.float32, device=dev)
    de = torch.empty((B, T, H, K), dtype=torch.float32, device=dev)
    dw = torch.empty((B, T, H, V), dtype=torch.float32, device=dev)
    nws = L.gdn2_scan_workspace_bytes(ctypes.byref(shape))
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=dev)
    if d_output is not None:
        if d_output.dtype != q.dtype:
            d_output = d_output.to(q.dtype)
        if not _rows_aligned(d_output):
            d_output = d_output.contiguous()
    views = [_view(x) for x in (q, k, v, alpha, erase, write, doc_start, doc_end)]
    dov = _view(d_output)
    with on_device(dev):
        rc = L.gdn2_backward(ctypes.byref(shape), *[ctypes.byref(x) for x in views],
                             _ptr(checkpoint), checkpoint.numel(),
                             ctypes.byref(dov) if d_output is not None else None, _ptr(dq),
                             _ptr(dk), _ptr(dv), _ptr(da), _ptr(de), _ptr(dw), _ptr(ws), nws,
                             _stream(q))
    check("gdn2_backward", rc)
    return dq, dk, dv, da, de, dw


class _DocScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, alpha, erase, write, doc_start, doc_end):
        out, ck = gdn2_scan_forward(q, k, v, alpha, erase, write, doc_start, doc_end)
        ctx.save_for_backward(q, k, v, alpha, erase, write, doc_start, doc_end)
        ctx.checkpoint = ck
        return out

    @staticmethod
    def backward(ctx, d_out):
        q, k, v, alpha, erase, write, doc_start, doc_end = ctx.saved_tensors
        grads = gdn2_backward(q, k, v, alpha, erase, write, d_out, ctx.checkpoint, doc_start,
                              doc_end)
        return grads + (None, None)


def gdn2_scan(q, k, v, alpha, erase, write, doc_start, doc_end):
    """Document-limit GDN-2 scan (crates/kernels/src/ops.rs:254-276): output
    [B,T,H,V] in q's dtype, differentiable in q, k, v, alpha, erase, write.
    doc_start/doc_end: int32 [B,T] inclusive limits; end < start marks padding
    and start == t resets the state.  The gates are taken in float32, as the
    reference casts them (ops.rs:264-267)."""
    B, T = q.shape[:2]
    _check_shapes(q, k, v, [("alpha", alpha, q.shape[3]), ("erase", erase, q.shape[3]),
                            ("write", write, v.shape[3])], doc_start, doc_end, None)
    _doc_limits(doc_start, doc_end, B, T, q.device)
    gates = [g if g.dtype == torch.float32 else g.float() for g in (alpha, erase, write)]
    return _DocScan.apply(q, k, v, *gates, doc_start, doc_end)


# ---- scalar-gate gated delta rule -------------------------------------------------


def gdn_scalar_forward(q, k, v, beta, g, valid, reset, initial=None, chunk: int = 64):
    """Raw forward of the scalar-gate scan.  Returns (output, final_state,
    scores, checkpoint); the checkpoint is private storage for the backward."""
    L = lib()
    shape = _shape(q, v)
    B, T, H, K = q.shape
    V = v.shape[3]
    dev = q.device
    out = torch.empty((B, T, H, V), dtype=q.dtype, device=dev)
    final = torch.empty((B, H, K, V), dtype=torch.float32, device=dev)
    scores = torch.empty((B, T, H), dtype=torch.float32, device=dev)
    nck = L.gdn_scalar_checkpoint_bytes(ctypes.byref(shape), chunk)
    if nck == 0:
        check("gdn_scalar_checkpoint_bytes", 1)
    ck = torch.empty((nck,), dtype=torch.uint8, device=dev)
    views = [_view(x) for x in (q, k, v, beta, g, valid, reset, initial)]
    with on_device(dev):
        rc = L.gdn_scalar_scan(ctypes.byref(shape), chunk, *[ctypes.byref(x) for x in views],
                               _ptr(out), _code(out), _ptr(final), _ptr(scores), _ptr(ck), nck,
                               _stream(q))
    check("gdn_scalar_scan", rc)
    return out, final, scores, ck


def gdn_scalar_backward(q, k, v, beta, g, valid, reset, checkpoint, chunk: int = 64,
                        d_output=None, d_final_state=None, d_scores=None):
    """Raw VJP of the scalar-gate scan.  Returns (dq, dk, dv, dbeta, dg, d_initial)."""
    L = lib()
    shape = _shape(q, v)
    B, T, H, K = q.shape
    V = v.shape[3]
    dev = q.device
    dq = torch.empty(q.shape, dtype=q.dtype, device=dev)
    dk = torch.empty(k.shape, dtype=k.dtype, device=dev)
    dv = torch.empty(v.shape, dtype=v.dtype, device=dev)
    db = torch.empty((B, T, H), dtype=torch.float32, device=dev)
    dg = torch.empty((B, T, H), dtype=torch.float32, device=dev)
    dinit = torch.empty((B, H, K, V), dtype=torch.float32, device=dev)
    nws = L.gdn_scalar_workspace_bytes(ctypes.byref(shape), chunk)
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=dev)
    if d_output is not None:
        if d_output.dtype != q.dtype:
            d_output = d_output.to(q.dtype)
        if not _rows_aligned(d_output):
            # Autograd often hands over an expanded (stride-0) upstream, e.g.
            # from out.sum(); the chunk kernels read 16-byte row pieces.
            d_output = d_output.contiguous()
    dfin = None if d_final_state is None else d_final_state.float().contiguous()
    dsc = None if d_scores is None else d_scores.float().contiguous()
    views = [_view(x) for x in (q, k, v, beta, g, valid, reset)]
    dov = _view(d_output)
    with on_device(dev):
        rc = L.gdn_scalar_backward(
            ctypes.byref(shape), chunk, *[ctypes.byref(x) for x in views], _ptr(checkpoint),
            checkpoint.numel(), ctypes.byref(dov) if d_output is not None else None, _ptr(dfin),
            _ptr(dsc), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(db), _ptr(dg), _ptr(dinit), _ptr(ws),
            nws, _stream(q))
    check("gdn_scalar_backward", rc)
    return dq, dk, dv, db, dg, dinit


class _ScalarScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, beta, g, valid, reset, initial, chunk):
        out, final, scores, ck = gdn_scalar_forward(q, k, v, beta, g, valid, reset, initial,
                                                    chunk)
        # Unused outputs reach backward as None (not zero tensors), so the
        # kernels skip the work of adjoints that are absent.
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(q, k, v, beta, g, valid, reset)
        ctx.checkpoint = ck
        ctx.chunk = chunk
        ctx.has_initial = initial is not None
        return out, final, scores

    @staticmethod
    def backward(ctx, d_out, d_final, d_scores):
        q, k, v, beta, g, valid, reset = ctx.saved_tensors
        dq, dk, dv, db, dg, dinit = gdn_scalar_backward(q, k, v, beta, g, valid, reset,
                                                        ctx.checkpoint, ctx.chunk, d_out,
                                                        d_final, d_scores)
        return dq, dk, dv, db, dg, None, None, (dinit if ctx.has_initial else None), None


def gdn_scalar_scan(q, k, v, beta, g, valid=None, reset=None, initial=None,
                    chunk_size: int = 64):
    """Scalar-gate gated delta rule: S = a S + b k (v - a S^T k)^T with
    a = exp(g), b = beta per token and head.  beta, g: [B,T,H] float32.
    Returns (output [B,T,H,V], final_state [B,H,K,V] f32, scores [B,T,H] f32),
    differentiable in q, k, v, beta, g and initial."""
    B, T, H, K = q.shape
    if valid is None:
        valid = torch.ones((B, T), dtype=torch.float32, device=q.device)
    if reset is None:
        reset = torch.zeros((B, T), dtype=torch.float32, device=q.device)
    _check_shapes(q, k, v, [("beta", beta, 0), ("g", g, 0)], valid, reset, initial)
    valid = _mask(valid, q)
    reset = _mask(reset, q)
    beta = beta if beta.dtype == torch.float32 else beta.float()
    g = g if g.dtype == torch.float32 else g.float()
    if initial is not None and initial.dtype != torch.float32:
        initial = initial.float()
    return _ScalarScan.apply(q, k, v, beta, g, valid, reset, initial, chunk_size)


# ---- decode ---------------------------------------------------------------------


def gdn_decode_step(state, q, k, v, alpha, erase, write, valid=None, reset=None):
    """One token per sequence on a carried state (updated in place).
    state: [B,H,K,V] f32 contiguous; q, k, alpha, erase: [B,1,H,K]; v, write:
    [B,1,H,V].  Returns (output [B,1,H,V], scores [B,1,H])."""
    L = lib()
    if not (state.is_contiguous() and state.dtype == torch.float32):
        raise ValueError("state must be a contiguous float32 [B,H,K,V] tensor")
    shape = _shape(q, v)
    B, T, H, K = q.shape
    V = v.shape[3]
    out = torch.empty((B, T, H, V), dtype=q.dtype, device=q.device)
    scores = torch.empty((B, T, H), dtype=torch.float32, device=q.device)
    views = [_view(x) for x in (q, k, v, alpha, erase, write)]
    vv = _view(valid) if valid is not None else None
    rv = _view(reset) if reset is not None else None
    with on_device(q.device):
        rc = L.gdn2_decode_step(ctypes.byref(shape), *[ctypes.byref(x) for x in views],
                                ctypes.byref(vv) if vv is not None else None,
                                ctypes.byref(rv) if rv is not None else None, _ptr(state),
                                _ptr(out), _code(out), _ptr(scores), _stream(q))
    check("gdn2_decode_step", rc)
    return out, scores


# ---- measurement ----------------------------------------------------------------


def stage_timing(enable: bool = True) -> None:
    """Record HIP events around each chunk-path kernel of the following calls
    (gdn2_stage_timing); not for use under graph capture."""
    check("gdn2_stage_timing", lib().gdn2_stage_timing(1 if enable else 0))


def stage_times() -> dict:
    """Per-kernel durations (ms) of the most recent timed calls, by stage name;
    call after synchronising the stream.  Stages that have not run are absent."""
    L = lib()
    out = {}
    for i in range(L.gdn2_stage_count()):
        ms = L.gdn2_stage_ms(i)
        if ms >= 0:
            out[L.gdn2_stage_name(i).decode()] = ms
    return out


from .mixer_ops import causal_conv, decay, l2_norm, rms_norm  # noqa: E402
from .train_ops import (FusedAdamW, adamw_update, cross_entropy_rows,  # noqa: E402
                        linear_cross_entropy)
from .hola_ops import HolaReadOutput, hola_read, hola_schedule  # noqa: E402
from . import lm_ops  # noqa: E402

__all__ += ["causal_conv", "l2_norm", "rms_norm", "decay", "cross_entropy_rows",
            "linear_cross_entropy", "adamw_update", "FusedAdamW", "HolaReadOutput", "hola_read",
            "hola_schedule", "lm_ops"]
