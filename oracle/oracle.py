"""ctypes front end of the CPU oracle (oracle/gdn2_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product path (the
HIP library and its Python mirror under delta-block-lm_amd/) never imports it.

Arrays use the reference layouts: sequences [batch, time, head, channel],
masks [batch, time], states [batch, head, key, value]
(reference crates/mixers/src/chunk.rs:126).

Parity status of each function (see tests/test_oracle.py for the checks):
  scan / backward        pinned (closed forms, central differences, reference
                         fixture assertions, triangular-solve special case)
  scalar_gates /
  scalar_gate_grads      pinned (f64 central differences on beta and g)
  doc_limits_to_masks    pinned (gdn2_reference.rs:85-99 cases, hand-built rows)
  normals / splitmix     pinned (SplitMix64 published test values)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libgdn2_oracle.so")
_lib = None

_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> str:
    """Compile the oracle library with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        i = ctypes.c_int
        L.gdn2_oracle_scan_bthw.argtypes = [i] * 5 + [_dp] * 6 + [_u8p] * 2 + [_dp] * 4
        L.gdn2_oracle_scan_bthw.restype = i
        L.gdn2_oracle_backward_bthw.argtypes = [i] * 5 + [_dp] * 6 + [_u8p] * 2 + [_dp] * 11
        L.gdn2_oracle_backward_bthw.restype = i
        L.gdn2_oracle_normals.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_int64, _dp]
        L.gdn2_oracle_splitmix_fill.argtypes = [
            ctypes.POINTER(ctypes.c_uint64), ctypes.c_int64, ctypes.POINTER(ctypes.c_uint64)]
        L.gdn2_oracle_threads.restype = i
        _lib = L
    return _lib


def _d(x):
    if x is None:
        return None
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64))


def _ptr(x, kind=_dp):
    return None if x is None else x.ctypes.data_as(kind)


def _masks(valid, reset):
    return (np.ascontiguousarray(np.asarray(valid) != 0, dtype=np.uint8),
            np.ascontiguousarray(np.asarray(reset) != 0, dtype=np.uint8))


def scan(q, k, v, alpha, erase, write, valid, reset, initial=None):
    """f64 forward (reference.rs:41-119).  Returns (output, final_state, scores)."""
    q, k, v, alpha, erase, write = map(_d, (q, k, v, alpha, erase, write))
    B, T, H, K = q.shape
    V = v.shape[3]
    valid, reset = _masks(valid, reset)
    initial = _d(initial)
    out = np.zeros((B, T, H, V))
    fin = np.zeros((B, H, K, V))
    sc = np.zeros((B, T, H))
    rc = lib().gdn2_oracle_scan_bthw(B, T, H, K, V, _ptr(q), _ptr(k), _ptr(v), _ptr(alpha),
                                     _ptr(erase), _ptr(write), _ptr(valid, _u8p),
                                     _ptr(reset, _u8p), _ptr(initial), _ptr(out), _ptr(fin),
                                     _ptr(sc))
    if rc:
        raise ValueError("nonfinite recurrence input")
    return out, fin, sc


def backward(q, k, v, alpha, erase, write, valid, reset, initial=None, upstream=None,
             final_adjoint=None, score_adjoint=None):
    """f64 VJP (reference.rs:127-257).  Returns a dict of gradients named after
    the inputs plus 'initial'."""
    q, k, v, alpha, erase, write = map(_d, (q, k, v, alpha, erase, write))
    B, T, H, K = q.shape
    V = v.shape[3]
    valid, reset = _masks(valid, reset)
    initial, upstream, final_adjoint, score_adjoint = map(
        _d, (initial, upstream, final_adjoint, score_adjoint))
    g = {n: np.zeros(x.shape) for n, x in
         zip(("q", "k", "v", "alpha", "erase", "write"), (q, k, v, alpha, erase, write))}
    g["initial"] = np.zeros((B, H, K, V))
    rc = lib().gdn2_oracle_backward_bthw(
        B, T, H, K, V, _ptr(q), _ptr(k), _ptr(v), _ptr(alpha), _ptr(erase), _ptr(write),
        _ptr(valid, _u8p), _ptr(reset, _u8p), _ptr(initial), _ptr(upstream),
        _ptr(final_adjoint), _ptr(score_adjoint), _ptr(g["q"]), _ptr(g["k"]), _ptr(g["v"]),
        _ptr(g["alpha"]), _ptr(g["erase"]), _ptr(g["write"]), _ptr(g["initial"]))
    if rc:
        raise ValueError("nonfinite recurrence input")
    return g


def normals(seed: int, n: int) -> np.ndarray:
    """n Box-Muller normals from SplitMix64 (reuse/.../dre-gdn2/src/tests.rs:7-32)."""
    st = ctypes.c_uint64(seed)
    out = np.zeros(n)
    lib().gdn2_oracle_normals(ctypes.byref(st), n, _ptr(out))
    return out


def splitmix(seed: int, n: int) -> np.ndarray:
    st = ctypes.c_uint64(seed)
    out = np.zeros(n, dtype=np.uint64)
    lib().gdn2_oracle_splitmix_fill(ctypes.byref(st), n, out.ctypes.data_as(
        ctypes.POINTER(ctypes.c_uint64)))
    return out


def threads() -> int:
    return lib().gdn2_oracle_threads()


# --- scalar-gate adapter --------------------------------------------------------
# The standard scalar gated delta rule S = a*S + b*k(v - a*S^T k)^T is the GDN-2
# recurrence with alpha[i]=exp(g), erase[i]=beta, write[j]=beta for every channel.


def scalar_gates(beta, g, K, V):
    beta = np.asarray(beta, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    alpha = np.repeat(np.exp(g)[..., None], K, axis=-1)
    erase = np.repeat(beta[..., None], K, axis=-1)
    write = np.repeat(beta[..., None], V, axis=-1)
    return alpha, erase, write


def scalar_gate_grads(g, grads):
    """Chain rule: dbeta = sum_i derase + sum_j dwrite, dg = exp(g) * sum_i dalpha."""
    g = np.asarray(g, dtype=np.float64)
    dbeta = grads["erase"].sum(-1) + grads["write"].sum(-1)
    dg = np.exp(g) * grads["alpha"].sum(-1)
    return dbeta, dg


def doc_limits_to_masks(doc_start, doc_end):
    """Integer document limits (gdn2_reference.rs:85-99) to valid/reset masks:
    padding where end < start; a reset where start == t on a valid token."""
    doc_start = np.asarray(doc_start)
    doc_end = np.asarray(doc_end)
    T = doc_start.shape[-1]
    t = np.arange(T)
    valid = doc_end >= doc_start
    reset = valid & (doc_start == t)
    return valid.astype(np.uint8), reset.astype(np.uint8)


# --- f32 chunked CPU scan (oracle/chunk_cpu.c) ------------------------------------
# The reference's CPU tensor solver chunk::scan (crates/mixers/src/chunk.rs:129-250)
# restated in f32; the "f32 chunked CPU scan" leg of bench.py's cpu_baseline.
# Pinned against scan() (f64) by tests/test_chunk_cpu.py.

_SO_CHUNK = os.path.join(_HERE, "_build", "libgdn2_chunk_cpu.so")
_chunk_lib = None
_fp = ctypes.POINTER(ctypes.c_float)


def _chunk():
    global _chunk_lib
    if _chunk_lib is None:
        if not os.path.exists(_SO_CHUNK):
            build()
        L = ctypes.CDLL(_SO_CHUNK)
        L.gdn2_chunk_cpu_f32.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int] + [_fp] * 12
        L.gdn2_chunk_cpu_f32.restype = ctypes.c_int
        L.gdn2_chunk_cpu_threads.restype = ctypes.c_int
        _chunk_lib = L
    return _chunk_lib


def chunk_threads() -> int:
    return _chunk().gdn2_chunk_cpu_threads()


def chunk_scan_f32(q, k, v, alpha, erase, write, valid, reset, initial=None, chunk=64):
    """f32 chunked forward (chunk.rs:129-250).  Returns (output, final_state, scores)."""
    f = lambda x: None if x is None else np.ascontiguousarray(np.asarray(x, dtype=np.float32))  # noqa
    q, k, v, alpha, erase, write, valid, reset, initial = map(
        f, (q, k, v, alpha, erase, write, valid, reset, initial))
    B, T, H, K = q.shape
    V = v.shape[3]
    out = np.empty((B, T, H, V), np.float32)
    fin = np.empty((B, H, K, V), np.float32)
    sc = np.empty((B, T, H), np.float32)
    p = lambda x: None if x is None else x.ctypes.data_as(_fp)  # noqa
    rc = _chunk().gdn2_chunk_cpu_f32(B, T, H, K, V, chunk, p(q), p(k), p(v), p(alpha), p(erase),
                                     p(write), p(valid), p(reset), p(initial), p(out), p(fin),
                                     p(sc))
    if rc != 0:
        raise RuntimeError(f"gdn2_chunk_cpu_f32 failed ({rc})")
    return out, fin, sc
