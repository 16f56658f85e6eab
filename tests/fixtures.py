"""Restatements of the reference's procedural GDN-2 fixtures (test data only).

Every builder returns plain numpy arrays in the reference layouts
([batch, time, head, channel] sequences, [batch, time] masks,
[batch, head, key, value] states).  Values are produced in float32 exactly as
the reference writes them (`(... as f64).sin() as f32`), so the f64 oracle and
the GPU path consume identical numbers.

  gdn_fixture(t)          crates/mixers/src/checks.rs:120-180 (Fixture::new, GDN-2 widths)
  aligned_fixture(t)      crates/mixers/src/checks.rs:181-198 (Fixture::aligned)
  gate_fixture(t, mode)   crates/mixers/src/kron_checks.rs:124-188 (GDN gate edits,
                          initial_data, score_seed, objectives 0..3)
  reset_padding_fixture() crates/mixers/src/chunk_tests.rs:25-75 (B2/T5/H2/K3/V4)
  dre_tokens(n, seed)     reuse/crates/dre-gdn2/src/tests.rs:35-51 (SplitMix tokens)
  kron_raw(b, t, seed)    crates/experiment/src/kron_benchmark.rs:73-116 (the isolated-scan
                          benchmark fixture, GDN-2 widths)
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32


def _sin32(x):
    return np.sin(np.asarray(x, dtype=np.float64)).astype(F32)


def _cos32(x):
    return np.cos(np.asarray(x, dtype=np.float64)).astype(F32)


class Fixture(dict):
    """dict of arrays with attribute access."""

    __getattr__ = dict.__getitem__


def gdn_fixture(t: int, k: int = 32, v: int = 64, b: int = 2, h: int = 4) -> Fixture:
    """The reference's widths are K = 32, V = 64 with B = 2, H = 4; other
    widths and sizes apply the same per-element formulas to a larger array."""
    widths = [k, k, v, k, k, v]
    data = []
    for field, width in enumerate(widths):
        i = np.arange(b * t * h * width, dtype=np.int64)
        signal = _sin32((i * 13 + field * 19 + 1).astype(np.float64) * 0.037)
        if field == 3:
            x = F32(0.91) + F32(0.03) * signal
        elif field >= 4:
            x = F32(0.45) + F32(0.1) * signal
        else:
            x = F32(0.1) * signal
        data.append(x.astype(F32).reshape(b, t, h, width))
    i = np.arange(b * t)
    r, p = i // t, i % t
    valid = (p < np.maximum(t - (r + 1), 0)) & (p != 9) & (p != 11)
    reset = (p == 0) | (p == 5) | (p == 19)
    iu = np.arange(b * t * h * v, dtype=np.float64)
    upstream = _cos32((iu * 7 + 3) * 0.051).reshape(b, t, h, v)
    ia = np.arange(b * h * k * v, dtype=np.float64)
    final_adjoint = (F32(0.03) * _sin32((ia * 3 + 1) * 0.04)).reshape(b, h, k, v)
    return Fixture(q=data[0], k=data[1], v=data[2], alpha=data[3], erase=data[4],
                   write=data[5], valid=valid.reshape(b, t).astype(np.uint8),
                   reset=reset.reshape(b, t).astype(np.uint8), upstream=upstream,
                   final_adjoint=final_adjoint, initial=None, score_adjoint=None)


def aligned_fixture(t: int) -> Fixture:
    f = gdn_fixture(t)
    for name in ("q", "k", "v", "alpha", "erase", "write"):
        x = f[name]
        width = x.shape[-1]
        if name == "alpha":
            x[...] = 1.0
        elif name in ("erase", "write"):
            x[...] = 0.5
        else:
            flat = x.reshape(-1)
            flat[...] = np.where(np.arange(flat.size) % width == 0, 1.0, 0.0)
    return f


def gate_fixture(t: int, mode: int = 0, K: int = 32, V: int = 64, b: int = 2,
                 h: int = 4) -> Fixture:
    """GDN gate fixture with the edits of kron_checks.rs:132-188.

    mode 0: output + final state + score objectives; 1: output only;
    2: final state only; 3: score only (kron_checks.rs:190-192).  K, V, b and h
    default to the reference's; other values apply the same formulas and
    edits (alpha zero on key channel 0 at p = 2, on every key channel at
    p = 16) to a larger problem."""
    f = gdn_fixture(t, K, V, b, h)
    valid = f.valid.astype(bool).reshape(-1)
    reset = f.reset.astype(bool).reshape(-1)
    reset[0] = False
    if t == 1:
        valid[:] = True
    for row in range(b):
        if t > 9:
            reset[row * t + 9] = True  # reset on padding must be ignored
        if row == 1 and t > 16:
            valid[row * t + 16:(row + 1) * t] = False  # includes an entire padded chunk
        for p in range(t):
            for hh in range(h):
                for name in ("k", "v"):
                    x = f[name][row, p, hh]
                    norm = np.sqrt(np.sum(x * x, dtype=F32), dtype=F32)
                    x /= norm
                if p == 1:  # exactly zero edit with nonzero key/value norms
                    f.erase[row, p, hh] = 0.0
                    f.write[row, p, hh] = 0.0
                elif p == 3:
                    f.write[row, p, hh] = -0.2
                elif p == 4:
                    f.k[row, p, hh] = 0.0  # zero key norm subgradient
                elif p == 6:
                    f.v[row, p, hh] = 0.0  # zero value norm
                if p == 2:
                    f.alpha[row, p, hh, :1] = 0.0
                elif p == 16:
                    f.alpha[row, p, hh, :K] = 0.0
    f["valid"] = valid.reshape(b, t).astype(np.uint8)
    f["reset"] = reset.reshape(b, t).astype(np.uint8)
    ii = np.arange(b * h * K * V).astype(F32)
    f["initial"] = (F32(0.03) * np.sin((ii * F32(11) + F32(7)) * F32(0.017)).astype(F32)).reshape(
        b, h, K, V)
    isd = np.arange(b * t * h).astype(F32)
    score_seed = (F32(0.07) * np.cos((isd * F32(7) + F32(2)) * F32(0.13)).astype(F32)).reshape(
        b, t, h)
    use_output = mode in (0, 1)
    use_final = mode in (0, 2)
    use_scores = mode in (0, 3)
    if not use_output:
        f["upstream"] = np.zeros_like(f.upstream)
    if not use_final:
        f["final_adjoint"] = np.zeros_like(f.final_adjoint)
    f["score_adjoint"] = score_seed if use_scores else np.zeros_like(score_seed)
    return f


def reset_padding_fixture() -> Fixture:
    """chunk_tests.rs:25-75: a padded reset between active tokens keeps the
    initial-state path; a later valid reset severs it."""
    b, t, h, k, v = 2, 5, 2, 3, 4
    valid = np.array([1, 0, 1, 1, 0, 1, 1, 0, 1, 0], dtype=np.uint8).reshape(b, t)
    reset = np.array([0, 1, 0, 1, 0, 1, 0, 1, 0, 1], dtype=np.uint8).reshape(b, t)
    initial = (F32(0.03) * (1 + np.arange(b * h * k * v) % 7).astype(F32)).reshape(b, h, k, v)
    upstream = (F32(0.04) * ((np.arange(b * t * h * v) % 9).astype(F32) - F32(3))).reshape(
        b, t, h, v)
    widths = [k, k, v, k, k, v]
    data = []
    for field, width in enumerate(widths):
        i = np.arange(b * t * h * width)
        if field == 3:
            x = np.where((i % (h * k) == 1) & ((i // (h * k)) % t == 2), F32(0),
                         F32(0.75) + F32(0.02) * (i % 5).astype(F32))
        elif field == 4:
            x = np.full(i.shape, F32(0.6))
        elif field == 5:
            x = np.where((i // (h * width)) % t == 2, F32(0), F32(-0.25))
        else:
            x = F32(0.08) * (((i + 3 * field) % 7).astype(F32) - F32(2))
        data.append(x.astype(F32).reshape(b, t, h, width))
    return Fixture(q=data[0], k=data[1], v=data[2], alpha=data[3], erase=data[4],
                   write=data[5], valid=valid, reset=reset, initial=initial,
                   upstream=upstream, final_adjoint=None, score_adjoint=None)


class SplitMix:
    """SplitMix64 stream (crates/experiment/src/data.rs:13-21)."""

    def __init__(self, seed: int):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def next(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    def uniform(self) -> float:
        return (self.next() >> 11) / float(1 << 53)

    def signed(self) -> float:
        return 2.0 * self.uniform() - 1.0

    def normal(self) -> float:
        radius = math.sqrt(-2.0 * math.log(1.0 - self.uniform()))
        return radius * math.cos(2.0 * math.pi * self.uniform())


def dre_tokens(n: int, seed: int = 7, K: int = 32, V: int = 64):
    """Tokens of reuse/crates/dre-gdn2/src/tests.rs:40-51 as [1, n, 1, width] f32."""
    rng = SplitMix(seed)
    fields = {name: [] for name in ("q", "k", "v", "alpha", "erase", "write")}
    spec = [("q", K, 0.0, 0.5), ("k", K, 0.0, 0.45), ("v", V, 0.0, 1.0),
            ("alpha", K, 0.875, 0.075), ("erase", K, 0.5, 0.2), ("write", V, 0.75, 0.25)]
    for _ in range(n):
        for name, width, center, spread in spec:
            fields[name].append([center + spread * rng.signed() for _ in range(width)])
    return {name: np.asarray(x, dtype=F32).reshape(1, n, 1, -1) for name, x in fields.items()}


def splitmix_block(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64 from seed (data.rs:13-21), vectorized:
    the state after step j is seed + j * 0x9E3779B97F4A7C15 (mod 2^64)."""
    with np.errstate(over="ignore"):
        j = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed) + j * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def kron_raw(b: int, t: int, seed: int = 1, h: int = 4) -> Fixture:
    """The reference's isolated-scan benchmark fixture (kron_benchmark.rs:73-116,
    GDN-2 widths K32/V64): one SplitMix64 stream drawn field by field; x = the top
    24 bits / 2^24; q, k, v = x - 0.5 with every row scaled to unit norm; alpha =
    0.90 + 0.09 x; erase and write = 0.1 + 0.8 x; all valid, no resets, zero
    initial state, all-ones upstream gradient."""
    widths = [32, 32, 64, 32, 32, 64]
    n = b * t * h * sum(widths)
    x = ((splitmix_block(seed, n) >> np.uint64(40)).astype(np.float32)
         / np.float32(1 << 24))
    out, off = [], 0
    for field, w in enumerate(widths):
        f = x[off:off + b * t * h * w].reshape(b, t, h, w)
        off += b * t * h * w
        if field == 3:
            f = np.float32(0.90) + np.float32(0.09) * f
        elif field >= 4:
            f = np.float32(0.1) + np.float32(0.8) * f
        else:
            f = f - np.float32(0.5)
            f = f / np.sqrt((f * f).sum(-1, keepdims=True, dtype=np.float32))
        out.append(f.astype(np.float32))
    return Fixture(q=out[0], k=out[1], v=out[2], alpha=out[3], erase=out[4], write=out[5],
                   valid=np.ones((b, t), np.uint8), reset=np.zeros((b, t), np.uint8),
                   initial=np.zeros((b, h, 32, 64), np.float32),
                   upstream=np.ones((b, t, h, 64), np.float32), final_adjoint=None,
                   score_adjoint=None)
