"""Synthetic GDN scan inputs for the benchmark configurations.

Generator: SplitMix64 (crates/experiment/src/data.rs:13-21) from seed 0, one
continuous stream; each N(0,1) draw takes two outputs, radius first, through
the Box-Muller cosine branch (reuse/crates/dre-gdn2/src/tests.rs:18-32).
SplitMix64's n-th output is a pure function of seed + n * golden-gamma, so
the stream is generated vectorised in numpy, block by block.

Draw order, each tensor row-major [B, T, H, .]: q_raw, k_raw, v, beta-logit,
g-logit, then dO (training configs) and then the decode state (config 3).
q, k = x / sqrt(sum x^2 + 1e-6) per head (crates/mixers/src/normalization.rs:21-24);
beta = sigmoid(x); g = -softplus(x) (log decay, alpha = exp(g)).
bf16 configurations round q, k, v and dO to bfloat16 (nearest even) after
generation; gates and states stay float32.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_BLOCK = 1 << 22


def splitmix_outputs(seed: int, start: int, n: int) -> np.ndarray:
    """Outputs number start+1 .. start+n of SplitMix64(seed)."""
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


class NormalStream:
    def __init__(self, seed: int = 0):
        self.seed = seed
        self.count = 0  # SplitMix outputs consumed

    def normals(self, n: int, dtype=np.float64) -> np.ndarray:
        out = np.empty(n, dtype=dtype)
        for s in range(0, n, _BLOCK):
            m = min(_BLOCK, n - s)
            u = splitmix_outputs(self.seed, self.count, 2 * m)
            self.count += 2 * m
            u1 = (u[0::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
            u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
            out[s:s + m] = np.sqrt(-2.0 * np.log(1.0 - u1)) * np.cos(2.0 * np.pi * u2)
        return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16, returned as float32 values."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) & np.uint64(0xFFFF0000)
    return u.astype(np.uint32).view(np.float32)


@dataclass(frozen=True)
class Config:
    name: str
    batch: int
    time: int
    heads: int
    keys: int
    values: int
    chunk: int
    bf16: bool
    grad: bool = True
    decode_state: bool = False


CONFIGS = {
    0: Config("cfg0-cpu-fwd", 1, 256, 2, 32, 32, 32, False, grad=False),
    1: Config("lm512", 16, 512, 8, 64, 64, 64, True),
    2: Config("long8k", 4, 8192, 16, 128, 128, 64, True),
    3: Config("decode", 256, 1024, 8, 64, 64, 64, False, grad=False, decode_state=True),
}


def _l2(x: np.ndarray) -> np.ndarray:
    return x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + 1e-6)


def generate(cfg: Config, seed: int = 0) -> dict:
    """Inputs of one configuration as float32 numpy arrays (bf16-rounded where
    the configuration is bf16)."""
    B, T, H, K, V = cfg.batch, cfg.time, cfg.heads, cfg.keys, cfg.values
    st = NormalStream(seed)
    out = {}
    q = _l2(st.normals(B * T * H * K).reshape(B, T, H, K)).astype(np.float32)
    k = _l2(st.normals(B * T * H * K).reshape(B, T, H, K)).astype(np.float32)
    v = st.normals(B * T * H * V).astype(np.float32).reshape(B, T, H, V)
    bl = st.normals(B * T * H).reshape(B, T, H)
    gl = st.normals(B * T * H).reshape(B, T, H)
    out["beta"] = (1.0 / (1.0 + np.exp(-bl))).astype(np.float32)
    out["g"] = (-(np.maximum(gl, 0) + np.log1p(np.exp(-np.abs(gl))))).astype(np.float32)
    if cfg.grad:
        out["d_output"] = st.normals(B * T * H * V).astype(np.float32).reshape(B, T, H, V)
    if cfg.decode_state:
        out["state"] = (0.02 * st.normals(B * H * K * V)).astype(np.float32).reshape(B, H, K, V)
    if cfg.bf16:
        q, k, v = round_bf16(q), round_bf16(k), round_bf16(v)
        if "d_output" in out:
            out["d_output"] = round_bf16(out["d_output"])
    out["q"], out["k"], out["v"] = q, k, v
    return out


def kron_benchmark_inputs(batch: int, time: int, seed: int = 1, heads: int = 4) -> dict:
    """The reference's isolated-scan benchmark inputs for GDN-2
    (crates/experiment/src/kron_benchmark.rs:73-116; default seed 1,
    crates/experiment/src/config.rs:405): one SplitMix64 stream drawn field by
    field, widths q, k 32, v 64, alpha, erase 32, write 64; x = (output >> 40) /
    2^24; q, k, v = x - 0.5 with every row scaled to unit norm; alpha = 0.90 +
    0.09 x; erase, write = 0.1 + 0.8 x.  All tokens valid, no resets, zero
    initial state [B, H, 32, 64] and an all-ones upstream gradient.  f32."""
    widths = (32, 32, 64, 32, 32, 64)
    names = ("q", "k", "v", "alpha", "erase", "write")
    total = batch * time * heads * sum(widths)
    x = (splitmix_outputs(seed, 0, total) >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)
    out, off = {}, 0
    for field, (name, w) in enumerate(zip(names, widths)):
        f = x[off:off + batch * time * heads * w].reshape(batch, time, heads, w)
        off += batch * time * heads * w
        if field == 3:
            f = np.float32(0.90) + np.float32(0.09) * f
        elif field >= 4:
            f = np.float32(0.1) + np.float32(0.8) * f
        else:
            f = f - np.float32(0.5)
            f = f / np.sqrt((f * f).sum(-1, keepdims=True, dtype=np.float32))
        out[name] = np.ascontiguousarray(f, dtype=np.float32)
    out["initial"] = np.zeros((batch, heads, 32, 64), np.float32)
    out["d_output"] = np.ones((batch, time, heads, 64), np.float32)
    return out
