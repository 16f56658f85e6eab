"""Write the golden vectors under tests/golden/ (test data only).

The reference holds no golden files for this path; these vectors are the
f64 oracle's answers (oracle/gdn2_oracle.c, a restatement of
crates/mixers/src/reference.rs:41-257) on the inputs below, stored with the
inputs so that the GPU tests and later builds check against fixed numbers:

  cfg0.npz           BASELINE configs[0]: B1 H2 T256 K=V=32 fp32, SplitMix64
                     seed 0 (delta_mixers.synthetic), scalar gates; forward
                     outputs plus the VJP for an upstream drawn from seed 1.
  reset_padding.npz  crates/mixers/src/chunk_tests.rs:25-75 (B2 T5 H2 K3 V4),
                     channel-wise gates, nonzero initial state.
  gate_t7.npz        crates/mixers/src/kron_checks.rs:124-188 GDN gate fixture
                     at T=7, objective 0 (output + final state + scores).

Inputs are stored exactly (float32); expected values are the f64 results
rounded to float32.  Run from the repository root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "delta-block-lm_amd"))
sys.path.insert(0, os.path.dirname(HERE))

import fixtures as fx  # noqa: E402
from delta_mixers.synthetic import CONFIGS, NormalStream, generate  # noqa: E402
from oracle import oracle  # noqa: E402

F32 = np.float32


def cfg0_inputs():
    cfg = CONFIGS[0]
    p = generate(cfg, seed=0)
    B, T, H, V = cfg.batch, cfg.time, cfg.heads, cfg.values
    upstream = NormalStream(1).normals(B * T * H * V).astype(F32).reshape(B, T, H, V)
    return {"q": p["q"], "k": p["k"], "v": p["v"], "beta": p["beta"], "g": p["g"],
            "upstream": upstream}


def cfg0_expected(x):
    K, V = x["q"].shape[3], x["v"].shape[3]
    B, T = x["q"].shape[:2]
    a, e, w = oracle.scalar_gates(x["beta"], x["g"], K, V)
    valid = np.ones((B, T), np.uint8)
    reset = np.zeros((B, T), np.uint8)
    out, fin, sc = oracle.scan(x["q"], x["k"], x["v"], a, e, w, valid, reset)
    gr = oracle.backward(x["q"], x["k"], x["v"], a, e, w, valid, reset, None, x["upstream"])
    dbeta, dg = oracle.scalar_gate_grads(x["g"], gr)
    return {"output": out, "final_state": fin, "scores": sc, "dq": gr["q"], "dk": gr["k"],
            "dv": gr["v"], "dbeta": dbeta, "dg": dg, "d_initial": gr["initial"]}


CHANNEL_INPUTS = ("q", "k", "v", "alpha", "erase", "write", "valid", "reset", "initial",
                  "upstream", "final_adjoint", "score_adjoint")


def channel_inputs(f):
    return {n: np.asarray(f[n]) for n in CHANNEL_INPUTS if f.get(n) is not None}


def channel_expected(x):
    g = lambda n: x.get(n)  # noqa: E731
    out, fin, sc = oracle.scan(x["q"], x["k"], x["v"], x["alpha"], x["erase"], x["write"],
                               x["valid"], x["reset"], g("initial"))
    gr = oracle.backward(x["q"], x["k"], x["v"], x["alpha"], x["erase"], x["write"], x["valid"],
                         x["reset"], g("initial"), g("upstream"), g("final_adjoint"),
                         g("score_adjoint"))
    res = {"output": out, "final_state": fin, "scores": sc}
    for n in ("q", "k", "v", "alpha", "erase", "write", "initial"):
        res["d" + n] = gr[n]
    return res


def fixtures():
    """name -> (inputs, expected-function)."""
    return {
        "cfg0": (cfg0_inputs(), cfg0_expected),
        "reset_padding": (channel_inputs(fx.reset_padding_fixture()), channel_expected),
        "gate_t7": (channel_inputs(fx.gate_fixture(7, 0)), channel_expected),
    }


def main():
    for name, (x, fn) in fixtures().items():
        exp = fn(x)
        arrays = {f"in_{k}": v for k, v in x.items()}
        arrays.update({f"out_{k}": np.asarray(v, np.float64).astype(F32) for k, v in exp.items()})
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
