"""Helpers for the GPU parity tests: device upload and the tolerance gates."""
from __future__ import annotations

import os

import numpy as np
import torch

# North-star gates, rms-floored (reuse/crates/dre-gdn2/src/tests.rs:106-119):
# |x - ref| <= tol * (|ref| + rms(ref)); tol 1e-4 for f32, 2e-2 for bf16 inputs.
TOL_F32 = 1e-4
TOL_BF16 = 2e-2
# Reference f32 gate of the GDN numerical checks (crates/mixers/src/checks.rs:73-74).
REF_ATOL, REF_RTOL = 2e-5, 3e-4


def dev(x, dtype=torch.float32):
    if x is None:
        return None
    return torch.as_tensor(np.ascontiguousarray(x)).to(device="cuda", dtype=dtype)


def host(t) -> np.ndarray:
    return t.detach().to(torch.float64).cpu().numpy()


def gate(name, got, ref, tol, exact_zero=None, ref_gate=False):
    """Assert the rms-floored gate (and optionally the reference's own gate)."""
    got = host(got) if torch.is_tensor(got) else np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64).reshape(got.shape)
    assert np.all(np.isfinite(got)), f"{name}: nonfinite values"
    scale = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    err = np.abs(got - ref)
    bound = tol * (np.abs(ref) + scale) + 1e-30
    bad = err > bound
    if exact_zero is not None:
        ez = np.broadcast_to(exact_zero, got.shape)
        assert np.all(got[ez] == 0), f"{name}: padding entries are not exactly zero"
        bad &= ~ez
    ratio = err / bound
    if exact_zero is not None:
        ratio = np.where(ez, 0.0, ratio)
    log = os.environ.get("GDN2_GATE_LOG")
    if log and ratio.size:
        # worst error-to-gate ratio per gated output, for the precision tables
        test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
        with open(log, "a") as fh:
            fh.write(f"{test}\t{name}\t{float(ratio.max()):.4f}\n")
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(
            f"{name}: {bad.sum()} of {bad.size} outside tol {tol} (rms {scale:.3e}); worst at "
            f"{i}: got {got[i]:.8e} ref {ref[i]:.8e} err {err[i]:.3e} bound {bound[i]:.3e}")
    if ref_gate:
        rb = REF_ATOL + REF_RTOL * np.abs(ref)
        assert np.all(err <= rb), f"{name}: outside the reference gate 2e-5 + 3e-4|ref|"
    return float(err.max()) if err.size else 0.0
