"""GPU parity against the committed golden vectors (tests/golden/*.npz).

cfg0 (B1 H2 T256 K=V=32 fp32, chunk 32) runs the
scalar-gate op forward and backward; the reference fixtures run the
channel-wise training op.  Gates: the north-star rms-floored 1e-4 for fp32
and the reference's own 2e-5 + 3e-4|ref| (crates/mixers/src/checks.rs:73-74);
padding entries must be exactly zero.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from golden_util import load  # noqa: E402
from gpu_util import TOL_F32, dev, gate  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


@pytest.mark.parametrize("chunk", [32, 64])
def test_cfg0_scalar_scan_matches_golden(dk, chunk):
    x, e = load("cfg0")
    xs = {n: dev(x[n]).requires_grad_(True) for n in ("q", "k", "v", "beta", "g")}
    out, fin, sc = dk.gdn_scalar_scan(xs["q"], xs["k"], xs["v"], xs["beta"], xs["g"],
                                      chunk_size=chunk)
    gate("output", out, e["output"], TOL_F32, ref_gate=True)
    gate("final_state", fin, e["final_state"], TOL_F32, ref_gate=True)
    gate("scores", sc, e["scores"], TOL_F32, ref_gate=True)
    (out * dev(x["upstream"])).sum().backward()
    for n in ("q", "k", "v", "beta", "g"):
        gate(f"d{n}", xs[n].grad, e[f"d{n}"], TOL_F32, ref_gate=True)


@pytest.mark.parametrize("name", ["reset_padding", "gate_t7"])
@pytest.mark.parametrize("chunk", [1, 5, 16])
def test_fixture_training_scan_matches_golden(dk, name, chunk):
    x, e = load(name)
    groups = ("q", "k", "v", "alpha", "erase", "write")
    xs = {n: dev(x[n]).requires_grad_(True) for n in groups}
    init = dev(x["initial"]).requires_grad_(True) if "initial" in x else None
    r = dk.gdn_training_scan(*[xs[n] for n in groups], dev(x["valid"]), dev(x["reset"]), init,
                             chunk)
    pad = (x["valid"] == 0)[:, :, None, None]
    gate("output", r.output, e["output"], TOL_F32, exact_zero=pad, ref_gate=True)
    gate("final_state", r.final_state, e["final_state"], TOL_F32, ref_gate=True)
    gate("scores", r.scores[..., 0], e["scores"], TOL_F32, exact_zero=pad[..., 0], ref_gate=True)
    loss = (r.output * dev(x["upstream"])).sum()
    if "final_adjoint" in x:
        loss = loss + (r.final_state * dev(x["final_adjoint"])).sum()
    if "score_adjoint" in x:
        loss = loss + (r.scores[..., 0] * dev(x["score_adjoint"])).sum()
    loss.backward()
    for n in groups:
        gate(f"d{n}", xs[n].grad, e[f"d{n}"], TOL_F32, exact_zero=pad, ref_gate=True)
    if init is not None:
        gate("d_initial", init.grad, e["dinitial"], TOL_F32, ref_gate=True)
