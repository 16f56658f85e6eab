"""HOLA cache read (gdn2_hola_*) through the C ABI against the f64 oracle.

Mirrors the reference's fixture checks (crates/mixers/src/hola_checks.rs:561-606):
both policies on (T, capacity, chunk) = (7,16,16), (35,16,1), (83,16,16),
(145,64,16) with packed documents, ties, resets and padding in the last
physical slot; the overflow fixture; strided q/k/v/scores/upstream; zero inputs
and adjoints; and the cancellation check (hola_checks.rs:466-512, analytic VJP
of the observed forward probability).  Outputs and gradients (q, k, v, sink) at
the reference's gate 2e-5 + 3e-4|ref| (checks.rs:73-74); final cache
positions and the positions-only schedule exactly.  Wider heads (K = V = 64,
128) against the oracle at the north-star fp32 gate.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import hola_fixtures as hf  # noqa: E402
from gpu_util import REF_ATOL, REF_RTOL, TOL_F32, gate  # noqa: E402
from oracle import hola_oracle as ho  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def dev(x, grad=False, strided=False):
    x = np.asarray(x, np.float32)
    if strided and x.ndim == 4:  # stored [b, h, t, w], viewed [b, t, h, w]
        t = torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 1, 3))).cuda().permute(0, 2, 1, 3)
    else:
        t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    return t.requires_grad_(True) if grad else t


def ref_gate(name, got, ref):
    got = got.detach().double().cpu().numpy()
    err = np.abs(got - ref)
    bad = ~np.isfinite(got) | (err > REF_ATOL + REF_RTOL * np.abs(ref))
    assert not bad.any(), f"{name}: {bad.sum()} outside 2e-5 + 3e-4|ref|, worst {err.max():.3e}"


def run(dk, f, strided=False):
    x = {n: dev(f[n], grad=n in ("q", "k", "v", "sink"), strided=strided)
         for n in ("q", "k", "v", "sink")}
    scores = dev(f["scores"], strided=strided)
    r = dk.hola_read(x["q"], x["k"], x["v"], scores, dev(f["valid"]), dev(f["docs"]), x["sink"],
                     f["capacity"], f["chunk"], f["recency"], return_final_positions=True)
    (r.output * dev(f["upstream"], strided=strided)).sum().backward()
    assert not scores.requires_grad
    return r, x


def check(dk, f, strided=False):
    r, x = run(dk, f, strided)
    ref = ho.hola_read(f["q"], f["k"], f["v"], f["scores"], f["valid"], f["docs"], f["sink"],
                       f["capacity"], f["chunk"], f["recency"], upstream=f["upstream"])
    ref_gate("output", r.output, ref["output"])
    np.testing.assert_array_equal(r.final_positions.cpu().numpy(), ref["positions"])
    for n, g in (("q", "dq"), ("k", "dk"), ("v", "dv"), ("sink", "dsink")):
        ref_gate(g, x[n].grad, ref[g])


@pytest.mark.parametrize("recency", [False, True])
@pytest.mark.parametrize("case", hf.CASES)
def test_reference_fixtures(dk, recency, case):
    t, cap, chunk = case
    check(dk, hf.hola_fixture(2, t, cap, chunk, recency, True))


def test_overflow_fixture(dk):
    check(dk, hf.overflow_fixture())


def test_strided_and_zero_inputs(dk):
    f = hf.hola_fixture(2, 35, 16, 16, False, True)
    check(dk, f, strided=True)
    for n in ("q", "k", "v", "upstream"):
        f[n] = np.zeros_like(f[n])
    f["sink"] = np.zeros_like(f["sink"])
    check(dk, f, strided=True)


def test_cancellation_vjp(dk):
    """hola_checks.rs:466-512: the VJP must match the analytic derivative of
    the forward's own probability p (dv = p, dsink = -p(1-p),
    dq = p(1-p) k / sqrt(32), dk = p(1-p) q / sqrt(32))."""
    f = hf.cancellation_fixture()
    r, x = run(dk, f)
    p = r.output.detach().double().cpu().numpy()[0, 0, :, 0]
    assert np.all((p > 0) & (p < 1))
    d = p * (1 - p)
    ref_gate("dv", x["v"].grad[0, 0, :, 0], p)
    ref_gate("dsink", x["sink"].grad, -d)
    ref_gate("dq", x["q"].grad[0, 0], d[:, None] * f["k"][0, 0] / np.sqrt(32))
    ref_gate("dk", x["k"].grad[0, 0], d[:, None] * f["q"][0, 0] / np.sqrt(32))


@pytest.mark.parametrize("recency", [False, True])
def test_schedule_matches_oracle(dk, recency):
    f = hf.hola_fixture(2, 145, 64, 16, recency, True)
    got = dk.hola_schedule(dev(f["scores"]), dev(f["valid"]), dev(f["docs"]), 64, 16, recency)
    want = ho.hola_schedule(f["scores"], f["valid"], f["docs"], 64, 16, recency)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("kv", [(64, 64), (128, 128), (32, 128)])
def test_wider_heads(dk, kv):
    K, V = kv
    rng = np.random.default_rng(K + V)
    f = hf.hola_fixture(2, 83, 8, 16, False, True)
    B, T, H = 2, 83, 4
    q = rng.normal(size=(B, T, H, K)).astype(np.float32)
    k = rng.normal(size=(B, T, H, K)).astype(np.float32)
    f.update(q=q / np.sqrt(K) ** 0.5, k=k / np.sqrt(K) ** 0.5,
             v=rng.normal(size=(B, T, H, V)).astype(np.float32),
             upstream=rng.normal(size=(B, T, H, V)).astype(np.float32))
    r, x = run(dk, f)
    ref = ho.hola_read(f["q"], f["k"], f["v"], f["scores"], f["valid"], f["docs"], f["sink"],
                       f["capacity"], f["chunk"], f["recency"], upstream=f["upstream"])
    gate("output", r.output, ref["output"], TOL_F32)
    for n, g in (("q", "dq"), ("k", "dk"), ("v", "dv"), ("sink", "dsink")):
        gate(g, x[n].grad, ref[g], TOL_F32)


def test_rejects_bad_shapes(dk):
    f = hf.hola_fixture(1, 7, 16, 16, False, False)
    args = [dev(f[n]) for n in ("q", "k", "v", "scores", "valid", "docs", "sink")]
    with pytest.raises(RuntimeError):
        dk.hola_read(*args, 16, 17)  # chunk above 16
    with pytest.raises(RuntimeError):
        dk.hola_read(*args, 65, 16)  # capacity above 64
