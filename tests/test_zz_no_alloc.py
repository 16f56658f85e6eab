"""gdn_scalar_backward_noalloc (the backward whose scratch is the library's
fixed device array) against gdn_scalar_backward with a caller workspace:
the same kernels on the same inputs, so the gradients must be bit-identical.
Two calls in a row, the second on a smaller problem, so the second runs on
scratch the first left behind; a shape above the fixed size is rejected."""
import ctypes

import pytest

torch = pytest.importorskip("torch")

from chunk_util import problem  # noqa: E402
from gpu_util import dev  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


def _noalloc_backward(dk, q, k, v, beta, g, valid, reset, ck, dO, dF, dS):
    from delta_kernels import _ptr, _shape, _stream, _view
    from delta_kernels._lib import check, lib
    L = lib()
    B, T, H, K = q.shape
    V = v.shape[3]
    shape = _shape(q, v)
    dq, dkk, dv = (torch.empty_like(x) for x in (q, k, v))
    db = torch.empty((B, T, H), dtype=torch.float32, device=q.device)
    dg = torch.empty((B, T, H), dtype=torch.float32, device=q.device)
    dinit = torch.empty((B, H, K, V), dtype=torch.float32, device=q.device)
    views = [_view(x) for x in (q, k, v, beta, g, valid, reset)]
    dov = _view(dO)
    rc = L.gdn_scalar_backward_noalloc(
        ctypes.byref(shape), 64, *[ctypes.byref(x) for x in views], _ptr(ck), ck.numel(),
        ctypes.byref(dov), _ptr(dF), _ptr(dS), _ptr(dq), _ptr(dkk), _ptr(dv), _ptr(db), _ptr(dg),
        _ptr(dinit), _stream(q))
    check("gdn_scalar_backward_noalloc", rc)
    return dq, dkk, dv, db, dg, dinit


def _case(dk, seed, B, T, H):
    p = problem(seed, B, T, H, masks=True)
    x = {n: dev(p[n], torch.bfloat16) for n in ("q", "k", "v", "dO")}
    beta, g, valid, reset = (dev(p[n]) for n in ("beta", "g", "valid", "reset"))
    init, dF, dS = dev(p["initial"]), dev(p["dF"]), dev(p["dS"])
    out, fin, sc, ck = dk.gdn_scalar_forward(x["q"], x["k"], x["v"], beta, g, valid, reset, init,
                                             64)
    ref = dk.gdn_scalar_backward(x["q"], x["k"], x["v"], beta, g, valid, reset, ck, 64, x["dO"],
                                 dF, dS)
    got = _noalloc_backward(dk, x["q"], x["k"], x["v"], beta, g, valid, reset, ck, x["dO"], dF,
                            dS)
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_backward_matches_workspace_backward(dk):
    names = ("dq", "dk", "dv", "dbeta", "dg", "d_initial")
    for seed, (B, T, H) in ((1, (16, 512, 8)), (2, (2, 130, 3))):
        print(f"noalloc case B={B} T={T} H={H}", flush=True)
        ref, got = _case(dk, seed, B, T, H)
        for n, a, b in zip(names, got, ref):
            assert torch.equal(a, b), f"{n} (B={B} T={T} H={H}) differs from the workspace call"


def test_noalloc_rejects_shapes_above_the_scratch(dk):
    from delta_kernels import _shape
    from delta_kernels._lib import Gdn2Error, check, lib
    L = lib()
    q = torch.empty((64, 4096, 8, 64), dtype=torch.bfloat16, device="meta")
    shape = _shape(q, q)
    need = L.gdn_scalar_workspace_bytes(ctypes.byref(shape), 64)
    assert need > (64 << 20)
    rc = L.gdn_scalar_backward_noalloc(ctypes.byref(shape), 64, *([None] * 7), None, 0, None,
                                       None, None, None, None, None, None, None, None, None)
    with pytest.raises(Gdn2Error, match="scratch"):
        check("gdn_scalar_backward_noalloc", rc)
