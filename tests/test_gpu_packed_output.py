"""The reference's packed training-scan output through the C ABI.

GdnTrainingOps returns one f32 buffer [output ; final_state ; scores]
(crates/kernels/src/gdn_training_ops.rs:300-332).  include/gdn2.h documents
that passing output = packed, final_state = packed + B*T*H*V and scores =
packed + B*T*H*V + B*H*K*V with an f32 output reproduces that packing; this
test calls gdn2_training_scan both ways and requires the packed buffer's
three slices to equal the separate buffers bit for bit, on the
token-sequential kernels (f32, d = 32) and on the chunk kernels (bf16 q/k/v,
d = 64, f32 output), with the packed tail left untouched."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from gpu_util import dev  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import delta_kernels
    delta_kernels.lib()
    return delta_kernels


@pytest.mark.parametrize("dtype,D", [(torch.float32, 32), (torch.bfloat16, 64)])
def test_packed_output_layout(dk, dtype, D):
    B, T, H = 2, 37, 3
    rng = np.random.default_rng(D)
    k = rng.normal(size=(B, T, H, D))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    x = {"q": dev(0.3 * rng.normal(size=(B, T, H, D)), dtype), "k": dev(k, dtype),
         "v": dev(rng.normal(size=(B, T, H, D)), dtype),
         "alpha": dev(rng.uniform(0.8, 1.0, size=(B, T, H, D))),
         "erase": dev(rng.uniform(0.2, 0.9, size=(B, T, H, D))),
         "write": dev(rng.uniform(0.2, 0.9, size=(B, T, H, D)))}
    valid = np.ones((B, T), np.float32)
    valid[1, 30:] = 0
    reset = np.zeros((B, T), np.float32)
    reset[0, 17] = 1
    init = dev(0.1 * rng.normal(size=(B, H, D, D)))
    L = dk.lib()
    shape = dk._shape(x["q"], x["v"])
    nck = L.gdn2_training_checkpoint_bytes(ctypes.byref(shape), 16)
    keep = (x["q"], x["k"], x["v"], x["alpha"], x["erase"], x["write"], dev(valid), dev(reset),
            init)  # the views hold raw pointers: keep the tensors alive
    views = [dk._view(t) for t in keep]
    n_out, n_fin, n_sc = B * T * H * D, B * H * D * D, B * T * H

    def scan(out_p, fin_p, sc_p):
        ck = torch.empty((nck,), dtype=torch.uint8, device="cuda")
        rc = L.gdn2_training_scan(ctypes.byref(shape), 16, *[ctypes.byref(v) for v in views],
                                  out_p, 0, fin_p, sc_p, dk._ptr(ck), nck, dk._stream(x["q"]))
        assert rc == 0, L.gdn2_last_error()
        torch.cuda.synchronize()

    out = torch.empty(n_out, dtype=torch.float32, device="cuda")
    fin = torch.empty(n_fin, dtype=torch.float32, device="cuda")
    sc = torch.empty(n_sc, dtype=torch.float32, device="cuda")
    scan(dk._ptr(out), dk._ptr(fin), dk._ptr(sc))
    tail = 7
    packed = torch.full((n_out + n_fin + n_sc + tail,), 12345.0, dtype=torch.float32,
                        device="cuda")
    base = packed.data_ptr()
    scan(ctypes.c_void_p(base), ctypes.c_void_p(base + 4 * n_out),
         ctypes.c_void_p(base + 4 * (n_out + n_fin)))
    assert torch.equal(packed[:n_out], out)
    assert torch.equal(packed[n_out:n_out + n_fin], fin)
    assert torch.equal(packed[n_out + n_fin:n_out + n_fin + n_sc], sc)
    assert torch.all(packed[-tail:] == 12345.0), "the packed buffer's tail was written"
    assert torch.all(out.view(B, T, H, D)[1, 30:] == 0) and torch.all(sc.view(B, T, H)[1, 30:] == 0)
