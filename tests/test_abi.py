"""CPU checks of the C-ABI boundary: the library loads, exports every symbol
include/gdn2.h declares, and rejects bad arguments before launching anything
(no GPU work is started by these calls)."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "gdn2.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"GDN2_API\s+(?:const\s+char\s*\*|int|size_t)\s*(\w+)\(", text)))


@pytest.fixture(scope="module")
def L():
    from delta_kernels import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libgdn2_amd.so not built")
    return _lib.lib()


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "gdn2_training_scan" in syms and "gdn2_training_backward" in syms
    assert len(syms) >= 10


def test_library_exports_all_declared_symbols(L):
    from delta_kernels import _lib
    for s in declared_symbols():
        assert hasattr(L, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"


def test_abi_version(L):
    assert L.gdn2_abi_version() == 101


def _shape(B=2, T=8, H=2, K=32, V=64):
    from delta_kernels._lib import Gdn2Shape
    return Gdn2Shape(B, T, H, K, V)


def _view(dtype=0, data=0x1000):
    from delta_kernels._lib import Gdn2View
    v = Gdn2View()
    v.data = data
    v.dtype = dtype
    return v


def _scan(L, shape, chunk=16, qdtype=0, gdtype=0, ck_bytes=None, out_dtype=0, nulls=(), ck=0x5000):
    vs = [_view(qdtype)] * 3 + [_view(gdtype)] * 3 + [_view(0)] * 2
    vs = [(_view(v.dtype, 0) if i in nulls else v) for i, v in enumerate(vs)]
    init = _view(0, 0)
    size = L.gdn2_training_checkpoint_bytes(ctypes.byref(shape), chunk) if ck_bytes is None \
        else ck_bytes
    return L.gdn2_training_scan(ctypes.byref(shape), chunk, *[ctypes.byref(v) for v in vs],
                                ctypes.byref(init), ctypes.c_void_p(0x2000), out_dtype,
                                ctypes.c_void_p(0x3000), ctypes.c_void_p(0x4000),
                                ctypes.c_void_p(ck), size, None)


@pytest.mark.parametrize("shape,msg", [((0, 8, 2, 32, 64), "nonempty"),
                                       ((2, 0, 2, 32, 64), "nonempty"),
                                       ((2, 8, 2, 0, 64), "widths"),
                                       ((2, 8, 2, 32, 129), "widths")])
def test_rejects_bad_shapes(L, shape, msg):
    rc = _scan(L, _shape(*shape), ck_bytes=1 << 30)
    assert rc == 2
    assert msg in L.gdn2_last_error().decode()


def test_rejects_bad_chunk(L):
    assert _scan(L, _shape(), chunk=0, ck_bytes=1 << 30) == 1
    assert _scan(L, _shape(), chunk=65, ck_bytes=1 << 30) == 1
    assert "chunk" in L.gdn2_last_error().decode()


def test_rejects_dtype_mismatch(L):
    assert _scan(L, _shape(), gdtype=1) == 3  # gates must be F32
    assert "alpha" in L.gdn2_last_error().decode()
    assert _scan(L, _shape(), out_dtype=7) == 3


def test_rejects_null_inputs(L):
    assert _scan(L, _shape(), nulls=(1,)) == 1
    assert "k: data is null" in L.gdn2_last_error().decode()


def test_rejects_small_checkpoint(L):
    s = _shape()
    need = L.gdn2_training_checkpoint_bytes(ctypes.byref(s), 16)
    assert need > 0
    assert _scan(L, s, ck_bytes=need - 1) == 4
    assert "checkpoint" in L.gdn2_last_error().decode()


def test_rejects_misaligned_checkpoint(L):
    """The chunk kernels read the checkpoint with 16-byte loads."""
    assert _scan(L, _shape(), ck=0x5004) == 1
    assert "16-byte aligned" in L.gdn2_last_error().decode()


def test_workspace_sizes_scale(L):
    a = L.gdn2_training_workspace_bytes(ctypes.byref(_shape(B=2)), 16)
    b = L.gdn2_training_workspace_bytes(ctypes.byref(_shape(B=4)), 16)
    assert b == 2 * a > 0
    assert L.gdn2_training_workspace_bytes(ctypes.byref(_shape(B=0)), 16) == 0
