"""ctypes binding of libgdn2_amd.so (declarations in include/gdn2.h).

Loading fails loudly when the library has not been built: there is no CPU or
eager-PyTorch fallback behind these functions.
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import torch

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "lib", "libgdn2_amd.so")

GDN2_F32 = 0
GDN2_BF16 = 1
GDN2_I32 = 2

STATUS = {0: "OK", 1: "ARGUMENT", 2: "SHAPE", 3: "DTYPE", 4: "WORKSPACE", 5: "LAUNCH"}


def raw_stream(device: torch.device) -> ctypes.c_void_p:
    """The handle of torch's current stream on device, for a library call."""
    idx = device.index
    if idx is None:
        idx = torch._C._cuda_getDevice()
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(idx))


def on_device(device: torch.device):
    """The context for a library call on device: none when device is already
    the current one (the common case: switching costs more than the call)."""
    idx = device.index
    if idx is None or idx == torch._C._cuda_getDevice():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


class Gdn2Shape(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("time", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("keys", ctypes.c_int64), ("values", ctypes.c_int64)]


class Gdn2View(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("stride", ctypes.c_int64 * 4)]


class Gdn2Error(RuntimeError):
    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn}: {STATUS.get(status, status)}: {message}")
        self.status = status


class Gdn2ConvShape(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("time", ctypes.c_int64),
                ("channels", ctypes.c_int64), ("taps", ctypes.c_int64)]


class Gdn2RowsShape(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("time", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("width", ctypes.c_int64)]


class Gdn2AdamwTensor(ctypes.Structure):
    _fields_ = [("param", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("first", ctypes.c_void_p),
                ("second", ctypes.c_void_p), ("numel", ctypes.c_int64)]


class Gdn2HolaShape(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("time", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("keys", ctypes.c_int64), ("values", ctypes.c_int64),
                ("capacity", ctypes.c_int32), ("chunk", ctypes.c_int32)]


class Gdn2LmMixerShape(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("time", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("keys", ctypes.c_int64), ("values", ctypes.c_int64), ("taps", ctypes.c_int64),
                ("z_stride", ctypes.c_int64)]


# Exported symbols and their signatures: (name, restype, argtypes).
_P = ctypes.c_void_p
_V = ctypes.POINTER(Gdn2View)
_S = ctypes.POINTER(Gdn2Shape)
_F = ctypes.c_void_p  # float*
_I = ctypes.c_int
_Z = ctypes.c_size_t
_L = ctypes.c_int64
_M = ctypes.POINTER(Gdn2LmMixerShape)
SIGNATURES = {
    "gdn2_abi_version": (_I, []),
    "gdn2_last_error": (ctypes.c_char_p, []),
    "gdn2_training_checkpoint_bytes": (_Z, [_S, _I]),
    "gdn2_training_workspace_bytes": (_Z, [_S, _I]),
    "gdn2_training_scan": (_I, [_S, _I] + [_V] * 9 + [_P, ctypes.c_int32, _F, _F, _P, _Z, _P]),
    "gdn2_training_backward": (_I, [_S, _I] + [_V] * 8 + [_P, _Z, _V, _F, _F] + [_P] * 3
                               + [_F] * 4 + [_P, _Z, _P]),
    "gdn2_scan_checkpoint_bytes": (_Z, [_S]),
    "gdn2_scan_workspace_bytes": (_Z, [_S]),
    "gdn2_scan": (_I, [_S] + [_V] * 8 + [_P, ctypes.c_int32, _P, _Z, _P]),
    "gdn2_backward": (_I, [_S] + [_V] * 8 + [_P, _Z, _V] + [_P] * 3 + [_F] * 3 + [_P, _Z, _P]),
    "gdn_scalar_checkpoint_bytes": (_Z, [_S, _I]),
    "gdn_scalar_workspace_bytes": (_Z, [_S, _I]),
    "gdn_scalar_scan": (_I, [_S, _I] + [_V] * 8 + [_P, ctypes.c_int32, _F, _F, _P, _Z, _P]),
    "gdn_scalar_backward": (_I, [_S, _I] + [_V] * 7 + [_P, _Z, _V, _F, _F] + [_P] * 3
                            + [_F] * 3 + [_P, _Z, _P]),
    "gdn_scalar_backward_noalloc": (_I, [_S, _I] + [_V] * 7 + [_P, _Z, _V, _F, _F] + [_P] * 3
                                    + [_F] * 3 + [_P]),
    "gdn2_decode_step": (_I, [_S] + [_V] * 8 + [_F, _P, ctypes.c_int32, _F, _P]),
    "gdn2_conv_forward": (_I, [ctypes.POINTER(Gdn2ConvShape)] + [_V] * 4 + [_I, _F, _P]),
    "gdn2_conv_workspace_bytes": (_Z, [ctypes.POINTER(Gdn2ConvShape)]),
    "gdn2_conv_backward": (_I, [ctypes.POINTER(Gdn2ConvShape)] + [_V] * 4 + [_I, _V, _F, _F, _P,
                                                                              _Z, _P]),
    "gdn2_norm_forward": (_I, [ctypes.POINTER(Gdn2RowsShape), _I, ctypes.c_float] + [_V] * 3
                          + [_F, _F, _P]),
    "gdn2_norm_workspace_bytes": (_Z, [ctypes.POINTER(Gdn2RowsShape)]),
    "gdn2_norm_backward": (_I, [ctypes.POINTER(Gdn2RowsShape), _I] + [_V] * 3 + [_F, _V]
                           + [_F] * 3 + [_P, _Z, _P]),
    "gdn2_decay_forward": (_I, [ctypes.POINTER(Gdn2RowsShape)] + [_V] * 3 + [_F, _P]),
    "gdn2_decay_workspace_bytes": (_Z, [ctypes.POINTER(Gdn2RowsShape)]),
    "gdn2_decay_backward": (_I, [ctypes.POINTER(Gdn2RowsShape)] + [_V] * 4 + [_F] * 3
                            + [_P, _Z, _P]),
    "gdn2_cross_entropy_forward": (_I, [ctypes.c_int64, ctypes.c_int64, _V, _P, ctypes.c_int64,
                                        _F, _F, _P]),
    "gdn2_cross_entropy_backward": (_I, [ctypes.c_int64, ctypes.c_int64, _V, _P, ctypes.c_int64,
                                         _F, _F, ctypes.c_int64, _P, _P]),
    "gdn2_cross_entropy_fused": (_I, [ctypes.c_int64, ctypes.c_int64, _V, _P, ctypes.c_int64,
                                      ctypes.c_float, _F, _P, _P]),
    "gdn2_adamw_workspace_bytes": (_Z, [ctypes.c_int32, ctypes.POINTER(Gdn2AdamwTensor)]),
    "gdn2_adamw_update": (_I, [ctypes.c_int32, ctypes.POINTER(Gdn2AdamwTensor), _I,
                               ctypes.c_int64, ctypes.c_double, ctypes.c_float, ctypes.c_float,
                               _I, _P, _Z, _P]),
    "gdn2_hola_schedule": (_I, [ctypes.POINTER(Gdn2HolaShape), _I] + [_V] * 3 + [_F, _P]),
    "gdn2_hola_checkpoint_bytes": (_Z, [ctypes.POINTER(Gdn2HolaShape)]),
    "gdn2_hola_read": (_I, [ctypes.POINTER(Gdn2HolaShape), _I] + [_V] * 7 + [_F, _F, _P, _Z, _P]),
    "gdn2_hola_workspace_bytes": (_Z, [ctypes.POINTER(Gdn2HolaShape)]),
    "gdn2_hola_backward": (_I, [ctypes.POINTER(Gdn2HolaShape)] + [_V] * 6 + [_P, _Z, _F, _V]
                           + [_F] * 4 + [_P, _Z, _P]),
    "gdn2_lm_norm_forward": (_I, [_L, _L, ctypes.c_float] + [_P] * 7),
    "gdn2_lm_norm_workspace_bytes": (_Z, [_L, _L]),
    "gdn2_lm_norm_backward": (_I, [_L, _L] + [_P] * 9 + [_Z, _P]),
    "gdn2_lm_mixer_in_forward": (_I, [_M] + [_P] * 10),
    "gdn2_lm_mixer_in_workspace_bytes": (_Z, [_M]),
    "gdn2_lm_mixer_in_backward": (_I, [_M] + [_P] * 16 + [_Z, _P]),
    "gdn2_lm_mixer_out_forward": (_I, [_M, _P, _P, _P, ctypes.c_float, _P, _P, _P]),
    "gdn2_lm_mixer_out_workspace_bytes": (_Z, [_M]),
    "gdn2_lm_mixer_out_backward": (_I, [_M] + [_P] * 9 + [_Z, _P]),
    "gdn2_lm_swiglu_forward": (_I, [_L, _L, _P, _P, _P]),
    "gdn2_lm_swiglu_backward": (_I, [_L, _L, _P, _P, _P, _P]),
    "gdn2_stage_timing": (_I, [_I]),
    "gdn2_stage_count": (_I, []),
    "gdn2_stage_name": (ctypes.c_char_p, [_I]),
    "gdn2_stage_ms": (ctypes.c_float, [_I]),
}

_lib = None


def lib():
    """Load the library (once).  Raises if it is missing or incomplete."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950). "
                "There is no fallback implementation.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, status: int):
    if status != 0:
        raise Gdn2Error(fn, status, lib().gdn2_last_error().decode())
