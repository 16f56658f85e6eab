"""Scan boundary: ScanInput/ScanOutput and the explicit backend selector.

Mirrors crates/mixers/src/chunk.rs:8-124 and the selector enums of
crates/mixers/src/lib.rs:39-85.  Dispatch is explicit and never falls back:
`fused_gdn2` (the reference's GDN-2 GPU selector) and its MI355X name
`hip_gdn2` both run libgdn2_amd.so; `tensor_solver` (the reference's Burn
tensor program) and the KronLSTM selectors are not part of this build and
raise instead of silently substituting another implementation.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Optional

import torch

import delta_kernels

MAX_CHUNK_SIZE = 64  # reference: 16 (chunk.rs:6); the HIP kernels accept 1..=64


class MixerKind(str, enum.Enum):
    GDN2 = "gdn2"
    KRON_LSTM = "kron_lstm"


class ScanBackend(str, enum.Enum):
    TENSOR_SOLVER = "tensor_solver"
    FUSED_GPU = "fused_gpu"
    FUSED_PARALLEL128 = "fused_parallel128"
    FUSED_PARALLEL256 = "fused_parallel256"
    FUSED_GDN2 = "fused_gdn2"
    HIP_GDN2 = "hip_gdn2"

    def is_tensor_solver(self) -> bool:
        return self is ScanBackend.TENSOR_SOLVER

    def supports(self, kind: MixerKind) -> bool:
        if self in (ScanBackend.FUSED_GDN2, ScanBackend.HIP_GDN2):
            return kind is MixerKind.GDN2
        if self is ScanBackend.TENSOR_SOLVER:
            return True
        return kind is MixerKind.KRON_LSTM

    def is_fused(self) -> bool:
        return not self.is_tensor_solver()

    def partitions(self) -> int:
        return {ScanBackend.FUSED_PARALLEL128: 2, ScanBackend.FUSED_PARALLEL256: 4}.get(self, 1)

    def training_algorithm(self) -> str:
        """Run-report label.  `fused_gdn2` keeps the reference's label (run reports
        compare by it); the explicit MI355X selector names its own kernels."""
        return {
            ScanBackend.TENSOR_SOLVER: "differentiable_chunk_tensor_solver",
            ScanBackend.FUSED_GPU: "fused_kron_gpu",
            ScanBackend.FUSED_PARALLEL128: "fused_kron_parallel128_gpu",
            ScanBackend.FUSED_PARALLEL256: "fused_kron_parallel256_gpu",
            ScanBackend.FUSED_GDN2: "fused_gdn2_gpu",
            ScanBackend.HIP_GDN2: "fused_gdn2_mi355x_hip",
        }[self]


@dataclass
class ScanInput:
    """chunk.rs:8-18.  erase/write are channel-wise for GDN-2."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    alpha: torch.Tensor
    erase: torch.Tensor
    write: torch.Tensor


@dataclass
class ScanOutput:
    """chunk.rs:20-26.  scores: norm of the active edit after decay."""
    output: torch.Tensor
    final_state: torch.Tensor
    scores: torch.Tensor


def assert_fused_device(device: torch.device):
    """chunk.rs:110-124: fused selection requires a GPU device, no CPU fallback."""
    if torch.device(device).type != "cuda":
        raise RuntimeError("fused GPU scan requires a GPU device; no CPU fallback")


def scan_selected(backend: ScanBackend, kind: MixerKind, input: ScanInput, valid: torch.Tensor,
                  reset: torch.Tensor, chunk_size: int,
                  initial: Optional[torch.Tensor] = None) -> ScanOutput:
    """Explicit dispatch (chunk.rs:28-108).  Requesting fused execution never
    falls back to another implementation."""
    backend = ScanBackend(backend)
    kind = MixerKind(kind)
    if backend in (ScanBackend.FUSED_GDN2, ScanBackend.HIP_GDN2):
        if kind is not MixerKind.GDN2:
            raise ValueError("fused_gdn2 requires GDN-2")
        assert_fused_device(input.q.device)
        if not 1 <= chunk_size <= MAX_CHUNK_SIZE:
            raise ValueError(f"computational chunk_size must be 1..={MAX_CHUNK_SIZE}")
        r = delta_kernels.gdn_training_scan(input.q, input.k, input.v, input.alpha, input.erase,
                                            input.write, valid, reset, initial, chunk_size)
        return ScanOutput(r.output, r.final_state, r.scores)
    if backend is ScanBackend.TENSOR_SOLVER:
        raise NotImplementedError(
            "tensor_solver is the reference's Burn tensor program; this build provides the "
            "MI355X kernels only (select fused_gdn2 / hip_gdn2)")
    raise NotImplementedError(f"{backend.value} selects a KronLSTM kernel, which is not part of "
                              "this build")


def scan(kind: MixerKind, input: ScanInput, valid, reset, chunk_size: int,
         initial: Optional[torch.Tensor] = None) -> ScanOutput:
    """chunk.rs:129-135 entry point, routed to the MI355X kernels."""
    return scan_selected(ScanBackend.HIP_GDN2, kind, input, valid, reset, chunk_size, initial)
