"""Mixer-level mirror of delta-block-lm's scan dispatch (crates/mixers).

`chunk.scan_selected` is the boundary the reference's mixer, SBD paths,
benchmarks and numerical gates call (crates/mixers/src/chunk.rs:29-108);
here every GDN-2 selector routes to the MI355X HIP kernels.
"""
from .chunk import MixerKind, ScanBackend, ScanInput, ScanOutput, scan, scan_selected

__all__ = ["MixerKind", "ScanBackend", "ScanInput", "ScanOutput", "scan", "scan_selected"]
