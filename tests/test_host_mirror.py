"""Host-side mirror of the reference's scan selector (CPU only).

crates/mixers/src/lib.rs:39-85: MixerKind / ScanBackend with snake_case serde
names, supports(), is_fused(), partitions() and training_algorithm(); and
chunk.rs:29-124: explicit dispatch that never falls back.
"""
import pytest

torch = pytest.importorskip("torch")

from delta_mixers import MixerKind, ScanBackend  # noqa: E402


def test_serde_names_match_reference():
    assert [b.value for b in ScanBackend][:5] == [
        "tensor_solver", "fused_gpu", "fused_parallel128", "fused_parallel256", "fused_gdn2"]
    assert [k.value for k in MixerKind] == ["gdn2", "kron_lstm"]


def test_supports_and_labels_match_reference():
    ref = {  # lib.rs:55-85
        ScanBackend.TENSOR_SOLVER: (True, True, False, 1, "differentiable_chunk_tensor_solver"),
        ScanBackend.FUSED_GPU: (False, True, True, 1, "fused_kron_gpu"),
        ScanBackend.FUSED_PARALLEL128: (False, True, True, 2, "fused_kron_parallel128_gpu"),
        ScanBackend.FUSED_PARALLEL256: (False, True, True, 4, "fused_kron_parallel256_gpu"),
        ScanBackend.FUSED_GDN2: (True, False, True, 1, "fused_gdn2_gpu"),
    }
    for b, (gdn, kron, fused, parts, label) in ref.items():
        assert b.supports(MixerKind.GDN2) is gdn
        assert b.supports(MixerKind.KRON_LSTM) is kron
        assert b.is_fused() is fused
        assert b.partitions() == parts
        assert b.training_algorithm() == label
    hip = ScanBackend.HIP_GDN2
    assert hip.supports(MixerKind.GDN2) and not hip.supports(MixerKind.KRON_LSTM)
    assert hip.is_fused() and hip.partitions() == 1


def test_unbuilt_selectors_raise_instead_of_substituting():
    from delta_mixers import ScanInput, scan_selected
    x = torch.zeros(1, 2, 1, 4)
    inp = ScanInput(q=x, k=x, v=x, alpha=x, erase=x, write=x)
    m = torch.ones(1, 2)
    for b in (ScanBackend.TENSOR_SOLVER, ScanBackend.FUSED_GPU):
        with pytest.raises(Exception):
            scan_selected(b, MixerKind.GDN2, inp, m, m, 1, None)
    # a fused selector on CPU tensors is an error, never a CPU fallback
    with pytest.raises(Exception):
        scan_selected(ScanBackend.FUSED_GDN2, MixerKind.GDN2, inp, m, m, 1, None)
