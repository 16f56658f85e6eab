"""The committed golden vectors (tests/golden/) against the generators that
made their inputs and the f64 oracle that made their outputs.

Inputs must regenerate bit-exactly (SplitMix64 seed 0 for BASELINE configs[0];
the fixture restatements of crates/mixers/src/chunk_tests.rs:25-75 and
kron_checks.rs:124-188), and the oracle must reproduce every stored output to
float32 rounding.  A change of generator or oracle that moves any of them fails
here before it can move the GPU parity tests that read the same files.
"""
import os
import sys

import numpy as np
import pytest

from golden_util import NAMES, load

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden as mg  # noqa: E402


@pytest.fixture(scope="module")
def made():
    return mg.fixtures()


@pytest.mark.parametrize("name", NAMES)
def test_golden_inputs_regenerate(made, name):
    inputs, _ = load(name)
    fresh, _ = made[name]
    assert sorted(inputs) == sorted(fresh)
    for k in inputs:
        assert np.array_equal(np.asarray(fresh[k]), inputs[k]), f"{name}: input {k} changed"


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(made, name):
    inputs, expected = load(name)
    _, fn = made[name]
    got = fn(inputs)
    assert sorted(got) == sorted(expected)
    for k, ref in expected.items():
        x = np.asarray(got[k], np.float64).reshape(ref.shape)
        ref = ref.astype(np.float64)
        scale = np.sqrt(np.mean(ref * ref)) if ref.size else 0.0
        # stored values are the f64 results rounded to float32: 2^-24 relative
        assert np.all(np.abs(x - ref) <= 1.2e-7 * (np.abs(ref) + 1e-6 * scale) + 1e-30), \
            f"{name}: {k} differs from the golden value"


def test_golden_files_are_small():
    total = sum(os.path.getsize(os.path.join(HERE, "golden", f"{n}.npz")) for n in NAMES)
    assert total < 2 << 20
