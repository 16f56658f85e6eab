"""Loading the committed golden vectors (tests/golden/*.npz)."""
from __future__ import annotations

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ("cfg0", "reset_padding", "gate_t7")


def load(name):
    """(inputs, expected) dicts of one golden file."""
    with np.load(os.path.join(GOLDEN, f"{name}.npz")) as z:
        inputs = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
        expected = {k[4:]: z[k] for k in z.files if k.startswith("out_")}
    return inputs, expected
