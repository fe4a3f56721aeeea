"""The committed golden fixtures (tests/golden/*.npz) reproduce bit for bit
from their seeded inputs through the oracle (CPU only)."""

import os

import numpy as np
import pytest

from golden import cases

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", sorted(cases.FIXTURES))
def test_fixture_reproduces(name):
    stored = np.load(os.path.join(HERE, name + ".npz"))
    fresh = cases.FIXTURES[name]()
    assert sorted(stored.files) == sorted(fresh)
    for key in stored.files:
        np.testing.assert_array_equal(stored[key], fresh[key], err_msg=f"{name}:{key}")
