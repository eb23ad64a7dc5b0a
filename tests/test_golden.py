"""The committed golden fixtures (tests/golden/): regenerating them from their
seeds reproduces the stored inputs bit for bit and the stored outputs, so the
fixtures, the seeded generator and the oracle stay consistent."""

from __future__ import annotations

import numpy as np
import pytest

from golden import make_golden


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_fixture_reproduces(name):
    stored = make_golden.load(name)
    fresh = make_golden.make(name)
    for key, val in fresh.items():
        assert key in stored, key
        assert np.array_equal(stored[key], val), (name, key)
    assert np.all(np.isfinite(stored["expected"]))
