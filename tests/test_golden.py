"""The committed fixtures are reproducible: regenerated inputs hash to the stored SHA-256, and the oracle
recomputes every stored output bit for bit."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import make_golden as G  # noqa: E402


@pytest.mark.parametrize("name", G.CASES)
def test_fixture_reproduces(name):
    fx = np.load(G.fixture_path(name))
    parts, C0, steps = G.case_inputs(name)
    assert str(fx["sha256"]) == G.sha(parts), "numpy's generator stream changed: regenerate the fixtures"
    assert np.array_equal(fx["C0"], C0) and int(fx["steps"]) == steps
    got = G.compute(name)
    for key in fx.files:
        assert np.array_equal(fx[key], got[key]), key
