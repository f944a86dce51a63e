"""The committed fixtures of tests/golden/ are exactly what the pinned oracle produces for their seeded inputs."""

import importlib.util

import numpy as np
import pytest

from conftest import GOLDEN

_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_fixture_matches_oracle(name):
    path = GOLDEN / f"{name}.npz"
    assert path.exists(), f"missing fixture {path}: run python tests/golden/make_golden.py"
    stored = np.load(path)
    fresh = make_golden.build(name)
    assert sorted(stored.files) == sorted(fresh)
    for k in fresh:
        assert stored[k].dtype == fresh[k].dtype and np.array_equal(stored[k], fresh[k]), (name, k)
