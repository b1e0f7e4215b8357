"""The committed golden fixtures still match the oracle (regression pin, CPU only)."""

import importlib.util
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent / "golden"
spec = importlib.util.spec_from_file_location("make_golden", HERE / "make_golden.py")
make_golden = importlib.util.module_from_spec(spec)
spec.loader.exec_module(make_golden)


@pytest.mark.parametrize("name", sorted(make_golden.MAKERS))
def test_fixture_is_reproduced(name):
    stored = np.load(HERE / f"{name}.npz")
    fresh = make_golden.MAKERS[name]()
    assert sorted(stored.files) == sorted(fresh)
    for key, value in fresh.items():
        assert np.array_equal(stored[key], value), f"{name}.{key} drifted"
