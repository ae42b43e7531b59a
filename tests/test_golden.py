"""The oracle reproduces the committed golden fixtures (CPU only).

The fixtures were written by tests/golden/make_golden.py from the oracle; this
test regenerates every case and compares, so any change to the oracle's
numerics shows up as a fixture mismatch.
"""
import os

import numpy as np
import pytest

from golden_util import GOLDEN_DIR, load

import importlib.util
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN_DIR, "make_golden.py"))
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)

CASES = make_golden.all_cases()


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    stored = load(name)
    fresh = CASES[name]
    assert sorted(stored) == sorted(fresh)
    for key, val in fresh.items():
        ref = stored[key]
        assert ref.dtype == np.asarray(val).dtype, (name, key)
        if np.issubdtype(ref.dtype, np.floating):
            np.testing.assert_allclose(np.asarray(val), ref, rtol=1e-6, atol=1e-7, err_msg=f"{name}:{key}")
        else:
            np.testing.assert_array_equal(np.asarray(val), ref, err_msg=f"{name}:{key}")
