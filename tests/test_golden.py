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


def test_adamw_fixture_matches_torch_adamw():
    # pins the stored trajectory itself (not only its reproducibility) to torch's AdamW
    import torch
    from golden_util import bf16
    d = load("adamw_3step")
    shapes = [(64, 32), (37,), (16, 9)]
    offs = [0, 2048, 2088]
    ps = [torch.nn.Parameter(torch.from_numpy(d[f"p{i}"]).clone()) for i in range(3)]
    opt = torch.optim.AdamW([{"params": [ps[0], ps[2]], "weight_decay": 0.1},
                             {"params": [ps[1]], "weight_decay": 0.0}],
                            lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    scale = 8.0
    for st in range(3):
        for i, p in enumerate(ps):
            p.grad = bf16(d[f"g{st}_{i}"]).float().view(shapes[i]) / scale
        torch.nn.utils.clip_grad_norm_(ps, 0.5)
        opt.step()
        m = torch.from_numpy(d[f"master{st}"])
        for p, o in zip(ps, offs):
            assert float((m[o:o + p.numel()] - p.detach().reshape(-1)).abs().max()) < 1e-6 * 0.4
        scale = float(d[f"scale{st}"])
