"""The committed golden vectors (tests/golden/*.npz) against the oracle that made them.

A change to the oracle's arithmetic that moves any output shows up here, on the
CPU; tests/test_gpu_golden.py holds the HIP library to the same vectors.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ["router", "fp4_dequant", "q2_dequant", "fp8", "requant"])
def test_oracle_reproduces_golden(name):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_fixtures", GOLDEN / "make_fixtures.py")
    mf = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mf)
    want = _load(name)
    got = mf.build(name)
    assert sorted(got) == sorted(want)
    for key, arr in want.items():
        g = np.asarray(got[key])
        assert g.dtype == arr.dtype and g.shape == arr.shape, key
        assert np.array_equal(g.view(np.uint8), arr.view(np.uint8)), key
