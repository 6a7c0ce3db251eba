"""The CPU oracle against the committed golden fixtures (tests/golden/).

Each case regenerates its seeded inputs (their sha256 must match the
fixture's) and reruns the oracle.  Outputs match to 1e-5 relative; on the
host the fixtures were written on they match bit for bit.  Arrays stored as
row subsets also compare their whole-array sum.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load():
    name = "qora_golden_fixtures"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, GOLDEN / "make_fixtures.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


F = _load()


@pytest.mark.parametrize("name", sorted(F.CASES))
def test_oracle_matches_golden(name):
    stored = dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))
    fresh = F.CASES[name]()
    assert str(fresh["inputs_sha256"]) == str(stored["inputs_sha256"]), "regenerated inputs differ"
    assert set(fresh) == set(stored)
    exact = True
    for key, want in stored.items():
        got = fresh[key]
        if key.endswith("__sha256") or key == "inputs_sha256":
            exact &= str(got) == str(want)
            continue
        if key.endswith("__rows"):
            assert np.array_equal(got, want)
            continue
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6, err_msg=f"{name}:{key}")
        exact &= np.array_equal(got, want)
    print(f"{name}: bit-identical to the fixture: {exact}")
