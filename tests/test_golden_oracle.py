"""The CPU oracle reproduces the committed golden fixtures (CPU only)."""
import glob
import os

import numpy as np
import pytest

import frnn_oracle as O
from conftest import ROOT

FILES = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "*.npz")))


def test_fixtures_present():
    assert len(FILES) >= 7


@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_fixture(path):
    z = np.load(path)
    X, K, r = z["X"], int(z["K"]), float(z["radius"])
    assert O.plan(len(X), X.shape[1], K, r)["path"] == str(z["path"])
    idx, dist = O.search(X, K, r)
    assert np.array_equal(idx, z["idx"])
    assert np.array_equal(dist.view(np.uint32), z["dist"].view(np.uint32))
