import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a GPU and the built HIP library (run on the MI355X box)")


@pytest.fixture(scope="session")
def golden():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "mask_golden.json")) as f:
        return json.load(f)["cases"]


@pytest.fixture(scope="session")
def golden_arrays():
    import numpy as np
    return np.load(os.path.join(ROOT, "tests", "golden", "mask_indices.npz"))


@pytest.fixture(scope="session")
def ref_tables():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "reference_tables.json")) as f:
        return json.load(f)
