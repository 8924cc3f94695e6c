import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden_cases():
    import numpy as np
    with np.load(os.path.join(ROOT, "tests", "golden", "cases.npz")) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="session")
def bitexact_shapes():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "bitexact_shapes.json")) as f:
        return json.load(f)["shapes"]
