import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


GOLDEN = os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="session")
def golden_cases():
    import numpy as np

    cases = {}
    for f in sorted(os.listdir(GOLDEN)):
        if f.endswith(".npz"):
            with np.load(os.path.join(GOLDEN, f), allow_pickle=False) as z:
                if "qtype" in z.files:  # matmul cases (the GGUF fixture has its own test)
                    cases[f[:-4]] = {key: z[key] for key in z.files}
    assert cases, "no golden fixtures found"
    return cases
