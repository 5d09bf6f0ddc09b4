"""Shared test setup: repo on sys.path, the ``gpu`` marker, golden tables."""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden" / "tables.json"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def golden_cases():
    with open(GOLDEN) as handle:
        return json.load(handle)["cases"]


def golden_tables(family, param=1.0, mean=0.0, zero_prob=0.0):
    """(encode int32[256], decode int32[1024], rare_length) from the fixtures."""
    for case in golden_cases():
        if (case["family"], case["param"], case["mean"], case["zero_prob"]) == (
                family, param, mean, zero_prob):
            return (np.array(case["encode"], dtype=np.int32),
                    np.array(case["decode"], dtype=np.int32), int(case["rare_length"]))
    raise KeyError((family, param, mean, zero_prob))


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle
