"""Shared pytest setup: repo root on sys.path, the ``gpu`` marker, fixture access."""
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_golden(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_meta(name=None):
    with open(os.path.join(GOLDEN, "index.json")) as f:
        idx = json.load(f)
    return idx if name is None else idx[name]


@pytest.fixture(scope="session")
def golden():
    return load_golden
