"""Shared pytest setup: the `gpu` marker, import paths and golden fixtures."""

import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
for path in (ROOT, ROOT / "tests"):   # the package, oracle/ and the test helper modules
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP (MI355X) device")


@pytest.fixture(scope="session")
def reference_vectors():
    return dict(np.load(GOLDEN / "reference_vectors.npz", allow_pickle=False))


@pytest.fixture(scope="session")
def hip_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def fixture_config(vectors, name):
    """The Config that make_reference_vectors.py ran case ``name`` with (stored as JSON)."""
    from memfast_amd import Config, Nonidealities

    stored = json.loads(str(vectors[f"case_{name}_config"]))
    kwargs = {k: tuple(v) if isinstance(v, list) else v for k, v in stored["config"].items()}
    return Config(**kwargs, nonidealities=Nonidealities(**stored["nonidealities"]))
