"""Shared test fixtures: markers, synthetic models, the oracle, the GPU batch."""

import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

from duck_gym_amd.microduck import write_model  # noqa: E402

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available():
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def models(tmp_path_factory):
    """MicroDuck-like models: standing (v1), self-contact (v2), dry friction."""
    base = tmp_path_factory.mktemp("models")
    out = {
        "standing": write_model(base / "standing"),
        "selfc": write_model(base / "selfc", self_contact=True),
        "friction": write_model(base / "friction", frictionloss=0.02),
        "limp": write_model(base / "limp", kp=0.0, frictionloss=0.01),
    }
    out["pendulum"] = GOLDEN / "pendulum.duck"
    return out


@pytest.fixture(scope="session")
def home():
    from duck_gym_amd.microduck import HOME, JOINT_NAMES

    return np.array([HOME[n] for n in JOINT_NAMES])


def meta_of(model):
    return json.loads((Path(model).parent / "metadata.json").read_text())
