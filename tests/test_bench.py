"""bench.py's CPU baseline leg: the reference's own CPU build timed on this
host (batch, single env in float64, and solver.cpp's CLI), with the host
facts, and a loud failure when that build is missing."""

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402

REF = ROOT / "oracle" / "_ref"


@pytest.mark.skipif(not any(REF.glob("_duck_reference*.so")), reason="reference build absent")
def test_cpu_baseline_fields(models, home):
    line = bench.cpu_baseline(models["standing"], home, seconds_budget=0.2)
    assert line["kind"] == "reference" and line["unit"] == "env-steps/s" and line["value"] > 0
    assert 1 <= line["cores"] <= 64 and "4096 envs" in line["sample"]
    host = line["host"]
    assert host["nproc"] >= 1 and host["cpu_model"] and "g++" in host["compiler"]
    assert "-ffp-contract=off" in host["flags"]
    assert line["single_env_fp64"]["steps"] == 200 and line["single_env_fp64"]["value"] > 0
    solver = line["solver_cpp"]
    assert solver["root_displacement_m"] > 10 and solver["unconverged_steps"] == 200


def test_cpu_baseline_requires_the_reference_build(models, home, monkeypatch):
    monkeypatch.setattr(bench, "ROOT", ROOT / "tests" / "golden")  # no oracle/_ref there
    monkeypatch.setitem(sys.modules, "_duck_reference", None)
    with pytest.raises(RuntimeError, match="reference CPU build is missing"):
        bench.cpu_baseline(models["standing"], np.asarray(home), seconds_budget=0.1)
