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


def test_roofline_object_carries_bound_valu_and_occupancy():
    """The roofline of a bench line: the metric's HBM figures, the true bound
    (latency, not HBM), the FP32-VALU fraction from the recorded op counts of
    the workload, and the kernel's occupancy as passed in."""
    occupancy = {"vgprs": 256, "workgroups_per_cu": 4, "waves_per_simd": 1.0}
    r = bench.roofline(90e-6, 17.5e6, 4096, "home", occupancy, traffic=19.9e6)
    assert r["bound"] == "latency" and "neither" in r["bound_detail"]
    assert r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert abs(r["achieved"] - 17.5e6 / 90e-6 / 1e9) < 1e-9
    assert abs(r["frac"] - r["achieved"] / 8000.0) < 1e-12 and r["traffic"] == 19.9e6
    flop = bench.flop_per_env_step("home")
    assert 7e5 < flop < 1e6  # op_count at HOME, profiles/flop_counts.md
    v = r["valu"]
    assert abs(v["achieved_tflops"] - flop * 4096 / 90e-6 / 1e12) < 1e-9
    assert abs(v["frac"] - v["achieved_tflops"] / 157.3) < 1e-12
    assert abs(v["frac_nonpacked"] - v["achieved_tflops"] / 78.6) < 1e-12
    assert r["occupancy"] is occupancy
    for workload in ("sweep", "drop", "servo"):
        assert bench.flop_per_env_step(workload) > 0
    assert bench.roofline(1e-4, 1e6, 1, "no-such-workload", None)["valu"] is None


def test_servo_bytes_count_the_actuator_buffers():
    plain = 2 * bench.state_bytes_per_env(8)
    assert bench.servo_bytes_per_env(8, 0) > plain
    assert bench.servo_bytes_per_env(8, 1) - bench.servo_bytes_per_env(8, 0) == 2 * 68
