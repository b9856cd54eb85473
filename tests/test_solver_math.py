"""The float solver's own math forms (duck_gym_amd/csrc/avbd_math.hpp),
built for the host and checked against closed forms: the fitted atan2, the
small-rotation series of exp/log and of the SO(3) log-Jacobian coefficient
(kernel.cuh:136-160, 841-850), that the fused helpers reduce, in double,
to the reference's operations in the same order (bitwise), and that the
ground passes' 5 mm duplicate test decides as the host's float hypot does
(kernel.cuh:601-653), and that the float block solve's own forms -- the
L D L^T factorisation and the sparse rotational Jacobian -- agree with the
reference's Cholesky solve and general form (kernel.cuh:177-228, 851-857)."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def probe(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc absent")
    out = tmp_path_factory.mktemp("math") / "probe"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "--offload-host-only",
                    f"-I{ROOT / 'duck_gym_amd' / 'csrc'}", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "native" / "solver_math_probe.cpp"), "-o", str(out)],
                   check=True, capture_output=True)
    text = subprocess.run([str(out)], check=True, capture_output=True, text=True).stdout
    return {k: float(v) for k, v in (line.split() for line in text.splitlines())}


def test_fitted_atan2(probe):
    # about one float ulp at pi (2.4e-7), signed zeros and axes exact to that
    assert probe["atan2_max_error"] < 4e-7
    assert probe["atan2_special_error"] < 4e-7


def test_small_rotation_series(probe):
    assert probe["expmap_max_error"] < 3e-7
    assert probe["logmap_max_error"] < 3e-7
    assert probe["logjac_max_rel_error"] < 1e-6


def test_fused_forms_are_the_reference_operations_in_double(probe):
    assert probe["double_fused_mismatches"] == 0


def test_five_mm_duplicate_test_matches_host_hypot(probe):
    assert probe["five_mm_mismatches"] == 0


def test_float_block_solve_matches_cholesky(probe):
    # float rounding of systems with condition numbers up to ~1e3
    assert probe["solve6_float_rel_error"] < 2e-3
    assert probe["solve6_indefinite_nan"] == 6


def test_sparse_rotation_jacobian(probe):
    assert probe["rotation_jacobian_max_error"] < 1e-15
