"""duck_reference_noalloc through the C ABI: the no-allocation variant of
duck_reference (CudaBatch.reference, extension.cu:385-415), whose state blob
and device inputs/outputs live in the library's static scratch.

Calls in a row on one device share that scratch, which keeps the previous
call's contents: a 20-body chain (the generic state, the larger blob), then
the MicroDuck-like biped (the smaller specialized blob), then the two-body
pendulum (the fewest inputs and outputs), then the chain again -- each equal
bit for bit to duck_reference on the same inputs, in float32 and float64."""

import ctypes

import numpy as np
import pytest
import torch

from duck_gym_amd import CudaBatch
from duck_gym_amd.native import library
from model_text import chain

pytestmark = pytest.mark.gpu
GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def _call(fn, batch, target, force, substeps, kp, limit):
    dt = np.float64 if batch.dtype == torch.float64 else np.float32
    t = np.ascontiguousarray(target, dtype=dt)
    f = np.ascontiguousarray(force, dtype=dt)
    b = np.full((batch.num_bodies, 13), np.nan, dt)
    j = np.full((batch.num_joints, 2), np.nan, dt)
    d = np.full(6, np.nan, dt)
    ptr = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
    code = fn(batch._h, ptr(t), ptr(f), int(substeps), float(kp), float(limit), ptr(b), ptr(j),
              ptr(d))
    assert code == 0, library().duck_last_error().decode()
    return b, j, d


@pytest.mark.parametrize("fp64", [False, True], ids=["fp32", "fp64"])
def test_noalloc_reference_equals_reference(tmp_path, models, home, fp64):
    lib = library()
    big = tmp_path / "chain.duck"
    # 19 links; 16 of them touch the ground
    big.write_text(chain(bodies=20, ground_flags=[1] * 16 + [0] * 3))
    rng = np.random.default_rng(5)
    cases = [(big, rng.uniform(-0.2, 0.2, 18), 6), (models["standing"], home, 5),
             (GOLDEN / "pendulum.duck", np.array([0.3]), 8), (big, rng.uniform(-0.2, 0.2, 18), 3)]
    for model, target, substeps in cases:
        batch = CudaBatch(model, 2, 0.005, 10, 0, fp64)
        force = np.array([0.1, -0.2, 0.0])
        torch.cuda.synchronize()
        want = _call(lib.duck_reference, batch, target, force, substeps, 8.0, 0.0)
        got = _call(lib.duck_reference_noalloc, batch, target, force, substeps, 8.0, 0.0)
        for w, g in zip(want, got):
            np.testing.assert_array_equal(g, w, err_msg=str(model))
        assert np.isfinite(got[0]).all() and got[2][5] == 0


def test_noalloc_reference_rejects_invalid_inputs(models):
    lib = library()
    batch = CudaBatch(models["standing"], 1, 0.005, 10, 0, False)
    t = np.zeros(14, np.float32)
    out = np.zeros(16 * 13 + 28 + 6, np.float32)
    ptr = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
    assert lib.duck_reference_noalloc(batch._h, ptr(t), ptr(t), 0, 8.0, 0.0, ptr(out), ptr(out),
                                      ptr(out)) != 0
    assert "Invalid CPU reference inputs" in lib.duck_last_error().decode()
    assert lib.duck_reference_noalloc(batch._h, ptr(t), None, 1, 8.0, 0.0, ptr(out), ptr(out),
                                      ptr(out)) != 0


def test_noalloc_largest_model_fits_and_allocates_nothing(tmp_path):
    """The largest state the loader admits -- 32 bodies, 30 hinges and 31
    ground shapes in float64, which runs the generic instance's blob (the
    largest blob) -- together with its inputs and outputs needs less than the
    64 KiB scratch, so no loadable model reaches the size rejection (it guards
    a future growth of the blob).  The call equals duck_reference bit for bit,
    and a warm call leaves the device's free memory unchanged."""
    lib = library()
    model = tmp_path / "chain32.duck"
    model.write_text(chain(bodies=32, ground_flags=[1] * 31))
    batch = CudaBatch(model, 1, 0.005, 10, 0, True)
    nb, nj = batch.num_bodies, batch.num_joints
    assert (nb, nj) == (32, 30)
    need = lib.duck_state_bytes(batch._h) + 8 * (6 + 3 * nj + 13 * nb)
    assert need <= 64 * 1024, need
    target = np.random.default_rng(9).uniform(-0.2, 0.2, nj)
    force = np.array([0.0, 0.1, 0.0])
    torch.cuda.synchronize()
    want = _call(lib.duck_reference, batch, target, force, 3, 8.0, 0.0)
    got = _call(lib.duck_reference_noalloc, batch, target, force, 3, 8.0, 0.0)
    for w, g in zip(want, got):
        np.testing.assert_array_equal(g, w)
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    again = _call(lib.duck_reference_noalloc, batch, target, force, 3, 8.0, 0.0)
    free_after = torch.cuda.mem_get_info()[0]
    assert free_after == free_before, (free_before, free_after)
    for w, g in zip(want, again):
        np.testing.assert_array_equal(g, w)
