"""The single-environment workload on the HIP path against the reference's
own output: the MicroDuck-like biped (15 dynamic bodies, 14 hinges with
kp = 8, kd = 0.2, ground friction 0.8) held at the fixed HOME pose with zero
action, dt = 1/200 s, 10 AVBD iterations, 200 steps.

The expected values are tests/golden/kernel_standing_home_fp{64,32}.npz,
written by src/cuda/kernel.cuh itself (compiled in place by oracle/Makefile
and driven by tests/golden/make_golden.py) at steps 1, 2, 3, 10, 40, 100
and 200: the snapshot (kernel.cuh:555-575), the joint multipliers and
penalties, the compacted contact list with its warm-start data, the
colouring, generalized_loads (kernel.cuh:504-554) with a root offset of
(0.001, -0.002, 0.003), contact_forces and contact_counts.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from duck_gym_amd import CudaBatch
from parity_support import compare_env, contact_keys, fixture_state, rotation_angle

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
DT, ITER, KP, DEV = 0.005, 10, 8.0, "cuda:0"
OFFSET = (0.001, -0.002, 0.003)


def _run(bits, tmp_path):
    """Step one environment from reset(HOME) through the fixture's last
    checkpoint; yield (checkpoint index, step, batch) at each checkpoint."""
    f = np.load(GOLDEN / f"kernel_standing_home_fp{bits}.npz")
    model = tmp_path / "standing.duck"
    model.write_text(str(f["model"]))
    fp64 = bits == 64
    dtype = torch.float64 if fp64 else torch.float32
    batch = CudaBatch(model, 1, DT, ITER, 0, fp64)
    target = torch.tensor(f["targets"][None], dtype=dtype, device=DEV)
    batch.reset(torch.ones(1, dtype=torch.bool, device=DEV), target.clone(),
                torch.zeros(1, 6, dtype=dtype, device=DEV))
    forces = torch.zeros(1, 3, dtype=dtype, device=DEV)
    steps = list(f["step"])
    for s in range(1, steps[-1] + 1):
        batch.step(target, forces, 1, KP, float(f["limit"]))
        if s in steps:
            yield f, steps.index(s), s, batch


def test_fp64_matches_reference_kernel_output(tmp_path):
    """float64: the compacted contact lists (bodies, shapes, features, stick
    flags), colours and counts bit-exact at every checkpoint; poses, rotation
    angles, velocities, joint and contact multipliers, contact points,
    snapshot, joint torques and contact forces within 1e-9.  Joint penalties
    (stiffness ramps driven by |C|) are held to 1e-5 relative: at step 200 a
    difference of 3e-13 m in the poses shows up as 4e-6 in a ramp."""
    checked = 0
    for f, i, step, batch in _run(64, tmp_path):
        what = f"HOME fp64 step {step}"
        ref = fixture_state(f, i)
        gpu = batch.codec().decode(batch.export_state().cpu().numpy()[0])
        d = compare_env(gpu, ref, 1e-9, what, gates=dict(joint_penalty=1e-5))
        b, j, diag = (t.cpu().numpy()[0] for t in batch.state())
        np.testing.assert_allclose(b, f["bodies"][i], rtol=0, atol=1e-9, err_msg=what)
        np.testing.assert_allclose(j, f["joints"][i], rtol=0, atol=1e-9, err_msg=what)
        np.testing.assert_allclose(diag, f["diag"][i], rtol=0, atol=1e-9, err_msg=what)
        assert diag[2] == f["diag"][i][2] and diag[3] == f["diag"][i][3] and diag[5] == 0
        offset = torch.tensor([OFFSET], dtype=torch.float64, device=DEV)
        loads = batch.generalized_loads(offset).cpu().numpy()[0]
        np.testing.assert_allclose(loads, f["loads"][i], rtol=1e-9, atol=1e-9, err_msg=what)
        forces = batch.contact_forces().cpu().numpy()[0]
        np.testing.assert_allclose(forces, f["forces"][i], rtol=1e-9, atol=1e-9, err_msg=what)
        np.testing.assert_array_equal(batch.contact_counts().cpu().numpy()[0], f["counts"][i])
        np.testing.assert_allclose(batch.self_contact_stats().cpu().numpy()[0], f["stats"][i],
                                   rtol=0, atol=1e-12)
        assert len(ref["gc"]) == 8, "HOME stands on 2 feet x 4 points"
        print(f"{what}: x {d['x']:.2e} rot {d['rot']:.2e} lambda {d['joint_lambda']:.2e}")
        checked += 1
    assert checked == 7


def test_fp32_pose_tolerances_against_reference_kernel_output(tmp_path):
    """float32 against the reference's float32 output: body positions and
    rotation angles within 1e-5 m / 1e-5 rad over the first three steps and
    within 1e-3 at steps 10-200; hinge angles likewise; the compacted contact
    list (bodies, shapes, features, order, stick flags) identical after one
    step from the common reset state; at every checkpoint the contact count,
    the colours and the contact SET -- the (body, shape, feature) of every
    ground contact, in any order -- equal the reference's.  Later lists may
    differ in order only: the four lowest corners of a foot resting flat lie
    within float rounding of each other, and the reference takes them lowest
    first (kernel.cuh:338-364), so two float builds that round a height
    differently list the same corners in another order; the test counts the
    checkpoints where that happens."""
    worst = {}
    for f, i, step, batch in _run(32, tmp_path):
        what = f"HOME fp32 step {step}"
        ref = fixture_state(f, i)
        b, j, diag = (t.cpu().double().numpy()[0] for t in batch.state())
        tol = 1e-5 if step <= 3 else 1e-3
        dx = np.abs(b[:, :3] - ref["x"]).max()
        rot = rotation_angle(b[:, 3:7], ref["q"]).max()
        dj = np.abs(j[:, 0] - ref["joints"][:, 0]).max()
        assert dx <= tol and rot <= tol and dj <= tol, (what, dx, rot, dj)
        gpu = batch.codec().decode(batch.export_state().cpu().numpy()[0])
        same = contact_keys(gpu["gc"]) == contact_keys(ref["gc"])
        if step == 1:
            assert same, what
        corners = lambda entries: sorted(k[:3] for k in contact_keys(entries))  # noqa: E731
        assert corners(gpu["gc"]) == corners(ref["gc"]), (what, corners(gpu["gc"]),
                                                          corners(ref["gc"]))
        assert list(gpu["colors"]) == list(ref["colors"]) and gpu["colorCount"] == ref["colorCount"]
        assert diag[2] == ref["diag"][2] and diag[5] == 0
        worst[step] = (dx, rot, dj, same)
    print("fp32 HOME (x, rotation, hinge angle, same contact list in order) by step:",
          {s: tuple(f"{v:.2e}" for v in w[:3]) + (w[3],) for s, w in worst.items()})
    print("checkpoints with the same contact set in another order:",
          [s for s, w in worst.items() if not w[3]])
