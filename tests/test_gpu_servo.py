"""The BAM servo substep on the GPU against the CPU oracle: the actuator
channels on seeded contact states in float64 (to rounding), the
ring-buffered delay and torque history, and the whole servo loop over 40
substeps with a 2-substep lag in float64 and float32, through the unfused
path (servoKernel, the implicit motor step, the queries) and the fused one
(one launch per substep, duck_servo_substep): the two are bit-identical in
the physics, and the refresh quantities of the fused launch match a float64
restatement of bam_env.py:128-155 (bam_env.py:307-337, actuator.py:16-77)."""

import numpy as np
import pytest
import torch

from duck_gym_amd import CudaBatch
from duck_gym_amd.microduck import model_text
from duck_gym_amd.servo import SYNTHETIC_SUPPLY, SYNTHETIC_XL330, ServoLoop, servo_params
from oracle import task_oracle as T
from oracle.oracle import Oracle
from oracle.servo_oracle import ServoOracle, xl330_m6
from parity_support import rotation_angle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT, ITER = 0.005, 10
OFFSET = np.array([0.002, -0.001, 0.004])


def _targets(home, n, seed):
    rng = np.random.default_rng(seed)
    return home + rng.uniform(-0.3, 0.3, (n, 14))


def _batch(model, home, n, fp64, seed=0):
    dt = torch.float64 if fp64 else torch.float32
    b = CudaBatch(model, n, DT, ITER, 0, fp64)
    q = torch.tensor(np.tile(home, (n, 1)), dtype=dt, device=DEV)
    b.reset(torch.ones(n, dtype=torch.bool, device=DEV), q, torch.zeros(n, 6, dtype=dt, device=DEV))
    return b


def test_actuator_channels_match_oracle_fp64(models, home):
    n = 16
    b = _batch(models["selfc"], home, n, True)
    targets = torch.tensor(_targets(home, n, 4), device=DEV)
    forces = torch.zeros(n, 3, dtype=torch.float64, device=DEV)
    for _ in range(20):  # reach a state with ground and body contacts
        b.step(targets, forces, 1, 8.0, 0.0)
    params = servo_params(**SYNTHETIC_SUPPLY, lag=0)
    rng = np.random.default_rng(9)
    prev_motor = torch.tensor(rng.uniform(-0.5, 0.5, (n, 14)), device=DEV)
    prev_applied = torch.tensor(rng.uniform(-0.5, 0.5, (n, 14)), device=DEV)
    pm, pa = prev_motor.cpu().numpy(), prev_applied.cpu().numpy()
    history = torch.zeros(1, n, 14, dtype=torch.float64, device=DEV)
    initialized = torch.zeros(n, dtype=torch.bool, device=DEV)
    offset = torch.tensor(np.tile(OFFSET, (n, 1)), device=DEV)
    supply = torch.empty(n, dtype=torch.float64, device=DEV)
    cmd = targets + 0.05
    motor = b.servo(params, cmd, history, 0, initialized, offset, prev_motor, prev_applied,
                    supply)
    loads = b.generalized_loads(offset).cpu().numpy()
    joints = b.state()[1].cpu().numpy()
    expect, raw, sup = xl330_m6(cmd.cpu().numpy(), joints[:, :, 0], joints[:, :, 1], pm, pa,
                                -loads[:, :, 0] + loads[:, :, 1], parameters=SYNTHETIC_XL330,
                                **SYNTHETIC_SUPPLY)
    np.testing.assert_allclose(motor.cpu().numpy(), expect, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(prev_motor.cpu().numpy(), raw, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(prev_applied.cpu().numpy(), expect[:, :, 0], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(supply.cpu().numpy(), sup[:, 0], rtol=1e-15)
    assert bool(initialized.all())
    assert torch.equal(history[0], cmd)
    # The load pass saw body contacts, so the friction budgets are load dependent.
    assert float(b.contact_counts()[:, 1].sum()) > 0


@pytest.mark.parametrize("fused", [False, True], ids=["unfused", "fused"])
@pytest.mark.parametrize("fp64", [True, False])
def test_servo_loop_matches_oracle(models, home, fp64, fused):
    n, lag, steps = 6, 2, 40
    b = _batch(models["standing"], home, n, fp64)
    dt = torch.float64 if fp64 else torch.float32
    params = servo_params(**SYNTHETIC_SUPPLY, lag=lag)
    loop = ServoLoop(b, params, home, OFFSET, fused=fused)
    oracles = []
    for e in range(n):
        o = Oracle(models["standing"], DT, ITER, fp64)
        o.reset(home)
        oracles.append(ServoOracle(o, home, OFFSET, lag, parameters=SYNTHETIC_XL330,
                                   **SYNTHETIC_SUPPLY))
    plan = [_targets(home, n, 100 + k) for k in range(steps // 4)]
    for k in range(steps // 4):  # 4 substeps per control step
        loop.substeps(torch.tensor(plan[k], dtype=dt, device=DEV), 4)
        for e, so in enumerate(oracles):
            for _ in range(4):
                so.substep(plan[k][e])
    bodies = b.state()[0].cpu().double().numpy()
    # float32: poses within 1e-3 m / 1e-3 rad after 40 substeps (measured
    # 1.2e-5 m, 4.4e-4 rad); applied torque within 2e-3 N m (measured
    # 6.3e-4).  The actuator's position loop (kp_fw) turns pose rounding into
    # torque: the reference's own float32 build differs from its float64 build
    # by the same 6.2e-4 N m / 6.4e-3 relative here, so a 1e-4 relative torque
    # gate is not a float32 property of this loop.
    tol = 1e-9 if fp64 else 1e-3
    for e, so in enumerate(oracles):
        ref = so.o.snapshot()[0]
        np.testing.assert_allclose(bodies[e, :, :3], ref[:, :3], rtol=0, atol=tol)
        assert rotation_angle(bodies[e, :, 3:7], ref[:, 3:7]).max() <= tol
        np.testing.assert_allclose(loop.previous_applied[e].cpu().double().numpy(),
                                   so.previous_applied, rtol=0, atol=1e-9 if fp64 else 2e-3)
    assert loop.cursor == steps % (lag + 1)
    assert not bool(b.state()[2][:, 5].any())


def test_servo_reset_refills_the_ring(models, home):
    n = 4
    b = _batch(models["standing"], home, n, True)
    params = servo_params(**SYNTHETIC_SUPPLY, lag=3)
    loop = ServoLoop(b, params, home, OFFSET)
    t1 = torch.tensor(_targets(home, n, 1), device=DEV)
    loop.substeps(t1, 2)
    mask = torch.tensor([True, False, True, False], device=DEV)
    loop.reset(mask)
    assert not bool(loop.initialized[mask].any()) and bool(loop.initialized[~mask].all())
    assert float(loop.previous_motor[mask].abs().sum()) == 0.0
    t2 = torch.tensor(_targets(home, n, 2), device=DEV)
    loop.substeps(t2, 1)
    for e in (0, 2):  # a reset env's ring is refilled with the new target
        assert torch.equal(loop.history[:, e], t2[e].expand(4, -1))
    for e in (1, 3):  # others keep their history: one slot holds t2
        assert int((loop.history[:, e] == t2[e]).all(-1).sum()) == 1
    with pytest.raises(RuntimeError):
        b.servo(params, t2, loop.history, 4, loop.initialized, loop.root_offset,
                loop.previous_motor, loop.previous_applied)


SITES = [[0.012, 0.004, -0.006], [0.012, -0.004, -0.006]]


def _frame():
    meta = model_text(self_contact=True)[1]
    names = meta["body_names"]
    return meta["root_iquat"], [names.index("left_foot"), names.index("right_foot")]


@pytest.mark.parametrize("fp64", [False, True])
def test_fused_substep_equals_unfused(models, home, fp64):
    """One launch per substep against the reference loop's five calls and
    torch arithmetic, on the biped with body contacts: states, actuator
    history, motor channels, self-contact maxima, foot forces and the
    air/contact timers bit for bit; the root-frame and site quantities to
    rounding (torch evaluates the same formulas in another order)."""
    n, lag = 8, 2
    dt = torch.float64 if fp64 else torch.float32
    principal, feet = _frame()
    kw = dict(root_principal_quat=principal, feet=feet, foot_sites=SITES)
    params = servo_params(**SYNTHETIC_SUPPLY, lag=lag)
    a, b = _batch(models["selfc"], home, n, fp64), _batch(models["selfc"], home, n, fp64)
    # reach states with body-body contacts first (as the channel test does)
    warm = torch.tensor(_targets(home, n, 4), dtype=dt, device=DEV)
    zero = torch.zeros(n, 3, dtype=dt, device=DEV)
    for _ in range(20):
        for batch in (a, b):
            batch.step(warm, zero, 1, 8.0, 0.0)
    touched = int((b.contact_counts()[:, 1] > 0).sum())
    assert touched > 0, "no body-body contacts before the servo loop"
    fused = ServoLoop(a, params, home, OFFSET, fused=True, **kw)
    plain = ServoLoop(b, params, home, OFFSET, fused=False, **kw)
    tol = 1e-12 if fp64 else 2e-6
    contact_steps = 0
    for k in range(12):
        target = warm + torch.tensor(np.random.default_rng(200 + k).uniform(-0.05, 0.05, (n, 14)),
                                     dtype=dt, device=DEV)
        for loop in (fused, plain):
            loop.substeps(target, 4)
        assert torch.equal(a.export_state(), b.export_state()), f"control step {k}"
        for name in ("history", "initialized", "previous_motor", "previous_applied", "motor",
                     "self_contacts", "self_penetration", "contact_force", "air_time",
                     "contact_time"):
            assert torch.equal(getattr(fused, name), getattr(plain, name)), (name, k)
        for name in ("gravity", "ang_vel", "lin_vel", "origin_velocity", "site_pos", "site_vel"):
            diff = float((getattr(fused, name) - getattr(plain, name)).abs().max())
            assert diff <= tol, (name, k, diff)
        touched += int((b.contact_counts()[:, 1] > 0).sum())
        contact_steps += int(fused.contact.sum())
    assert touched > 0 and contact_steps > 0, (touched, contact_steps)
    assert fused.cursor == plain.cursor


@pytest.mark.parametrize("fp64", [False, True])
def test_fused_refresh_quantities(models, home, fp64):
    """The fused launch's refresh quantities against bam_env.py:128-155
    restated in float64 (task oracle quaternion maps) on the state it left,
    and its foot forces against duck_contact_forces(ground_only)."""
    n = 8
    dt = torch.float64 if fp64 else torch.float32
    principal, feet = _frame()
    params = servo_params(**SYNTHETIC_SUPPLY, lag=1)
    a = _batch(models["selfc"], home, n, fp64)
    loop = ServoLoop(a, params, home, OFFSET, root_principal_quat=principal, feet=feet,
                     foot_sites=SITES)
    tol = 1e-12 if fp64 else 3e-6
    for k in range(6):
        loop.substeps(torch.tensor(_targets(home, n, 300 + k), dtype=dt, device=DEV), 4)
        bodies = a.state()[0].cpu().double().numpy()
        q1 = bodies[:, 1, 3:7]
        root = T.quat_multiply(q1, np.asarray(principal) * np.array([1, -1, -1, -1]))
        down = np.broadcast_to([0.0, 0.0, -1.0], (n, 3))
        root_r = -T.inverse_rotate(q1 * np.array([1, -1, -1, -1]), np.broadcast_to(OFFSET, (n, 3)))
        origin = bodies[:, 1, 7:10] + np.cross(bodies[:, 1, 10:13], root_r)
        expect = dict(gravity=T.inverse_rotate(root, down),
                      ang_vel=T.inverse_rotate(root, bodies[:, 1, 10:13]),
                      origin_velocity=origin, lin_vel=T.inverse_rotate(root, origin))
        foot = bodies[:, feet]
        r = T.inverse_rotate(foot[:, :, 3:7] * np.array([1, -1, -1, -1]),
                             np.broadcast_to(SITES, (n, 2, 3)))
        expect["site_pos"] = foot[:, :, :3] + r
        expect["site_vel"] = foot[:, :, 7:10] + np.cross(foot[:, :, 10:13], r)
        for name, ref in expect.items():
            got = getattr(loop, name).cpu().double().numpy()
            np.testing.assert_allclose(got, ref, rtol=0, atol=tol, err_msg=f"{name} step {k}")
        assert torch.equal(loop.contact_force, a.contact_forces(ground_only=True)[:, feet])
    assert bool(loop.contact.any())
