"""The BAM servo substep on the GPU (servoKernel + the implicit motor step)
against the CPU oracle: the actuator channels on seeded contact states in
float64 (to rounding), the ring-buffered delay and torque history, and the
whole servo loop over 40 substeps with a 2-substep lag in float64 and
float32 (bam_env.py:307-337, actuator.py:16-77)."""

import numpy as np
import pytest
import torch

from duck_gym_amd import CudaBatch
from duck_gym_amd.servo import SYNTHETIC_SUPPLY, SYNTHETIC_XL330, ServoLoop, servo_params
from oracle.oracle import Oracle
from oracle.servo_oracle import ServoOracle, xl330_m6

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


@pytest.mark.parametrize("fp64", [True, False])
def test_servo_loop_matches_oracle(models, home, fp64):
    n, lag, steps = 6, 2, 40
    b = _batch(models["standing"], home, n, fp64)
    dt = torch.float64 if fp64 else torch.float32
    params = servo_params(**SYNTHETIC_SUPPLY, lag=lag)
    loop = ServoLoop(b, params, home, OFFSET)
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
    tol = 1e-9 if fp64 else 2e-3
    for e, so in enumerate(oracles):
        ref = so.o.snapshot()[0]
        np.testing.assert_allclose(bodies[e, :, :7], ref[:, :7], atol=tol)
        np.testing.assert_allclose(loop.previous_applied[e].cpu().double().numpy(),
                                   so.previous_applied, atol=tol if fp64 else 5e-2)
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
