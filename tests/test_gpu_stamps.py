"""A step writes the drive parameters (kp, maxTorque, torque, frictionloss,
damping) and the colouring back to the state only when they change; the
state records what those blob fields hold (`drive`, `modelColours`).  These
tests check that every launch still leaves the fields exactly as a step that
rewrote them would (kernel.cuh:448-466 setTargets/setMotor, 596-598 and
717-720 colours): after target launches with equal and changed kp and limit,
motor launches, held launches and imports whose bytes contradict the record.
"""

import numpy as np
import pytest
import torch

from duck_gym_amd import CudaBatch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT, ITER = 0.005, 10
DRIVE = ("kp", "maxTorque", "torque", "frictionloss", "damping")


def _reset_home(batch, home):
    n = batch.num_envs
    batch.reset(torch.ones(n, dtype=torch.bool, device=DEV),
                torch.tensor(np.tile(home, (n, 1)), dtype=torch.float32, device=DEV),
                torch.zeros(n, 6, device=DEV))


def _drive(batch):
    """[E, J (all slots), 5] drive fields and [E, B (all slots)] colours, raw."""
    codec = batch.codec()
    L, J, B = codec.L, codec.L["J"], codec.L["B"]
    raw = batch.export_state().cpu().numpy()
    drive = np.stack([raw[:, L[f]: L[f] + 4 * J].copy().view(np.float32) for f in DRIVE], axis=-1)
    colours = raw[:, L["colors"]: L["colors"] + 4 * B].copy().view(np.int32)
    return drive, colours


def _expected_target(defaults, nj, kp, limit):
    e = np.zeros_like(defaults)
    e[:, :nj, 0] = np.float32(kp)
    e[:, :nj, 1] = np.float32(limit)
    e[:, :nj, 2:] = defaults[:, :nj, 2:]
    return e


def test_drive_fields_after_every_kind_of_launch(models, home):
    n = 8
    b = CudaBatch(models["friction"], n, DT, ITER)
    nj = b.num_joints
    _reset_home(b, home)
    defaults, model_colours = _drive(b)
    assert np.all(defaults[:, :nj, 3] == np.float32(0.02))
    forces = torch.zeros(n, 3, device=DEV)
    rng = np.random.default_rng(5)

    def target(kp, limit):
        t = torch.tensor(home + rng.uniform(-0.2, 0.2, (n, nj)), dtype=torch.float32, device=DEV)
        b.step(t, forces, 1, kp, limit)
        return _drive(b)

    def motor():
        m = torch.tensor(np.stack([rng.uniform(-0.1, 0.1, (n, nj)), rng.uniform(0, 0.02, (n, nj)),
                                   rng.uniform(0, 0.05, (n, nj))], axis=-1),
                         dtype=torch.float32, device=DEV)
        b.step_motor(m, forces)
        want = np.zeros_like(defaults)
        want[:, :nj, 2:] = m.cpu().numpy()
        return _drive(b), want

    for kp, limit in ((8.0, 0.0), (8.0, 0.0), (4.0, 0.3), (4.0, 0.3), (4.0, 0.0)):
        (got, colours) = target(kp, limit)
        assert np.array_equal(got, _expected_target(defaults, nj, kp, limit)), (kp, limit)
        assert np.array_equal(colours, model_colours)
    for _ in range(2):
        (got, _), want = motor()
        assert np.array_equal(got, want)
    before = got
    b.advance(2)
    assert np.array_equal(_drive(b)[0], before)
    got, _ = target(4.0, 0.0)
    assert np.array_equal(got, _expected_target(defaults, nj, 4.0, 0.0))
    b.advance(1)
    assert np.array_equal(_drive(b)[0], got)


def test_import_clears_records_the_bytes_contradict(models, home):
    n = 4
    b = CudaBatch(models["friction"], n, DT, ITER)
    nj = b.num_joints
    _reset_home(b, home)
    forces = torch.zeros(n, 3, device=DEV)
    t = torch.tensor(np.tile(home, (n, 1)), dtype=torch.float32, device=DEV)
    b.step(t, forces, 1, 8.0, 0.0)
    defaults, model_colours = _drive(b)
    # export -> import of the same batch is the identity
    raw = b.export_state()
    b.import_state(raw.clone())
    assert torch.equal(b.export_state(), raw)
    # env 0: a kp and a colour the record does not cover
    codec = b.codec()
    host = raw.cpu().numpy()
    s = codec.decode(host[0])
    s["kp"] = s["kp"].copy()
    s["kp"][3] = 7.0
    s["colors"] = s["colors"].copy()
    s["colors"][2] = 5
    codec.encode(host[0], s)
    b.import_state(torch.tensor(host, device=DEV))
    got, colours = _drive(b)
    assert got[0, 3, 0] == np.float32(7.0) and colours[0, 2] == 5
    # the same kp and limit as the record: env 0's fields are rewritten
    b.step(t, forces, 1, 8.0, 0.0)
    got, colours = _drive(b)
    assert np.array_equal(got, _expected_target(defaults, nj, 8.0, 0.0))
    assert np.array_equal(colours, model_colours)
