"""TensorEnv's gait-table options (gait, foot_clearance, load_transfer;
python/duck_gym/tensor_env.py:260-277, 338-357) against the task oracle's
restatement, on a synthetic gait.npz: a table per command direction of
HOME plus a smooth per-joint swing, period 0.8 s, lift 8 mm, the feet's
body-frame collision points.

Two environments run in lockstep from the same seed and actions: one with
the gait reference only, one with the reference and both shaping terms.  The
applied targets of both (formed inside the targets launch) equal the
oracle's gait reference at the episode counters before the step, and equal
bit for bit the reference's torch expressions on the same tensors; the
difference of their rewards (the shaping terms join the reward inside the
task launch, before the control period scales it, as in the reference)
equals the oracle's shaping terms evaluated on the GPU state after the step,
times the control period, wherever the env has not failed."""

import json

import numpy as np
import pytest
import torch

from duck_gym_amd.microduck import _links, qconj, qrot, write_model
from oracle import task_oracle as T

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
E = 64


@pytest.fixture(scope="module")
def gait_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("gait")
    write_model(d)
    meta = json.loads((d / "metadata.json").read_text())
    home = np.array(meta["home"])
    count = 16
    phase = np.arange(count) / count
    table = np.empty((4, count, 14))
    for k in range(4):
        swing = 0.15 * np.sin(2 * np.pi * (phase[:, None] + 0.1 * k + np.arange(14)[None] / 14))
        table[k] = home + swing
    names = meta["body_names"]
    feet = [names.index("left_foot"), names.index("right_foot")]
    # the feet's hull vertices in their body frames: each shape sits at its
    # body's centre of mass, in the frame conjugate to the body's HOME frame
    links = {l["name"]: l for l in _links()}
    points = np.array([[qrot(qconj(links[n]["frame"]), v) for v in links[n]["hull"]]
                       for n in ("left_foot", "right_foot")])
    np.savez(d / "gait.npz", targets=table, period=0.8, lift=0.008, speed=0.05,
             foot_collision_points=points, foot_bodies=np.array(feet))
    return d, meta, table, feet, points


def test_gait_reference_and_shaping_terms(gait_dir):
    from duck_gym_amd.tensor_env import TensorEnv

    d, meta, table, feet, points = gait_dir
    kw = dict(iterations=10, dt=0.005, substeps=4, seed=7, task="locomotion", gait=True,
              auto_reset=False, episode_seconds=2.0)
    shaped = TensorEnv(d, E, foot_clearance=True, load_transfer=True, **kw)
    plain = TensorEnv(d, E, **kw)
    home, dt = np.array(meta["home"]), shaped.control_dt
    rng = np.random.default_rng(3)
    checked = terms = 0
    for step in range(30):
        actions = torch.tensor(rng.uniform(-0.4, 0.4, (E, 14)), dtype=torch.float32, device=DEV)
        episode = shaped.episode_length_buf.cpu().numpy().copy()
        commands = shaped.commands.cpu().double().numpy()
        ref = T.gait_reference(episode, commands, table, 0.8, home, dt)
        _, expected = T.targets(actions.cpu().double().numpy(), home, np.array(meta["lower"]),
                                np.array(meta["upper"]), shaped.action_scale, ref)
        # the reference's torch expressions of the targets (tensor_env.py:
        # 263-283) on the same tensors: the targets launch repeats them bit
        # for bit
        torch_targets = [(env.reference() + env.action_scale * actions.clamp(-1, 1))
                         .clamp(env.lower, env.upper) for env in (plain, shaped)]
        _, r1, _, info1 = shaped.step(actions)
        _, r0, _, info0 = plain.step(actions)
        for info, want in zip((info0, info1), torch_targets):
            np.testing.assert_allclose(info["applied_targets"].cpu().double().numpy(), expected,
                                       rtol=0, atol=2e-6)
            assert torch.equal(info["applied_targets"], want), f"step {step}"
        bodies = shaped.native.state()[0].cpu().double().numpy()
        forces = shaped.native.contact_forces()[:, feet, 2].cpu().double().numpy()
        after = shaped.episode_length_buf.cpu().numpy()
        extra = (T.foot_clearance_penalty(bodies, feet, points, after, dt, 0.8, 0.008)
                 + T.load_transfer_penalty(forces, meta["mass"], after, dt, 0.8)) * dt
        failed = info1["failed"].cpu().numpy()
        assert np.array_equal(failed, info0["failed"].cpu().numpy())
        extra[failed] = 0
        got = (r1 - r0).cpu().double().numpy()
        np.testing.assert_allclose(got, extra, rtol=1e-4, atol=1e-6, err_msg=f"step {step}")
        checked += E
        terms += int((np.abs(extra) > 1e-4).sum())
    assert checked == 30 * E and terms > E, terms
