"""CPU oracle of the tensor-env control step (test infrastructure only).

A float64 numpy restatement of python/duck_gym/tensor_env.py's observation,
reward and termination assembly, evaluated on a state snapshot
(bodies [E,B,13], joints [E,J,2], diag [E,6]):

  quat_multiply      tensor_env.py:9-18
  inverse_rotate     tensor_env.py:21-23
  root_frame         tensor_env.py:221-236 (q = q_body1 * conj(root_iquat),
                     projected gravity, local v and w, yaw vector)
  observe            tensor_env.py:238-258 (+ the 48-wide rollout layout)
  step_outputs       tensor_env.py:294-327, 358-368 (failure, reward, returns,
                     counters, timeouts)
  targets            tensor_env.py:279-285, 331-335
  gait_reference     tensor_env.py:260-277 (gait=True)
  foot_clearance_penalty, load_transfer_penalty
                     tensor_env.py:338-357 (the gait-table reward terms)

Pinned by tests/test_task_oracle.py against independent rotation matrices
(scipy), closed-form states (upright, pure tilt, pure yaw, known local
velocities) whose every observation entry and reward term is known by hand,
and the failure thresholds.  Only the tests, `__graft_entry__.smoke()` and
bench.py's CPU baseline use this module.
"""

from __future__ import annotations

import math

import numpy as np

STANDING, LOCOMOTION, ROLLOUT = 0, 1, 2


def quat_multiply(a, b):
    aw, av = a[..., :1], a[..., 1:]
    bw, bv = b[..., :1], b[..., 1:]
    return np.concatenate((aw * bw - (av * bv).sum(-1, keepdims=True),
                           aw * bv + bw * av + np.cross(av, bv)), axis=-1)


def inverse_rotate(q, v):
    u = -q[..., 1:]
    t = 2 * np.cross(u, v)
    return v + q[..., :1] * t + np.cross(u, t)


def root_frame(bodies, iquat):
    """(q, gravity, v_local, w_local, yaw[cos, sin]) of the root body 1."""
    conj = np.asarray(iquat, float) * np.array([1.0, -1, -1, -1])
    q = quat_multiply(bodies[:, 1, 3:7], np.broadcast_to(conj, bodies[:, 1, 3:7].shape))
    down = np.broadcast_to(np.array([0.0, 0, -1]), bodies[:, 1, :3].shape)
    gravity = inverse_rotate(q, down)
    v = inverse_rotate(q, bodies[:, 1, 7:10])
    w = inverse_rotate(q, bodies[:, 1, 10:13])
    yaw = np.stack((1 - 2 * (q[:, 2] ** 2 + q[:, 3] ** 2),
                    2 * (q[:, 0] * q[:, 3] + q[:, 1] * q[:, 2])), axis=-1)
    return q, gravity, v, w, yaw


def targets(actions, home, lower, upper, scale, reference=None):
    a = np.clip(actions, -1, 1)
    ref = np.broadcast_to(home, a.shape) if reference is None else reference
    return a, np.clip(ref + scale * a, lower, upper)


def observe(kind, bodies, joints, actions, meta, *, commands=None, episode=None,
            control_dt=None, gait_period=0.8, filtered=None):
    """Observation rows (float64) of tensor_env.py:238-258 / the rollout layout."""
    _, g, v, w, yaw = root_frame(bodies, meta["root_iquat"])
    height = bodies[:, 1, 2:3] - meta["root_height"]
    q = joints[:, :, 0] - np.asarray(meta["home"])
    qd = 0.1 * joints[:, :, 1]
    if kind == ROLLOUT:
        return np.concatenate((g, w, q, qd, actions), axis=-1)
    pieces = [g, v, w, height, q, qd, actions]
    if kind == LOCOMOTION:
        phase = np.asarray(episode, float) * control_dt * (2 * math.pi / gait_period)
        pieces += [commands, yaw, np.stack((np.sin(phase), np.cos(phase)), axis=-1)]
        if filtered is not None:
            pieces.append(filtered)
    return np.concatenate(pieces, axis=-1)


def step_outputs(kind, bodies, joints, diag, action, last_action, meta, *, control_dt,
                 episode, max_episode_length, commands=None, filtered=None, alpha=1.0,
                 tracking_weight=4.0, heading_weight=0.4, tracking_sigma=0.04,
                 fall_height=0.08):
    """(failed, reward, new_episode, timeout, done, new_filtered) after one
    physics step; `episode` is the counter before the step."""
    _, g, v, w, yaw = root_frame(bodies, meta["root_iquat"])
    height = bodies[:, 1, 2] - meta["root_height"]
    finite = np.isfinite(bodies).all(axis=(1, 2))
    if kind == ROLLOUT:
        failed = bodies[:, 1, 2] < fall_height
    else:
        failed = ((g[:, 2] > -np.float32(math.cos(np.float32(0.5)))) | (np.abs(height) > 0.04)
                  | (diag[:, 0] > 0.005) | (diag[:, 1] > 0.005))
    failed = failed | (diag[:, 5] > 0) | ~finite
    pose = ((joints[:, :, 0] - np.asarray(meta["home"])) ** 2).sum(-1)
    a2 = (action ** 2).sum(-1)
    da2 = ((action - last_action) ** 2).sum(-1)
    tilt = (g[:, :2] ** 2).sum(-1)
    w2 = (w ** 2).sum(-1)
    new_filtered = filtered
    if kind == STANDING:
        reward = (1.5 * np.exp(-20 * tilt) + np.exp(-2000 * height ** 2)
                  + 0.5 * np.exp(-10 * (v ** 2).sum(-1)) - 0.02 * w2 - 0.05 * pose
                  - 0.01 * a2 - 0.02 * da2)
    else:
        velocity = bodies[:, 1, 7:9]
        if filtered is not None:
            new_filtered = (1 - alpha) * filtered + alpha * velocity
            velocity = new_filtered
        error = ((velocity - commands) ** 2).sum(-1)
        reward = (1.0 * np.exp(-20 * tilt) + np.exp(-2000 * height ** 2)
                  + tracking_weight * np.exp(-error / tracking_sigma ** 2) - 0.1 * w2
                  - heading_weight * (1 - yaw[:, 0]) - 0.02 * a2 - 0.03 * da2)
    reward = np.where(failed, -2.0, reward) * control_dt
    new_episode = np.asarray(episode) + 1
    timeout = (new_episode >= max_episode_length) & ~failed
    return failed, reward, new_episode, timeout, failed | timeout, new_filtered


GAIT_DIRECTIONS = np.array([[1.0, 0], [-1, 0], [0, 1], [0, -1]])


def gait_reference(episode, commands, table, period, home, control_dt):
    """Servo reference with the gait table (tensor_env.py:260-277): the table
    row of the direction the command points to most ([4, count, J]: forward,
    backward, left, right), linearly interpolated at phase
    episode * control_dt / period (wrapping from the last node to the first),
    blended in from HOME over the first second of the episode."""
    episode = np.asarray(episode, dtype=np.float64)
    count = table.shape[1]
    index = (episode * control_dt / period % 1) * count
    lo = np.floor(index).astype(int)
    frac = (index - lo)[:, None]
    d = np.argmax(np.asarray(commands) @ GAIT_DIRECTIONS.T, axis=-1)
    ref = table[d, lo] * (1 - frac) + table[d, (lo + 1) % count] * frac
    blend = np.clip(episode * control_dt, 0, 1)[:, None]
    return home + (ref - home) * blend


def foot_clearance_penalty(bodies, foot_bodies, foot_points, episode_after, control_dt,
                           period, lift):
    """Foot-clearance term (tensor_env.py:338-351), before the control_dt
    factor: -20000 sum over both feet of (max(0, h) - desired)^2, with h the
    lowest of the foot's points (body frame [2, V, 3]) above the ground and
    desired = lift sin^2(pi s), s = clip((phase - 0.6) / 0.4, 0, 1), phase the
    gait phase after the step (the right foot's half a period later)."""
    poses = bodies[:, foot_bodies]
    up = np.broadcast_to(np.array([0.0, 0, 1]), poses[:, :, :3].shape)
    local_up = inverse_rotate(poses[:, :, 3:7], up)
    heights = (local_up[:, :, None, :] * foot_points[None]).sum(-1) + poses[:, :, None, 2]
    clearance = heights.min(-1)
    phase = (np.asarray(episode_after, float)[:, None] * control_dt / period
             + np.array([0.0, 0.5])) % 1
    swing = np.clip((phase - 0.6) / 0.4, 0, 1)
    desired = lift * np.sin(np.pi * swing) ** 2
    return -20000 * ((np.maximum(clearance, 0) - desired) ** 2).sum(-1)


def load_transfer_penalty(foot_forces_z, total_mass, episode_after, control_dt, period):
    """Load-transfer term (tensor_env.py:352-357), before the control_dt
    factor: -3 sum over both feet of (clip(F_z / (m g), 0, 3) - wanted)^2,
    wanted = (l, 1 - l), l = 1/2 + sin(2 pi (cycle - 0.05)) / 2."""
    forces = np.asarray(foot_forces_z, float) / (total_mass * 9.81)
    cycle = np.asarray(episode_after, float) * control_dt / period
    left = 0.5 + 0.5 * np.sin(2 * np.pi * (cycle - 0.05))
    wanted = np.stack((left, 1 - left), axis=-1)
    return -3 * ((np.clip(forces, 0, 3) - wanted) ** 2).sum(-1)
