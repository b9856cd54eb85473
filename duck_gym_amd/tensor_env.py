"""Tensor VecEnv for rsl-rl on one MI355X: the `TensorEnv` contract of
python/duck_gym/tensor_env.py, with the control step in HIP kernels.

Per control step the reference runs the physics launch and then ~40 torch
ops for targets, state snapshot, observation, reward, termination and reset
bookkeeping (tensor_env.py:178-219, 221-391).  Here the same step is

  task_targets  clamp(actions) and servo targets              (1 launch)
  step          the AVBD physics, `substeps` steps per launch (1 launch)
  task_step     failure, reward, counters, observation, diag  (1 launch)
  reset         the torch random draws of the reference, the masked state
                reset and a task_observe launch for the reset bookkeeping and
                the post-reset observation

The random draws (`torch.rand`/`torch.randint` on `self.generator`) are made
exactly as the reference makes them, so a seed gives the same perturbations.
The gait-table options (tensor_env.py:151-170, 263-277, 328-354) run in the
same launches: the gait reference in task_targets, the foot-clearance and
load-transfer terms in task_step, which adds them to the reward before the
failure and the control period apply, as the reference does.

Extension: task="rollout" is the 48-wide observation (projected gravity,
local angular velocity, q - HOME, 0.1 qdot, last action) with the locomotion
reward and a fall at base height < `fall_height` (default 0.08 m).
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import torch

from .native import (MAX_JOINTS, TASK_LOCOMOTION, TASK_ROLLOUT, TASK_STANDING, CudaBatch,
                     DuckTask)

_TASKS = {"standing": TASK_STANDING, "locomotion": TASK_LOCOMOTION, "rollout": TASK_ROLLOUT}


def multiply(a, b):
    """Hamilton product of [...,4] wxyz quaternions (tensor_env.py:9-18)."""
    return torch.cat(
        (a[..., :1] * b[..., :1] - (a[..., 1:] * b[..., 1:]).sum(-1, keepdim=True),
         a[..., :1] * b[..., 1:] + b[..., :1] * a[..., 1:]
         + torch.linalg.cross(a[..., 1:], b[..., 1:])),
        dim=-1)


def inverse_rotate(q, v):
    """Rotate v by the conjugate of the unit quaternion q (tensor_env.py:21-23)."""
    u = -q[..., 1:]
    t = 2 * torch.linalg.cross(u, v)
    return v + q[..., :1] * t + torch.linalg.cross(u, t)


class TensorEnv:
    def __init__(self, model_dir, num_envs=128, iterations=200, dt=0.001, substeps=20, seed=42,
                 action_scale=0.3, episode_seconds=30, task="standing", randomize=True,
                 auto_reset=True, fp64=False, command_speed=0.05, backend="cuda", cpu_threads=1,
                 gait=False, foot_clearance=False, tracking_sigma=None, load_transfer=False,
                 velocity_filter_seconds=0.0, tracking_weight=4.0, heading_weight=0.4,
                 command_direction="all", fall_height=0.08):
        if substeps < 1 or episode_seconds <= 0 or action_scale <= 0:
            raise ValueError("Invalid control configuration")
        if backend not in ("cpu", "cuda"):
            raise ValueError(backend)
        if backend == "cpu":
            raise ValueError("backend 'cpu' is not provided: this TensorEnv steps on the GPU")
        self.device = "cuda:0"
        self.num_envs = num_envs
        self.num_actions = 14
        self.dtype = torch.float64 if fp64 else torch.float32
        self.model_dir = Path(model_dir)
        self.meta = json.loads((self.model_dir / "metadata.json").read_text())
        self.native = CudaBatch(str(self.model_dir / "microduck.duck"), num_envs, dt, iterations,
                                0, fp64)
        if self.native.joint_names != self.meta["joint_names"]:
            raise ValueError("Joint order mismatch")
        if task not in _TASKS:
            raise ValueError(task)
        self.task = task
        if any(not math.isfinite(x) or x < 0 for x in (tracking_weight, heading_weight)):
            raise ValueError("Reward weights must be finite and nonnegative")
        self.tracking_weight = tracking_weight
        self.heading_weight = heading_weight
        self.randomize = randomize
        self.auto_reset = auto_reset
        self.velocity_filter_seconds = velocity_filter_seconds
        if not math.isfinite(velocity_filter_seconds) or velocity_filter_seconds < 0:
            raise ValueError("velocity filter must be nonnegative")
        if velocity_filter_seconds > 0 and task != "locomotion":
            raise ValueError("Velocity filter is for locomotion")
        self.filtered_velocity = torch.zeros(num_envs, 2, device=self.device, dtype=self.dtype)
        self.control_dt = dt * substeps
        self.velocity_alpha = (1 - math.exp(-self.control_dt / velocity_filter_seconds)
                               if velocity_filter_seconds > 0 else 1.0)
        self.substeps = substeps
        self.action_scale = action_scale
        self.max_episode_length = round(episode_seconds / self.control_dt)
        self.episode_length_buf = torch.zeros(num_envs, device=self.device, dtype=torch.long)
        self.generator = torch.Generator(device=self.device).manual_seed(seed)
        t = lambda x: torch.tensor(x, device=self.device, dtype=self.dtype)  # noqa: E731
        self.home = t(self.meta["home"])
        self.lower = t(self.meta["lower"])
        self.upper = t(self.meta["upper"])
        self.iquat = t(self.meta["root_iquat"]) * torch.tensor([1, -1, -1, -1], device=self.device)
        # uploaded once, not on every state() call
        self._down = t([0.0, 0, -1])
        self.actions = torch.zeros(num_envs, 14, device=self.device, dtype=self.dtype)
        self.forces = torch.zeros(num_envs, 3, device=self.device, dtype=self.dtype)
        self.commands = torch.zeros(num_envs, 2, device=self.device, dtype=self.dtype)
        self.gait = gait
        self.foot_clearance = foot_clearance
        self.load_transfer = load_transfer
        self.tracking_sigma = tracking_sigma if tracking_sigma is not None else (
            0.02 if gait else 0.04)
        if self.tracking_sigma <= 0:
            raise ValueError("tracking sigma must be positive")
        if gait or foot_clearance or load_transfer:
            import numpy as np

            record = np.load(self.model_dir / "gait.npz")
            self.gait_table = t(record["targets"])
            self.gait_period = float(record["period"])
            self.gait_lift = float(record["lift"]) if "lift" in record else 0.008
            if foot_clearance or load_transfer:
                self.foot_points = t(record["foot_collision_points"])
                self.foot_bodies = torch.tensor(record["foot_bodies"], device=self.device,
                                                dtype=torch.long)
            if abs(float(record["speed"]) - command_speed) > 1e-8:
                raise ValueError("Gait command speed mismatch")
            self.gait_directions = t([[1.0, 0], [-1, 0], [0, 1], [0, -1]])
        self.command_speed = command_speed
        self.direction_names = ("forward", "backward", "left", "right")
        if command_direction not in ("all", *self.direction_names):
            raise ValueError("Invalid command direction")
        self.command_direction = command_direction
        self.returns = torch.zeros(num_envs, device=self.device)
        self.spec = self._spec(fall_height)
        self.obs_dim = self.native.task_obs_dim(self.spec)
        self._obs = None
        self.reset(torch.ones(num_envs, device=self.device, dtype=torch.bool))

    def _spec(self, fall_height):
        s = DuckTask()
        s.kind = _TASKS[self.task]
        s.velocity_filter = int(self.velocity_filter_seconds > 0)
        J = len(self.meta["home"])
        if J > MAX_JOINTS:
            raise ValueError("too many joints")
        for name in ("home", "lower", "upper"):
            getattr(s, name)[:J] = [float(x) for x in self.meta[name]]
        s.iquat[:] = [float(x) for x in self.meta["root_iquat"]]
        s.root_height = float(self.meta["root_height"])
        s.action_scale = float(self.action_scale)
        s.control_dt = float(self.control_dt)
        s.gait_period = float(getattr(self, "gait_period", 0.8))
        s.tracking_weight = float(self.tracking_weight)
        s.heading_weight = float(self.heading_weight)
        s.tracking_sigma = float(self.tracking_sigma)
        s.velocity_alpha = float(self.velocity_alpha)
        s.fall_height = float(fall_height)
        s.max_episode_length = int(self.max_episode_length)
        if self.gait:
            table = self.gait_table
            if table.dim() != 3 or table.shape[0] != 4 or table.shape[2] != J:
                raise ValueError("gait table must be [4, phases, joints]")
            self.gait_table = table.contiguous()
            s.gait, s.gait_phases = 1, int(table.shape[1])
            s.gait_table = self.gait_table.data_ptr()
        if self.foot_clearance or self.load_transfer:
            if self.foot_bodies.numel() != 2:
                raise ValueError("gait shaping needs two foot bodies")
            s.feet[:] = [int(b) for b in self.foot_bodies.cpu()]
            s.foot_clearance, s.load_transfer = int(self.foot_clearance), int(self.load_transfer)
            s.gait_lift = float(self.gait_lift)
            s.weight = float(self.meta["mass"] * 9.81)
            points = self.foot_points
            if points.dim() != 3 or points.shape[0] != 2 or points.shape[2] != 3:
                raise ValueError("foot points must be [2, points, 3]")
            self.foot_points = points.contiguous()
            s.foot_points = int(points.shape[1])
            s.foot_point = self.foot_points.data_ptr()
        return s

    @property
    def _commands(self):
        return self.commands if self.task != "standing" else None

    @property
    def _filtered(self):
        return self.filtered_velocity if self.velocity_filter_seconds > 0 else None

    # ------------------------------------------------------------------ reset
    def reset(self, mask):
        """Masked reset with the reference's random draws (tensor_env.py:178-219).
        The draws are the reference's, in its order, on `self.generator`; q,
        the root offsets and the new commands that it computes from them with
        a dozen torch operations come from one launch
        (duck_task_reset_inputs), rounded as those operations round."""
        E, J = self.num_envs, len(self.meta["home"])
        mask = mask.contiguous()
        joint_draws = root_draws = selected = commands = None
        direction = -1
        if self.randomize:
            joint_draws = torch.rand((E, J), generator=self.generator, device=self.device,
                                     dtype=self.dtype)
            root_draws = torch.rand((E, 2), generator=self.generator, device=self.device,
                                    dtype=self.dtype)
        if self.task != "standing":
            commands = torch.empty_like(self.commands)
            if self.command_direction == "all":
                selected = torch.randint(4, (E,), generator=self.generator, device=self.device)
            else:
                direction = self.direction_names.index(self.command_direction)
        q = torch.empty(E, J, device=self.device, dtype=self.dtype)
        roots = torch.empty(E, 6, device=self.device, dtype=self.dtype)
        self.native.task_reset_inputs(self.spec, mask, joint_draws, root_draws, selected,
                                      direction, self.command_speed,
                                      self.commands if commands is not None else None, q, roots,
                                      commands)
        self.native.reset(mask, q, roots)
        if commands is not None:
            self.commands = commands
        obs = torch.empty(self.num_envs, self.obs_dim, device=self.device)
        self.native.task_observe(self.spec, mask, self.actions, self._commands,
                                 self.episode_length_buf, self._filtered, self.returns,
                                 self.forces, obs)
        self._obs = obs

    # ------------------------------------------------------------ observation
    def state(self):
        """(bodies, joints, diag, gravity, v, w, yaw) as tensor_env.py:221-236."""
        b, j, d = [v.to(self.dtype) for v in self.native.state()]
        q = multiply(b[:, 1, 3:7], self.iquat.expand(self.num_envs, -1))
        down = self._down
        gravity = inverse_rotate(q, down.expand(self.num_envs, -1))
        v = inverse_rotate(q, b[:, 1, 7:10])
        w = inverse_rotate(q, b[:, 1, 10:13])
        yaw = torch.stack((1 - 2 * (q[:, 2] ** 2 + q[:, 3] ** 2),
                           2 * (q[:, 0] * q[:, 3] + q[:, 1] * q[:, 2])), dim=-1)
        return b, j, d, gravity, v, w, yaw

    def observations(self, state):
        """Observation rows from a `state()` tuple, assembled in torch
        (tensor_env.py:238-258); get_observations() assembles the same rows
        from the device state in one kernel."""
        b, j, d, g, v, w, yaw = state
        if self.task == "rollout":
            pieces = [g, w, j[:, :, 0] - self.home, 0.1 * j[:, :, 1], self.actions]
        else:
            pieces = [g, v, w, b[:, 1, 2:3] - self.meta["root_height"], j[:, :, 0] - self.home,
                      0.1 * j[:, :, 1], self.actions]
        if self.task == "locomotion":
            phase = (self.episode_length_buf.to(self.dtype) * self.control_dt
                     * (2 * torch.pi / getattr(self, "gait_period", 0.8)))
            pieces.extend([self.commands, yaw, torch.stack((phase.sin(), phase.cos()), dim=-1)])
            if self.velocity_filter_seconds > 0:
                pieces.append(self.filtered_velocity)
        return torch.cat(pieces, dim=-1).float()

    def get_observations(self):
        obs = torch.empty(self.num_envs, self.obs_dim, device=self.device)
        self.native.task_observe(self.spec, None, self.actions, self._commands,
                                 self.episode_length_buf, self._filtered, self.returns, None, obs)
        return obs, {"observations": {}}

    def reference(self):
        """Servo reference: HOME (None), or the blended gait table in torch
        (tensor_env.py:263-277); step() forms the same reference inside its
        targets launch."""
        if not self.gait:
            return None
        phase = self.episode_length_buf.to(self.dtype) * self.control_dt / self.gait_period
        count = self.gait_table.shape[1]
        index = (phase % 1) * count
        lo = index.long()
        fraction = (index - lo)[:, None]
        direction = (self.commands @ self.gait_directions.T).argmax(-1)
        ref = (self.gait_table[direction, lo] * (1 - fraction)
               + self.gait_table[direction, (lo + 1) % count] * fraction)
        blend = (self.episode_length_buf.to(self.dtype) * self.control_dt).clamp(0, 1)[:, None]
        return (self.home + (ref - self.home) * blend).contiguous()

    # ------------------------------------------------------------------- step
    def step(self, actions):
        E, J = self.num_envs, self.num_actions
        raw = actions.to(dtype=self.dtype).contiguous()
        a = torch.empty(E, J, device=self.device, dtype=self.dtype)
        target = torch.empty_like(a)
        self.native.task_targets(self.spec, raw, None, a, target, self.episode_length_buf,
                                 self.commands)
        self.native.step(target, self.forces.contiguous(), self.substeps, self.meta["kp"],
                         self.meta["torque_limit"])
        obs = torch.empty(E, self.obs_dim, device=self.device)
        reward = torch.empty(E, device=self.device)
        failed = torch.empty(E, device=self.device, dtype=torch.bool)
        timeout = torch.empty_like(failed)
        done = torch.empty_like(failed)
        diag = torch.empty(E, 6, device=self.device, dtype=self.dtype)
        self.native.task_step(self.spec, a, self.actions, self._commands,
                              self.episode_length_buf, self._filtered, self.returns, obs, reward,
                              failed, timeout, done, diag)
        peaks = diag[:, :2].amax(0)  # the two maxima in one reduction
        info = {
            "observations": {},
            "time_outs": timeout,
            "failed": failed,
            "diagnostics": diag,
            "applied_targets": target,
            "terminal_observation": obs,
            "terminal_mask": done,
            "log": {
                "physics/failed_fraction": failed.mean(dtype=torch.float32),
                "physics/max_joint_error_m": peaks[0],
                "physics/max_penetration_m": peaks[1],
            },
        }
        if self.task == "locomotion":
            b, _, _, _, _, _, yaw = self.state()
            velocity = self.filtered_velocity if self.velocity_filter_seconds > 0 \
                else b[:, 1, 7:9]
            error = (velocity - self.commands).square().sum(-1)
            direction = self.commands / max(self.command_speed, 1e-8)
            info["log"].update({
                "tracking/instant_error_mps": (b[:, 1, 7:9] - self.commands).norm(dim=-1).mean(),
                "tracking/command_direction_mps": (b[:, 1, 7:9] * direction).sum(-1).mean(),
                "tracking/reward_velocity_error_mps": error.sqrt().mean(),
                "tracking/absolute_yaw_rad": torch.atan2(yaw[:, 1], yaw[:, 0]).abs().mean(),
            })
        if self.auto_reset:
            self.reset(done)
            obs = self._obs
        return obs, reward, done, info
