"""BAM servo loop on the GPU: the physics substeps of the reference's
`BamEnv.step` (python/duck_gym/bam_env.py:307-337) with the XL330/m6
actuator (python/duck_gym/actuator.py:16-77).

Per physics substep the reference runs `generalized_loads`, ~15 torch ops of
actuator arithmetic, the ring-buffer bookkeeping, `step_motor`, a state
snapshot with the root-frame and foot arithmetic of `refresh()`, a ground
contact-force query and `self_contact_stats`.  Here a substep is one launch
(`CudaBatch.servo_substep`): the ring buffer, the Newton-Euler load pass and
the actuator run in the step kernel's prologue on the state it staged, the
motor step follows, and its epilogue folds the self-contact statistics into
their maxima and writes the refresh quantities.  The unfused path (servo
kernel, motor step, queries, torch arithmetic) is kept for comparison.

The actuator parameter VALUES come from the pinned BAM parameter file
(xl330/m6.json at Rhoban/bam 62bd8ce) through the official `config.json`;
neither is available offline, so `SYNTHETIC_XL330` is a declared,
physically plausible set for tests and benchmarks -- not BAM's fitted values.
"""

from __future__ import annotations

import math

import torch

from .native import DuckServo

# Declared parameter set (XL330-class servo at 5 V: stall torque ~0.52 N m,
# stall current ~1.5 A, so kt ~0.35 N m/A and R ~3.4 ohm).
SYNTHETIC_XL330 = dict(
    kt=0.35, R=3.4, dtheta_stribeck=0.2, alpha=1.5, friction_base=0.02,
    friction_stribeck=0.02, load_friction_external=0.05, load_friction_motor=0.05,
    load_friction_external_stribeck=0.02, load_friction_motor_stribeck=0.02,
    load_friction_external_quad=0.1, load_friction_motor_quad=0.1, friction_viscous=0.01)
SYNTHETIC_SUPPLY = dict(vin=5.0, vin_drop_gain=0.05, vin_min=4.0, kp_fw=400.0,
                        force_limit=0.5)


def servo_params(parameters=None, *, vin, vin_drop_gain, vin_min, kp_fw, force_limit,
                 kp_scale=1.0, kd_scale=1.0, friction_scale=1.0, lag=0):
    """A `DuckServo` from a BAM parameter dictionary and the supply/gain
    settings the reference passes to xl330_m6 (bam_env.py:317-329)."""
    p = dict(SYNTHETIC_XL330 if parameters is None else parameters)
    s = DuckServo()
    s.kt, s.resistance = float(p["kt"]), float(p["R"])
    for name in ("dtheta_stribeck", "alpha", "friction_base", "friction_stribeck",
                 "load_friction_external", "load_friction_motor",
                 "load_friction_external_stribeck", "load_friction_motor_stribeck",
                 "load_friction_external_quad", "load_friction_motor_quad", "friction_viscous"):
        setattr(s, name, float(p[name]))
    s.vin, s.vin_drop_gain, s.vin_min = float(vin), float(vin_drop_gain), float(vin_min)
    s.kp_fw, s.force_limit = float(kp_fw), float(force_limit)
    s.kp_scale, s.kd_scale, s.friction_scale = float(kp_scale), float(kd_scale), \
        float(friction_scale)
    s.lag = int(lag)
    return s


def _multiply(a, b):
    w1, x1, y1, z1 = a.unbind(-1)
    w2, x2, y2, z2 = b.unbind(-1)
    return torch.stack((w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2,
                        w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                        w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2,
                        w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2), dim=-1)


def _inverse_rotate(q, v):
    u = -q[..., 1:]
    t = 2 * torch.linalg.cross(u, v)
    return v + q[..., :1] * t + torch.linalg.cross(u, t)


class ServoLoop:
    """The actuator state and substep loop of `BamEnv` over a `CudaBatch`:
    target history ring, previous raw / applied torques, per-step maxima of
    the self-contact statistics, and after every substep the quantities
    `BamEnv.refresh` derives (bam_env.py:128-155): `gravity`, `ang_vel`,
    `lin_vel` and `origin_velocity` of the root, the ground `contact_force`
    on each foot and its `contact` flag, foot `site_pos` / `site_vel`, and
    the `air_time` / `contact_time` timers (bam_env.py:336-337).  With
    `mean_velocity_tau` > 0, `mean_velocity` [E,3] low-passes the root-origin
    world velocity every substep (bam_env.py:343-345, weight
    -expm1(-dt / tau)); `reset` clears it.

    `fused` (default) runs a substep as one launch (`CudaBatch.servo_substep`);
    otherwise as the reference loop does: the servo kernel, the motor step,
    the self-contact query and the refresh arithmetic in torch.  The root
    frame is body 1's frame times the conjugate of `root_principal_quat`
    (bam_env.py:64); `feet` are body indices with `foot_sites` [F,3] in their
    body frames."""

    def __init__(self, batch, params, home, root_offset, *, root_principal_quat=(1.0, 0.0, 0.0, 0.0),
                 feet=(), foot_sites=None, fused=True, mean_velocity_tau=0.0):
        if mean_velocity_tau < 0:
            raise ValueError("mean_velocity_tau must be non-negative")
        self.batch = batch
        self.params = params
        self.fused = fused
        E, J = batch.num_envs, batch.num_joints
        dev, dt = batch.device, batch.dtype
        F = len(feet)
        self.home = torch.as_tensor(home, device=dev, dtype=dt).expand(E, J).contiguous()
        self.root_offset = torch.as_tensor(root_offset, device=dev, dtype=dt).expand(
            E, 3).contiguous()
        self.root_principal_quat = tuple(float(v) for v in root_principal_quat)
        self.root_rotation_inv = torch.tensor(self.root_principal_quat, device=dev, dtype=dt) * \
            torch.tensor([1.0, -1, -1, -1], device=dev, dtype=dt)
        self.feet = [int(b) for b in feet]
        sites = [[0.0, 0.0, 0.0]] * F if foot_sites is None else foot_sites
        self.foot_sites = [[float(v) for v in site] for site in sites]
        self.history = self.home[None].expand(params.lag + 1, E, J).contiguous()
        self.initialized = torch.zeros(E, device=dev, dtype=torch.bool)
        self.cursor = 0
        self.previous_motor = torch.zeros(E, J, device=dev, dtype=dt)
        self.previous_applied = torch.zeros(E, J, device=dev, dtype=dt)
        self.motor = torch.zeros(E, J, 3, device=dev, dtype=dt)
        self.forces = torch.zeros(E, 3, device=dev, dtype=dt)
        self.self_contacts = torch.zeros(E, device=dev, dtype=dt)
        self.self_penetration = torch.zeros(E, device=dev, dtype=dt)
        z3 = lambda *shape: torch.zeros(*shape, device=dev, dtype=dt)  # noqa: E731
        self.gravity, self.ang_vel, self.lin_vel, self.origin_velocity = (z3(E, 3) for _ in range(4))
        self.contact_force, self.site_pos, self.site_vel = (z3(E, F, 3) for _ in range(3))
        self.air_time, self.contact_time = z3(E, F), z3(E, F)
        self.mean_velocity_tau = float(mean_velocity_tau)
        self.mean_alpha = -math.expm1(-batch.dt / self.mean_velocity_tau) \
            if self.mean_velocity_tau else 0.0
        self.mean_velocity = z3(E, 3)

    @property
    def contact(self):
        return self.contact_force.norm(dim=-1) > 1e-5

    def reset(self, mask):
        """bam_env.py:266-282: clear the actuator history of reset envs."""
        self.previous_motor[mask] = 0
        self.previous_applied[mask] = 0
        self.initialized[mask] = False
        self.history[:, mask] = self.home[mask]
        self.self_contacts[mask] = 0
        self.self_penetration[mask] = 0
        self.air_time[mask] = 0
        self.contact_time[mask] = 0
        self.mean_velocity[mask] = 0

    def _refresh(self):
        """bam_env.py:128-155 and 336-337 in torch (the unfused path)."""
        b = self.batch.state()[0]
        root_quat = _multiply(b[:, 1, 3:7], self.root_rotation_inv.expand(b.shape[0], -1))
        down = torch.tensor([0.0, 0.0, -1.0], device=b.device, dtype=b.dtype).expand(b.shape[0], -1)
        self.gravity.copy_(_inverse_rotate(root_quat, down))
        self.ang_vel.copy_(_inverse_rotate(root_quat, b[:, 1, 10:13]))
        conj = torch.tensor([1.0, -1, -1, -1], device=b.device, dtype=b.dtype)
        root_r = -_inverse_rotate(b[:, 1, 3:7] * conj, self.root_offset)
        self.origin_velocity.copy_(b[:, 1, 7:10] + torch.linalg.cross(b[:, 1, 10:13], root_r))
        self.lin_vel.copy_(_inverse_rotate(root_quat, self.origin_velocity))
        if self.feet:
            self.contact_force.copy_(self.batch.contact_forces(ground_only=True)[:, self.feet])
            foot = b[:, self.feet]
            sites = torch.tensor(self.foot_sites, device=b.device, dtype=b.dtype)
            r = _inverse_rotate(foot[:, :, 3:7] * conj, sites[None].expand(b.shape[0], -1, -1))
            self.site_pos.copy_(foot[:, :, :3] + r)
            self.site_vel.copy_(foot[:, :, 7:10] + torch.linalg.cross(foot[:, :, 10:13], r))

    def _after_callback(self):
        """bam_env.py:341-347 in torch (the unfused path): the self-contact
        maxima, the mean-velocity filter, then the air/contact timers."""
        stats = self.batch.self_contact_stats()
        torch.maximum(self.self_contacts, stats[:, 0], out=self.self_contacts)
        torch.maximum(self.self_penetration, stats[:, 1], out=self.self_penetration)
        if self.mean_velocity_tau:
            # mean + alpha (origin - mean), the operations of the fused epilogue
            self.mean_velocity.add_(self.mean_alpha * (self.origin_velocity - self.mean_velocity))
        if self.feet:
            contact = self.contact
            dt = self.batch.dt
            self.air_time.copy_(torch.where(contact, 0.0, self.air_time + dt))
            self.contact_time.copy_(torch.where(contact, self.contact_time + dt, 0.0))

    def substeps(self, target, count, substep_callback=None):
        """`count` physics substeps toward `target` [E,J] (bam_env.py:307-337).
        The callback sees the state and refresh quantities of each substep.
        The unfused path calls it where the reference does, before the
        self-contact maxima, the mean-velocity filter and the timers take
        this substep in; in the fused path, one launch per substep, they
        already include it when the callback runs."""
        target = target.contiguous()
        self.self_contacts.zero_()
        self.self_penetration.zero_()
        for _ in range(count):
            if self.fused:
                self.batch.servo_substep(
                    self.params, target, self.history, self.cursor, self.initialized,
                    self.root_offset, self.previous_motor, self.previous_applied,
                    root_principal_quat=self.root_principal_quat, feet=self.feet,
                    foot_sites=self.foot_sites, motor=self.motor, self_contacts=self.self_contacts,
                    self_penetration=self.self_penetration, gravity=self.gravity,
                    angular_velocity=self.ang_vel, linear_velocity=self.lin_vel,
                    origin_velocity=self.origin_velocity, foot_forces=self.contact_force,
                    site_positions=self.site_pos, site_velocities=self.site_vel,
                    air_time=self.air_time, contact_time=self.contact_time,
                    mean_velocity=self.mean_velocity if self.mean_velocity_tau else None,
                    mean_velocity_alpha=self.mean_alpha)
                self.cursor = (self.cursor + 1) % (self.params.lag + 1)
                if substep_callback is not None:
                    substep_callback(self)
                continue
            motor = self.batch.servo(self.params, target, self.history, self.cursor,
                                     self.initialized, self.root_offset, self.previous_motor,
                                     self.previous_applied)
            self.motor.copy_(motor)
            self.cursor = (self.cursor + 1) % (self.params.lag + 1)
            self.batch.step_motor(motor, self.forces)
            self._refresh()
            if substep_callback is not None:
                substep_callback(self)
            self._after_callback()
