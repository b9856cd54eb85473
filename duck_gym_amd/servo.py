"""BAM servo loop on the GPU: the physics substeps of the reference's
`BamEnv.step` (python/duck_gym/bam_env.py:307-337) with the XL330/m6
actuator (python/duck_gym/actuator.py:16-77).

Per physics substep the reference runs `generalized_loads`, ~15 torch ops of
actuator arithmetic, the ring-buffer bookkeeping, `step_motor`, a state
snapshot and `self_contact_stats`.  Here a substep is two launches, the
servo kernel (ring buffer + Newton-Euler load pass + actuator) and the
implicit motor step, plus the self-contact query the loop accumulates.

The actuator parameter VALUES come from the pinned BAM parameter file
(xl330/m6.json at Rhoban/bam 62bd8ce) through the official `config.json`;
neither is available offline, so `SYNTHETIC_XL330` is a declared,
physically plausible set for tests and benchmarks -- not BAM's fitted values.
"""

from __future__ import annotations

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


class ServoLoop:
    """The actuator state and substep loop of `BamEnv` over a `CudaBatch`:
    target history ring, previous raw / applied torques, per-step maxima of
    the self-contact statistics."""

    def __init__(self, batch, params, home, root_offset):
        self.batch = batch
        self.params = params
        E, J = batch.num_envs, batch.num_joints
        dev, dt = batch.device, batch.dtype
        self.home = torch.as_tensor(home, device=dev, dtype=dt).expand(E, J).contiguous()
        self.root_offset = torch.as_tensor(root_offset, device=dev, dtype=dt).expand(
            E, 3).contiguous()
        self.history = self.home[None].expand(params.lag + 1, E, J).contiguous()
        self.initialized = torch.zeros(E, device=dev, dtype=torch.bool)
        self.cursor = 0
        self.previous_motor = torch.zeros(E, J, device=dev, dtype=dt)
        self.previous_applied = torch.zeros(E, J, device=dev, dtype=dt)
        self.forces = torch.zeros(E, 3, device=dev, dtype=dt)
        self.self_contacts = torch.zeros(E, device=dev, dtype=dt)
        self.self_penetration = torch.zeros(E, device=dev, dtype=dt)

    def reset(self, mask):
        """bam_env.py:266-282: clear the actuator history of reset envs."""
        self.previous_motor[mask] = 0
        self.previous_applied[mask] = 0
        self.initialized[mask] = False
        self.history[:, mask] = self.home[mask]
        self.self_contacts[mask] = 0
        self.self_penetration[mask] = 0

    def substeps(self, target, count, substep_callback=None):
        """`count` physics substeps toward `target` [E,J] (bam_env.py:307-333)."""
        target = target.contiguous()
        self.self_contacts.zero_()
        self.self_penetration.zero_()
        for _ in range(count):
            motor = self.batch.servo(self.params, target, self.history, self.cursor,
                                     self.initialized, self.root_offset, self.previous_motor,
                                     self.previous_applied)
            self.cursor = (self.cursor + 1) % (self.params.lag + 1)
            self.batch.step_motor(motor, self.forces)
            if substep_callback is not None:
                substep_callback(self)
            stats = self.batch.self_contact_stats()
            torch.maximum(self.self_contacts, stats[:, 0], out=self.self_contacts)
            torch.maximum(self.self_penetration, stats[:, 1], out=self.self_penetration)
