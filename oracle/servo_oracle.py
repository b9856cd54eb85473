"""CPU oracle of the BAM servo substep (test infrastructure only).

  xl330_m6     python/duck_gym/actuator.py:16-77 restated in float64 numpy
  ServoOracle  the substep loop of python/duck_gym/bam_env.py:307-337 over
               one oracle environment (oracle.Oracle: kernel.cuh semantics):
               ring-buffered delayed target, external load = -bias +
               constraint of the Newton-Euler pass, actuator, motor step

The actuator arithmetic is pinned by tests/test_servo_oracle.py with
hand-computed values (stall, back-EMF limit, duty window, supply sag,
Stribeck and load friction terms switched on one at a time).  The BAM
parameter values themselves (xl330/m6.json) are not available offline: the
values used are a declared set, so parameter parity is unpinned.
"""

from __future__ import annotations

import math

import numpy as np

ERROR_GAIN = (4096 / (2 * math.pi)) / (256 * 885)


def xl330_m6(target, position, velocity, previous_motor, previous_applied, external, *,
             parameters, vin, vin_drop_gain, vin_min, kp_fw, kp_scale=1.0, kd_scale=1.0,
             friction_scale=1.0, force_limit):
    """(motor [...,J,3], raw [...,J], supply [...,1]) for joint arrays [...,J]."""
    p = parameters
    supply = np.maximum(vin - vin_drop_gain * np.abs(previous_motor).sum(-1, keepdims=True),
                        vin_min)
    speed = velocity * kd_scale
    duty = (target - position) * kp_fw * kp_scale * ERROR_GAIN
    center = p["kt"] * speed / supply
    span = p["R"] * 1.75 / supply
    duty = np.clip(np.minimum(np.maximum(duty, center - span), center + span), -1.0, 1.0)
    raw = p["kt"] * supply * duty / p["R"] - p["kt"] ** 2 * speed / p["R"]
    stribeck = np.exp(-np.power(np.abs(velocity) / p["dtheta_stribeck"], p["alpha"]))
    mot, ext = previous_applied, external
    budget = (p["friction_base"] + stribeck * p["friction_stribeck"]
              + np.abs(ext * p["load_friction_external"] - mot * p["load_friction_motor"])
              + stribeck * np.abs(ext * p["load_friction_external_stribeck"]
                                  - mot * p["load_friction_motor_stribeck"])
              + stribeck * np.where(np.abs(mot) > np.abs(ext),
                                    p["load_friction_external_quad"] * ext ** 2,
                                    p["load_friction_motor_quad"] * mot ** 2)) * friction_scale
    applied = np.clip(raw, -force_limit, force_limit)
    damping = np.full_like(applied, p["friction_viscous"])
    return np.stack((applied, budget, damping), axis=-1), raw, supply


class ServoOracle:
    """One environment's servo loop on an oracle.Oracle.  `dtype` is the
    actuator's arithmetic: float64, or float32 as the reference's float32
    BamEnv evaluates actuator.py (float32 torch tensors, Python scalars
    rounded to float32); the history, torques and the state read from the
    oracle are held in it."""

    def __init__(self, oracle, home, root_offset, lag, dtype=np.float64, **supply):
        self.o = oracle
        self.lag = lag
        self.dtype = dtype
        self.root_offset = np.asarray(root_offset, float)
        self.history = np.tile(np.asarray(home, dtype), (lag + 1, 1))
        self.initialized = False
        self.cursor = 0
        J = len(home)
        self.previous_motor = np.zeros(J, dtype)
        self.previous_applied = np.zeros(J, dtype)
        self.supply = supply

    def substep(self, target):
        target = np.asarray(target, self.dtype)
        self.history[self.cursor] = target
        if not self.initialized:
            self.history[:] = target
            self.initialized = True
        delayed = self.history[(self.cursor - self.lag) % (self.lag + 1)]
        self.cursor = (self.cursor + 1) % (self.lag + 1)
        loads = self.o.generalized_loads(self.root_offset).astype(self.dtype)
        joints = self.o.snapshot()[1].astype(self.dtype)
        motor, raw, _ = xl330_m6(delayed, joints[:, 0], joints[:, 1], self.previous_motor,
                                 self.previous_applied, -loads[:, 0] + loads[:, 1],
                                 **self.supply)
        self.previous_motor = raw
        self.previous_applied = motor[:, 0]
        self.o.set_motor(motor)
        self.o.advance(1)
        return motor
