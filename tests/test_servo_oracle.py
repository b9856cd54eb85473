"""Pin the XL330/m6 actuator oracle (oracle/servo_oracle.py) with values
computed by hand from the equations' physical meaning: stall torque, the
back-EMF duty window, supply sag with its floor, the Stribeck curve and each
load-friction term switched on alone, the force clamp, and the delay ring of
the servo loop.  The parameter set is declared here (BAM's fitted xl330/m6
values are not available offline)."""

import math

import numpy as np
import pytest

from oracle.servo_oracle import ERROR_GAIN, ServoOracle, xl330_m6

P = dict(kt=0.5, R=2.0, dtheta_stribeck=0.5, alpha=2.0, friction_base=0.01,
         friction_stribeck=0.02, load_friction_external=0.1, load_friction_motor=0.2,
         load_friction_external_stribeck=0.03, load_friction_motor_stribeck=0.04,
         load_friction_external_quad=0.5, load_friction_motor_quad=0.6, friction_viscous=0.007)
KP_FW = 400.0


def run(err=0.0, velocity=0.0, prev_motor=None, prev_applied=0.0, external=0.0, **kw):
    args = dict(parameters=P, vin=5.0, vin_drop_gain=0.5, vin_min=4.0, kp_fw=KP_FW,
                force_limit=10.0)
    args.update(kw)
    prev_motor = np.zeros(2) if prev_motor is None else np.asarray(prev_motor, float)
    one = np.ones(2)
    motor, raw, supply = xl330_m6(err * one, 0 * one, velocity * one, prev_motor,
                                  prev_applied * one, external * one, **args)
    return motor[0], raw[0], supply[0]


def test_error_gain_is_counts_per_radian_over_firmware_scale():
    assert ERROR_GAIN == pytest.approx(4096 / (2 * math.pi) / 226560, rel=1e-15)


def test_stall_torque_inside_the_duty_window():
    err = 0.2 / (KP_FW * ERROR_GAIN)  # duty 0.2
    motor, raw, supply = run(err)
    assert supply == 5.0
    assert raw == pytest.approx(0.5 * 5 * 0.2 / 2)  # kt V duty / R
    assert motor[0] == raw and motor[2] == 0.007
    assert motor[1] == pytest.approx(0.01 + 0.02)  # static: base + full Stribeck


def test_back_emf_window_limits_duty():
    # speed 2: centre kt w / V = 0.2, half-width R 1.75 / V = 0.7.
    _, raw, _ = run(100.0, velocity=2.0)
    assert raw == pytest.approx(0.5 * 5 * 0.9 / 2 - 0.25 * 2 / 2)
    _, raw, _ = run(-100.0, velocity=2.0)
    assert raw == pytest.approx(0.5 * 5 * -0.5 / 2 - 0.25 * 2 / 2)
    # Without motion the window [-0.7, 0.7] binds before the +-1 clamp.
    _, raw, _ = run(100.0)
    assert raw == pytest.approx(0.5 * 5 * 0.7 / 2)
    motor, raw, _ = run(100.0, velocity=2.0, force_limit=0.6)
    assert motor[0] == 0.6 and raw > 0.6
    # kd_scale scales the speed seen by the controller, kp_scale the error.
    _, raw, _ = run(100.0, velocity=1.0, kd_scale=2.0)
    assert raw == pytest.approx(0.5 * 5 * 0.9 / 2 - 0.25 * 2 / 2)
    err = 0.1 / (KP_FW * ERROR_GAIN)
    _, raw, _ = run(err, kp_scale=3.0)
    assert raw == pytest.approx(0.5 * 5 * 0.3 / 2)


def test_supply_sag_and_floor():
    assert run(prev_motor=[1.0, 0.0])[2] == pytest.approx(4.5)
    assert run(prev_motor=[1.0, -2.0])[2] == 4.0  # 5 - 0.5*3 = 3.5, floored at 4
    err = 0.2 / (KP_FW * ERROR_GAIN)
    assert run(err, prev_motor=[1.0, 0.0])[1] == pytest.approx(0.5 * 4.5 * 0.2 / 2)


def test_friction_budget_terms():
    m, _, _ = run(velocity=0.5)  # (|w| / 0.5)^2 = 1
    assert m[1] == pytest.approx(0.01 + 0.02 * math.exp(-1))
    # ext 1, motor 0.5: |0.1 - 0.1| = 0, |0.03 - 0.02| = 0.01, quad on the motor
    # side (|mot| <= |ext|): 0.6 * 0.25.
    m, _, _ = run(external=1.0, prev_applied=0.5)
    assert m[1] == pytest.approx(0.03 + 0.0 + 0.01 + 0.15)
    # ext 0.5, motor 1: |0.05 - 0.2| = 0.15, |0.015 - 0.04| = 0.025, quad on the
    # external side: 0.5 * 0.25.
    m, _, _ = run(external=0.5, prev_applied=1.0)
    assert m[1] == pytest.approx(0.03 + 0.15 + 0.025 + 0.125)
    m2, _, _ = run(external=0.5, prev_applied=1.0, friction_scale=2.0)
    assert m2[1] == pytest.approx(2 * m[1])
    # Moving fast: Stribeck-weighted terms vanish.
    m, _, _ = run(velocity=50.0, external=0.5, prev_applied=1.0)
    assert m[1] == pytest.approx(0.01 + 0.15)


class _Stub:
    """Oracle stand-in: joints at rest at zero, no loads."""

    def __init__(self, J):
        self.J = J
        self.motors = []

    def generalized_loads(self, offset):
        return np.zeros((self.J, 3))

    def snapshot(self):
        return None, np.zeros((self.J, 2)), None

    def set_motor(self, motor):
        self.motors.append(np.array(motor))

    def advance(self, n):
        pass


def test_servo_loop_delays_targets_by_lag_substeps():
    stub = _Stub(2)
    loop = ServoOracle(stub, np.zeros(2), np.zeros(3), 2, parameters=P, vin=5.0,
                       vin_drop_gain=0.0, vin_min=4.0, kp_fw=KP_FW, force_limit=10.0)
    scale = 0.5 * 5 * KP_FW * ERROR_GAIN / 2  # applied torque per radian of delayed target
    targets = [0.01 * (k + 1) for k in range(6)]
    for t in targets:
        loop.substep(np.full(2, t))
    delayed = [m[0, 0] / scale for m in stub.motors]
    # First substep fills the ring with its own target, then a 2-substep lag.
    np.testing.assert_allclose(delayed, [0.01, 0.01, 0.01, 0.02, 0.03, 0.04], rtol=1e-12)
