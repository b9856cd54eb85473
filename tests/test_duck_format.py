"""The `.duck` tooling (duck_gym_amd/duck_format.py): text round trips, v2 body
pairs and the MJCF-subset importer.

Pins: the reference's own fixture tests/fixtures/pendulum.duck (exported by
scripts/model_io.py from MuJoCo) rebuilt from a four-line MJCF; closed-form
box and capsule inertias; a convex-hull mesh against the box it spans; the
loader's acceptance of every generated model (the oracle's C++ reader,
src/solver.cpp:67-174); the exporter's refusals (scripts/model_io.py:89-272).
"""

import math

import numpy as np
import pytest

from duck_gym_amd import duck_format as D
from duck_gym_amd.microduck import model_text

from conftest import GOLDEN

PENDULUM_MJCF = """
<mujoco>
  <compiler angle="radian"/>
  <worldbody>
    <body name="pendulum" pos="0 0 1">
      <joint name="hinge" axis="0 1 0"/>
      <geom type="capsule" size="0.03 0.25" pos="0 0 -0.25" mass="1" friction="0.8"/>
    </body>
  </worldbody>
  <keyframe><key qpos="0.5"/></keyframe>
</mujoco>
"""


def assert_same_model(a: str, b: str, tol=1e-12):
    ta, tb = a.split(), b.split()
    assert len(ta) == len(tb)
    for x, y in zip(ta, tb):
        try:
            fx, fy = float(x), float(y)
        except ValueError:
            assert x == y
            continue
        assert abs(fx - fy) <= tol * max(1.0, abs(fy)), (x, y)


def test_round_trip_is_textual():
    for self_contact in (False, True):
        text = model_text(self_contact=self_contact)[0]
        model = D.read_duck(text)
        assert model.version == (2 if self_contact else 1)
        assert D.write_duck(model) == text
    fixture = (GOLDEN / "pendulum.duck").read_text()
    assert_same_model(D.write_duck(D.read_duck(GOLDEN / "pendulum.duck")), fixture, 0.0)


@pytest.mark.parametrize("bad,message", [
    ("DUCK_MODEL 3 2 0 0\n0 0 -9.81 0\n", "Invalid model header"),
    ("DUCK_MODEL 1 2 0 0\n0 0 -9.81 0\nworld 0 0 0 0 0 0 0 1 0 0 0\n", "Truncated model"),
    ("DUCK_MODEL 1 1 0 0\n0 0 -9.81 0\nb -1 1 1 1 0 0 0 1 0 0 0 0 0 0 0 0 0\n", "Invalid mass/inertia"),
    ("DUCK_MODEL 1 1 0 0\n0 0 -9.81 0\nb 1 1 1 1 0 0 0 1 0 0 0 0 0 0 0 0 0\nextra\n", "Unexpected model data"),
])
def test_reader_rejects(bad, message):
    with pytest.raises(ValueError, match=message):
        D.read_duck(bad)


def test_pendulum_fixture_from_mjcf():
    """The reference's exported fixture, rebuilt without MuJoCo: capsule mass
    properties, forward kinematics at the keyframe, hinge frames and tangents."""
    text = D.write_duck(D.from_mjcf(PENDULUM_MJCF))
    assert_same_model(text, (GOLDEN / "pendulum.duck").read_text())


def test_box_and_capsule_inertia_closed_forms():
    vol, c, per_mass = D._solid(D.BOX, np.array([0.1, 0.2, 0.3]), None, 1.0)
    assert vol == pytest.approx(0.2 * 0.4 * 0.6)
    np.testing.assert_allclose(np.diag(per_mass), [(0.16 + 0.36) / 12, (0.04 + 0.36) / 12,
                                                   (0.04 + 0.16) / 12])
    # capsule -> sphere when the cylinder vanishes
    vol, c, per_mass = D._solid(D.CAPSULE, np.array([0.05, 0.0]), None, 1.0)
    assert vol == pytest.approx(4 / 3 * math.pi * 0.05 ** 3)
    np.testing.assert_allclose(np.diag(per_mass), [0.4 * 0.05 ** 2] * 3)


def test_mesh_hull_matches_the_box_it_spans():
    half = np.array([0.02, 0.05, 0.01])
    corners = np.array([[sx, sy, sz] for sx in (-1, 1) for sy in (-1, 1) for sz in (-1, 1)]) * half
    offset = np.array([0.3, -0.1, 0.2])
    vb, cb, ib = D._solid(D.BOX, half, None, 1.0)
    vm, cm, im = D._solid(D.MESH, None, corners + offset, 1.0)
    assert vm == pytest.approx(vb, rel=1e-12)
    np.testing.assert_allclose(cm, offset, atol=1e-15)
    np.testing.assert_allclose(im, ib, rtol=1e-10, atol=1e-18)


def test_rotated_geom_principal_axes():
    """A box geom turned 30 degrees about z: the body frame is its principal
    frame (moments largest first) and the shape sits unrotated in it."""
    mjcf = """
    <mujoco>
      <worldbody>
        <body name="root" pos="0 0 0.5">
          <freejoint/>
          <geom type="box" size="0.1 0.2 0.3" euler="0 0 30" mass="2"/>
        </body>
      </worldbody>
    </mujoco>"""
    m = D.from_mjcf(mjcf)
    body = m.bodies[1]
    expected = 2 * np.array([0.16 + 0.36, 0.04 + 0.36, 0.04 + 0.16]) / 12
    np.testing.assert_allclose(body.inertia, expected, rtol=1e-12)
    # the principal frame is the geom frame (same moment order), so the shape
    # is at the body origin with the identity quaternion, up to sign
    s = m.shapes[0]
    np.testing.assert_allclose(s.center, 0, atol=1e-12)
    assert abs(abs(s.q[0]) - 1) < 1e-12
    np.testing.assert_allclose(body.x, [0, 0, 0.5], atol=1e-15)
    assert abs(D._qrot(body.q, [1, 0, 0])[0] - math.cos(math.radians(30))) < 1e-12


CHAIN = """
<mujoco>
  <default>
    <joint damping="0.1" armature="0.01"/>
    <geom friction="0.7" contype="1" conaffinity="2"/>
    <default class="foot"><geom friction="1.1"/></default>
  </default>
  <worldbody>
    <geom type="plane" size="1 1 0.1" contype="2" conaffinity="1"/>
    <body name="base" pos="0 0 0.3">
      <freejoint/>
      <geom type="box" size="0.05 0.05 0.05" mass="1"/>
      <body name="upper" pos="0 0 -0.1">
        <joint name="hip" axis="1 0 0" range="-1 1"/>
        <geom type="capsule" fromto="0 0 0 0 0 -0.1" size="0.02" mass="0.2"/>
        <body name="foot" pos="0 0 -0.12">
          <joint name="knee" axis="0 1 0" range="-60 60"/>
          <geom class="foot" type="mesh" mesh="hull"/>
        </body>
      </body>
      <body name="arm" pos="0.1 0 0">
        <joint name="shoulder" axis="0 0 1"/>
        <geom type="sphere" size="0.03" mass="0.1" pos="0.02 0 0"/>
      </body>
    </body>
  </worldbody>
  <asset>
    <mesh name="hull" vertex="-0.03 -0.02 -0.01  0.03 -0.02 -0.01  -0.03 0.02 -0.01  0.03 0.02 -0.01
                             -0.03 -0.02 0.01  0.03 -0.02 0.01  -0.03 0.02 0.01  0.03 0.02 0.01"/>
  </asset>
  <keyframe><key qpos="0 0 0.3 1 0 0 0  0.2 -0.3 0.1"/></keyframe>
</mujoco>
"""
CHAIN_SELF = CHAIN.replace('contype="1" conaffinity="2"', 'contype="1" conaffinity="1"').replace(
    'contype="2" conaffinity="1"', 'contype="1" conaffinity="1"')


def test_chain_import_defaults_units_and_loader(tmp_path):
    m = D.from_mjcf(CHAIN)
    assert [b.name for b in m.bodies] == ["world", "base", "upper", "foot", "arm"]
    assert [(j.name, j.a, j.b) for j in m.joints] == [("hip", 1, 2), ("knee", 2, 3), ("shoulder", 1, 4)]
    hip, knee, shoulder = m.joints
    # MJCF angles are in degrees unless <compiler angle="radian">
    assert hip.limited == 1 and hip.lo == pytest.approx(-math.radians(1)) and hip.hi == pytest.approx(math.radians(1))
    assert knee.lo == pytest.approx(-math.radians(60)) and knee.hi == pytest.approx(math.radians(60))
    assert shoulder.limited == 0
    assert hip.damping == 0.1 and hip.armature == 0.01
    assert [s.kind for s in m.shapes] == [D.BOX, D.CAPSULE, D.MESH, D.SPHERE]
    assert [s.friction for s in m.shapes] == [0.7, 0.7, 1.1, 0.7]
    assert m.ground == 1 and m.version == 1
    # the anchors of each hinge coincide in the world from both bodies
    for j in m.joints:
        a, b = m.bodies[j.a], m.bodies[j.b]
        pa = np.asarray(a.x) + D._qrot(a.q, j.anchor_a)
        pb = np.asarray(b.x) + D._qrot(b.q, j.anchor_b)
        np.testing.assert_allclose(pa, pb, atol=1e-14)
        np.testing.assert_allclose(D._qrot(a.q, j.axis_a), D._qrot(b.q, j.axis_b), atol=1e-14)
    # the hinge angle the reference measures from the tangents is the keyframe's
    for j, angle in zip(m.joints, (0.2, -0.3, 0.1)):
        a, b = m.bodies[j.a], m.bodies[j.b]
        axis = D._qrot(a.q, j.axis_a)
        t, u = D._qrot(a.q, j.tangent_a), D._qrot(b.q, j.tangent_b)
        assert math.atan2(np.dot(axis, np.cross(t, u)), np.dot(t, u)) == pytest.approx(angle, abs=1e-12)
    # the oracle's C++ reader (the reference loader's checks) accepts it
    from oracle.oracle import Oracle

    path = tmp_path / "chain.duck"
    D.write_duck(m, path)
    o = Oracle(str(path))
    o.step(np.zeros(3), None, 1, 0.0, 0.0)
    assert not o.failed


def test_body_pairs_rule_and_v2_loader(tmp_path):
    m = D.from_mjcf(CHAIN)
    pairs = D.body_pairs(m)
    # shapes: 0 base, 1 upper, 2 foot, 3 arm; hinge-linked: base-upper,
    # upper-foot, base-arm -> left: base-foot, upper-arm, foot-arm
    assert [(a, b) for a, b, _ in pairs] == [(0, 2), (1, 3), (2, 3)]
    assert [mu for _, _, mu in pairs] == [1.1, 0.7, 1.1]
    v2 = D.with_body_pairs(m)
    assert v2.version == 2 and all(s.ground == 1 for s in v2.shapes)
    text = D.write_duck(v2)
    assert D.write_duck(D.read_duck(text)) == text
    from oracle.oracle import Oracle

    path = tmp_path / "chain2.duck"
    path.write_text(text)
    o = Oracle(str(path))
    o.step(np.zeros(3), None, 1, 0.0, 0.0)
    assert not o.failed
    # the MJCF route, with robot geoms that collide with each other, gives the
    # same pairs under self_contacts and refuses them without
    direct = D.from_mjcf(CHAIN_SELF, self_contacts=True)
    assert direct.pairs == pairs
    with pytest.raises(ValueError, match="Body-body collision requires self_contacts"):
        D.from_mjcf(CHAIN_SELF, self_contacts=False)


@pytest.mark.parametrize("fragment,message", [
    ('<body name="b" pos="0 0 1"><joint type="slide"/><geom size="0.1" mass="1"/></body>',
     "Only free and hinge joints"),
    ('<body name="b" pos="0 0 1"><freejoint/><geom size="0.1" mass="1"/>'
     '<body name="c"><geom size="0.1" mass="1"/></body></body>', "Fixed child body"),
    ('<body name="b" pos="0 0 1"><freejoint/><geom size="0.1" mass="1"/>'
     '<body name="c"><joint axis="1 0 0"/><joint axis="0 1 0"/><geom size="0.1" mass="1"/></body></body>',
     "Only one hinge per body"),
    ('<geom type="box" size="1 1 1"/>', "Only a plane is supported"),
    ('<body name="b" pos="0 0 1"><freejoint/><geom type="cylinder" size="0.1 0.1" mass="1"/></body>',
     "Unsupported collision geom type"),
])
def test_importer_refuses_what_the_exporter_refuses(fragment, message):
    with pytest.raises(ValueError, match=message):
        D.from_mjcf(f"<mujoco><worldbody>{fragment}</worldbody></mujoco>")

