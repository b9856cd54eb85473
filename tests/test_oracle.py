"""Pinning the CPU oracle (oracle/avbd_oracle.cpp) before it is trusted.

1. Golden fixtures written by the reference's own C++ (tests/golden/
   make_golden.py): trajectories, contact lists, colours, multipliers and
   queries of src/cuda/kernel.cuh, and FP64 trajectories of src/solver.cpp's
   duck_sim -- reproduced bit for bit.
2. A live differential check against the in-place reference build
   (oracle/_ref), when present, on seeded random scenarios.
3. Closed forms and invariants that fix the answer independently of any
   implementation: force units and freefall (tests/test_python.py:71-84,
   scripts/validate_cpu.py:91-95), hinge torque/inertia and stiction
   (tests/test_motor.py:34-44), static weight on the ground, body-contact
   momentum conservation (tests/test_body_contacts.py:28-54), MPR depths
   (tests/test_convex.py:20-34, 72-84) and the static gravity torque that the
   RNEA bias column must equal.
"""

import tempfile
from pathlib import Path

import numpy as np
import pytest

from oracle.oracle import (EXPLICIT_SEQUENTIAL, IMPLICIT_COLOURED, Oracle, ReferenceProbe,
                           convex_query, probe_available)

GOLDEN = Path(__file__).resolve().parent / "golden"
KERNEL_FIXTURES = sorted(GOLDEN.glob("kernel_*.npz"))


def _model_file(text, tmp_path, name="m.duck"):
    path = tmp_path / name
    path.write_text(str(text))
    return path


@pytest.mark.parametrize("fixture", KERNEL_FIXTURES, ids=lambda p: p.stem)
def test_oracle_reproduces_reference_kernel_fixtures(fixture, tmp_path):
    f = np.load(fixture)
    model = _model_file(f["model"], tmp_path)
    fp64 = bool(f["fp64"])
    o = Oracle(model, 0.005, 10, fp64, IMPLICIT_COLOURED)
    targets = f["targets"]
    o.reset(targets)
    motor = f["motor"] if "motor" in f.files else None
    checkpoints = list(f["step"])
    saw_self = saw_limit = False
    for s in range(1, checkpoints[-1] + 1):
        if motor is not None:
            o.set_motor(motor[s - 1])
            o.advance(1)
        else:
            o.step(targets, None, 1, 8.0, float(f["limit"]))
        if s not in checkpoints:
            continue
        i = checkpoints.index(s)
        b, j, d = o.snapshot()
        np.testing.assert_array_equal(b, f["bodies"][i])
        np.testing.assert_array_equal(j, f["joints"][i])
        np.testing.assert_array_equal(d, f["diag"][i])
        np.testing.assert_array_equal(o.joint_state(), f["joint_state"][i])
        n = int(f["contact_count"][i])
        ints, reals = o.contacts(64)
        assert len(ints) == n
        np.testing.assert_array_equal(ints, f["contact_ints"][i][:n])
        np.testing.assert_array_equal(reals, f["contact_reals"][i][:n])
        colors, count = o.colors()
        np.testing.assert_array_equal(colors, f["colors"][i])
        assert count == int(f["color_count"][i])
        np.testing.assert_array_equal(o.generalized_loads([0.001, -0.002, 0.003]), f["loads"][i])
        np.testing.assert_array_equal(o.contact_forces(), f["forces"][i])
        np.testing.assert_array_equal(o.self_contact_stats(), f["stats"][i])
        np.testing.assert_array_equal(o.contact_counts(), f["counts"][i])
        saw_self |= bool((ints[:, 3] >= 0).any()) if n else False
        saw_limit |= bool((np.abs(o.joint_state()[:, 5:7]) > 0).any())
    if "selfc" in fixture.stem:
        assert saw_self and saw_limit, "fixture must exercise body contacts and hinge limits"


@pytest.mark.parametrize("name,steps", [("solver_limp_fp64", 150), ("solver_pendulum_fp64", 400)])
def test_oracle_explicit_mode_reproduces_duck_sim(name, steps, tmp_path):
    f = np.load(GOLDEN / f"{name}.npz")
    o = Oracle(_model_file(f["model"], tmp_path), 0.005, 10, True, EXPLICIT_SEQUENTIAL)
    traj = f["trajectory"]
    np.testing.assert_array_equal(o.snapshot()[0][1:], traj[0])
    for s in range(1, steps + 1):
        o.advance(1)
        np.testing.assert_array_equal(o.snapshot()[0][1:], traj[s])


@pytest.mark.parametrize("name", ["solver_standing_kp8_dt5ms_fp64", "solver_standing_kp8_dt1ms_fp64"])
def test_oracle_explicit_pd_reproduces_duck_sim(name, tmp_path):
    """The explicit PD drive of solver.cpp (solver.cpp:339-347, kp = 8 from
    the model file, HOME targets) bit for bit at every checkpoint of
    duck_sim's own 200-step trajectories."""
    f = np.load(GOLDEN / f"{name}.npz")
    o = Oracle(_model_file(f["model"], tmp_path), float(f["dt"]), 10, True, EXPLICIT_SEQUENTIAL)
    steps = list(f["step"])
    np.testing.assert_array_equal(o.snapshot()[0][1:], f["trajectory"][0])
    for s in range(1, steps[-1] + 1):
        o.advance(1)
        if s in steps:
            np.testing.assert_array_equal(o.snapshot()[0][1:], f["trajectory"][steps.index(s)])


def test_solver_cpp_diverges_on_the_single_env_workload():
    """The reference's own duck_sim on the single-env workload (the biped at
    HOME, kp = 8 with its explicit PD drive, dt = 5 ms, 10 iterations): the
    root leaves for tens of metres and no step converges; at dt = 1 ms the
    same model stays within a few centimetres of its start.  This is why the
    GPU path (the CudaBatch semantics: the PD drive stamped implicitly into
    the Hessian) is checked against kernel.cuh, not against solver.cpp."""
    import json

    f = np.load(GOLDEN / "solver_standing_kp8_dt5ms_fp64.npz")
    root = f["trajectory"][:, 0, :3]
    summary = json.loads(str(f["summary"]))
    assert np.linalg.norm(root[-1] - root[0]) > 10.0
    assert summary["unconverged_steps"] == 200 and summary["max_contacts"] > 16
    g = np.load(GOLDEN / "solver_standing_kp8_dt1ms_fp64.npz")
    bounded = g["trajectory"][:, 0, :3]
    assert np.linalg.norm(bounded[-1] - bounded[0]) < 0.2


@pytest.mark.skipif(not probe_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("fp64", [False, True])
def test_oracle_matches_reference_build_live(fp64, models, home):
    """Seeded random scenarios on every model: bit-exact with kernel.cuh."""
    rng = np.random.default_rng(123 if fp64 else 321)
    for name in ("standing", "selfc", "friction", "limp"):
        o, p = Oracle(models[name], 0.005, 10, fp64), ReferenceProbe(models[name], 0.005, 10, fp64)
        q = home + rng.uniform(-0.5, 0.5, 14)
        root = np.r_[rng.uniform(-0.01, 0.01, 3), rng.uniform(-0.3, 0.3, 3)]
        for x in (o, p):
            x.reset(q, root)
        for s in range(25):
            if s % 4 == 0:
                t = home + rng.uniform(-0.6, 0.6, 14)
                force = rng.normal(0, 0.3, 3)
                limit = float(rng.choice([0.0, 0.2, 1.0]))
            for x in (o, p):
                x.step(t, force, 1, 8.0, limit)
            for a, b in zip(o.snapshot(), p.snapshot()):
                np.testing.assert_array_equal(a, b)
            np.testing.assert_array_equal(o.joint_state(), p.joint_state())
            for a, b in zip(o.contacts(), p.contacts()):
                np.testing.assert_array_equal(a, b)


@pytest.mark.skipif(not probe_available(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("fp64", [False, True])
def test_oracle_matches_reference_build_on_generic_model(fp64, tmp_path):
    """The generic state (kernel.cuh:365, BasicState<32, 32, 160>) on a
    25-body caterpillar: 96 ground contacts plus body contacts between
    segments i and i + 2 and up to 7 colours, bit-exact with kernel.cuh."""
    from model_text import caterpillar

    model = _model_file(caterpillar(), tmp_path)
    rng = np.random.default_rng(5 if fp64 else 6)
    o, p = Oracle(model, 0.005, 10, fp64), ReferenceProbe(model, 0.005, 10, fp64)
    for x in (o, p):
        x.reset(np.zeros(23))
    target = 1.05 + rng.uniform(-0.1, 0.1, 23)
    most = [0, 0, 0]
    for _ in range(40):
        for x in (o, p):
            x.step(target, None, 1, 8.0, 0.0)
        for a, b in zip(o.snapshot(), p.snapshot()):
            np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(o.joint_state(), p.joint_state())
        for a, b in zip(o.contacts(256), p.contacts(256)):
            np.testing.assert_array_equal(a, b)
        assert o.colors()[1] == p.colors()[1]
        counts = o.contact_counts()
        most = [max(most[0], counts[0]), max(most[1], counts[1]), max(most[2], o.colors()[1])]
    assert most[0] == 96 and most[1] > 0 and most[2] > 2, most


# --------------------------------------------------------------- closed forms
FREE_BODY = """DUCK_MODEL 1 2 0 0
0 0 -9.81 0
world 0 0 0 0 0 0 0 1 0 0 0 0 0 0 0 0 0
base 1 .1 .1 .1 0 0 1 1 0 0 0 0 0 0 0 0 0
"""


@pytest.mark.parametrize("mode", [IMPLICIT_COLOURED, EXPLICIT_SEQUENTIAL])
def test_force_units_and_freefall(mode, tmp_path):
    model = _model_file(FREE_BODY, tmp_path)
    o = Oracle(model, 0.001, 200, True, mode)
    for _ in range(100):
        o.step(np.zeros(0), [1.0, 0, 9.81], 1, 0.0, 1.0)
    b = o.snapshot()[0][1]
    assert abs(b[2] - 1) < 1e-12  # 9.81 N holds 1 kg against gravity
    assert abs(b[0] - 0.00505) < 1e-10  # x = h^2 F/m n(n+1)/2
    assert abs(b[7] - 0.1) < 1e-10
    o = Oracle(model, 0.001, 200, True, mode)
    n = 50
    for _ in range(n):
        o.step(np.zeros(0), [0, 0, 0], 1, 0.0, 1.0)
    z = o.snapshot()[0][1][2]
    assert abs(z - (1 - 9.81 * 0.001 ** 2 * n * (n + 1) / 2)) < 1e-12


MOTOR = """DUCK_MODEL 1 2 1 0
0 0 0 0
world 0 0 0 0 0 0 0 1 0 0 0 0 0 0 0 0 0
rotor 1 .01 .01 .01 0 0 0 1 0 0 0 0 0 0 0 0 0
motor 0 1 0 0 0 0 0 0 0 0 1 0 0 1 1 0 0 1 0 0 0 0 0 0 0.002 0 0 0 0 0
"""


def test_hinge_torque_inertia_and_stiction(tmp_path):
    model = _model_file(MOTOR, tmp_path)
    rates = []
    for torque, budget in ((0.02, 0.0), (-0.02, 0.0), (0.02, 0.04)):
        o = Oracle(model, 0.001, 1000, True)
        for _ in range(100):
            o.set_motor([[torque, budget, 0.0]])
            o.advance(1)
        _, joints, diag = o.snapshot()
        rates.append(joints[0])
        assert not diag[5]
    expected = 0.02 / (0.01 + 0.002) * 0.1  # omega = tau / (I + armature) t
    assert abs(rates[0][1] - expected) < 2e-4 and abs(rates[1][1] + expected) < 2e-4
    assert abs(rates[2][0]) < 1e-5  # dry friction budget above the torque: no slip


BOX_ON_GROUND = """DUCK_MODEL 1 2 0 1
0 0 -9.81 1
world 0 0 0 0 0 0 0 1 0 0 0 0 0 0 0 0 0
box 0.5 0.001 0.001 0.001 0 0 0.0501 1 0 0 0 0 0 0 0 0 0
1 1 0 0 0 1 0 0 0 0.05 0.04 0.05 0.8 0
"""


@pytest.mark.parametrize("fp64", [False, True])
def test_static_weight_on_ground(fp64, tmp_path):
    o = Oracle(_model_file(BOX_ON_GROUND, tmp_path), 0.005, 50, fp64)
    for _ in range(100):
        o.step(np.zeros(0), None, 1, 0.0, 1.0)
    forces = o.contact_forces()
    assert abs(forces[1, 2] - 0.5 * 9.81) < 1e-3  # contact forces carry m g
    assert abs(forces[1, 0]) < 1e-6 and abs(forces[1, 1]) < 1e-6
    assert o.contact_counts()[0] == 4


TWO_SPHERES = """DUCK_MODEL 2 3 0 2
0 0 0 0
world 0 0 0 0 0 0 0 1 0 0 0 0 0 0 0 0 0
a 1 .0004 .0004 .0004 0 0 0 1 0 0 0 0.5 0 0 0 0 0
b 2 .0008 .0008 .0008 0.05 0.001 0 1 0 0 0 -0.25 0 0 0 0 0
1 0 0 0 0 1 0 0 0 0.02 0 0 0.5 0 0
2 0 0 0 0 1 0 0 0 0.02 0 0 0.5 0 0
1
0 1 0.5
"""


def test_body_contact_conserves_momentum(tmp_path):
    o = Oracle(_model_file(TWO_SPHERES, tmp_path), 0.001, 50, True)
    p0 = 1 * 0.5 + 2 * -0.25
    touched = False
    for _ in range(150):
        o.advance(1)
        b = o.snapshot()[0]
        p = 1 * b[1, 7:10] + 2 * b[2, 7:10]
        assert np.abs(p - [p0, 0, 0]).max() < 2e-5
        f = o.contact_forces()
        assert np.abs(f[1] + f[2]).max() < 1e-9  # equal and opposite
        touched |= o.contact_counts()[1] > 0
    assert touched
    b = o.snapshot()[0]
    assert np.linalg.norm(b[1, :3] - b[2, :3]) > 0.04 - 2e-5  # separated again


def test_mpr_depth_and_normal():
    box = np.array([[sx, sy, sz] for sx in (-1, 1) for sy in (-1, 1) for sz in (-1, 1)]) * 0.01
    poses = np.array([[0, 0, 0, 1, 0, 0, 0], [0.025, 0, 0, 1, 0, 0, 0]], float)
    for fp64 in (False, True):
        assert convex_query(box, box, poses, fp64=fp64)["status"] == 0
        poses[1, 0] = 0.019
        c = convex_query(box, box, poses, fp64=fp64)
        assert c["status"] == 1 and abs(c["depth"] - 0.001) < 2e-6
        np.testing.assert_allclose(c["normal"], [-1, 0, 0], atol=1e-6)
        poses[1, 0] = 0.021
        c = convex_query(box, box, poses, 0.003, fp64=fp64)
        assert c["status"] == 1 and abs(c["depth"] - 0.002) < 2e-6
        same = np.array([[0, 0, 0, 1, 0, 0, 0]] * 2, float)
        c = convex_query(box, box, same, fp64=fp64)
        assert c["status"] == 1 and abs(c["depth"] - 0.02) < 2e-6
        poses[1, 0] = 0.025


def test_mpr_separates_random_boxes():
    """Moving box A by the reported depth along the reported normal must
    separate it from B (brute-force check with the separating-axis test)."""
    rng = np.random.default_rng(87)
    ea, eb = np.array([0.015, 0.025, 0.04]), np.array([0.03, 0.02, 0.015])
    va = np.array([[sx, sy, sz] for sx in (-1, 1) for sy in (-1, 1) for sz in (-1, 1)]) * ea
    vb = np.array([[sx, sy, sz] for sx in (-1, 1) for sy in (-1, 1) for sz in (-1, 1)]) * eb

    def rot(q):
        w, x, y, z = q
        return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                         [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                         [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])

    def sat_overlap(pa, ra, pb, rb, margin):
        axes = list(ra.T) + list(rb.T) + [np.cross(a, b) for a in ra.T for b in rb.T]
        for ax in axes:
            n = np.linalg.norm(ax)
            if n < 1e-9:
                continue
            ax = ax / n
            ha = np.abs(ra.T @ ax) @ ea
            hb = np.abs(rb.T @ ax) @ eb
            if abs((pb - pa) @ ax) > ha + hb + margin:
                return False
        return True

    hits = 0
    for _ in range(300):
        q = rng.normal(size=(2, 4))
        q /= np.linalg.norm(q, axis=1, keepdims=True)
        pos = rng.uniform(-0.045, 0.045, (2, 3))
        poses = np.c_[pos, q]
        c = convex_query(va, vb, poses, fp64=True)
        assert c["status"] != -1
        expect = sat_overlap(pos[0], rot(q[0]), pos[1], rot(q[1]), -1e-9)
        assert (c["status"] == 1) == expect
        if c["status"]:
            hits += 1
            assert c["depth"] > 0 and abs(np.linalg.norm(c["normal"]) - 1) < 1e-6
            moved = pos[0] + c["normal"] * (c["depth"] + 5e-6)
            assert not sat_overlap(moved, rot(q[0]), pos[1], rot(q[1]), -5e-6)
    assert 30 < hits < 270


def test_rnea_bias_equals_static_gravity_torque(models, home):
    """At rest, column 0 of generalized_loads is the gravity torque of each
    hinge's subtree about its axis: axis . sum_i (x_i - anchor) x (-m_i g)."""
    from duck_gym_amd.microduck import model_text

    text, _ = model_text()
    lines = text.splitlines()
    nb, nj = 16, 14
    masses = np.array([float(l.split()[1]) for l in lines[2:2 + nb]])
    joints = [l.split() for l in lines[2 + nb:2 + nb + nj]]
    parent = {int(j[2]): int(j[1]) for j in joints}
    rng = np.random.default_rng(4)
    for trial in range(5):
        o = Oracle(models["standing"], 0.005, 10, True)
        q = home + rng.uniform(-0.4, 0.4, 14)
        o.reset(q, np.r_[0, 0, 0.1, rng.uniform(-0.5, 0.5, 3)])
        loads = o.generalized_loads([0, 0, 0])
        bodies = o.snapshot()[0]
        g = np.array([0, 0, -9.81])

        def rotate(qq, v):
            w, u = qq[0], qq[1:]
            return v + 2 * np.cross(u, np.cross(u, v) + w * v)

        for k, j in enumerate(joints):
            a, b = int(j[1]), int(j[2])
            rb = np.array([float(x) for x in j[6:9]])
            axis_a = np.array([float(x) for x in j[9:12]])
            anchor = bodies[b, :3] + rotate(bodies[b, 3:7], rb)
            axis = rotate(bodies[a, 3:7], axis_a)
            subtree = [i for i in range(1, nb) if _descends(i, b, parent)]
            tau = sum(np.cross(bodies[i, :3] - anchor, -masses[i] * g) for i in subtree)
            assert abs(loads[k, 0] - axis @ tau) < 1e-12, (trial, k)
            assert loads[k, 1] == 0  # no contacts or active limits after reset


def _descends(i, root, parent):
    while True:
        if i == root:
            return True
        if i not in parent:
            return False
        i = parent[i]


def test_exact_operation_count(tmp_path):
    """oracle/op_count: the oracle instantiated with an operation-counting
    number type gives the exact FLOP per env-step of the reference algorithm
    (about 0.84 MFLOP for the MicroDuck HOME step by a count of the code's
    structure)."""
    import shutil
    import subprocess

    from duck_gym_amd.microduck import HOME, JOINT_NAMES, write_model

    if shutil.which("g++") is None:
        pytest.skip("g++ absent")
    root = Path(__file__).resolve().parents[1] / "oracle"
    subprocess.run(["make", "-s", "-C", str(root), "op_count"], check=True, capture_output=True)
    model = write_model(tmp_path / "m")
    q = [str(HOME[n]) for n in JOINT_NAMES]
    out = subprocess.run([str(root / "op_count"), str(model), "40", "10", "0.005", "8", *q],
                         check=True, capture_output=True, text=True).stdout
    counts = {k: float(v) for k, v in (line.split() for line in out.splitlines())}
    assert counts["failed"] == 0
    total = counts["add_sub"] + counts["mul"] + counts["div"] + counts["sqrt"]
    assert counts["flop_per_step"] == pytest.approx(total)
    assert 5e5 < counts["flop_per_step"] < 1.5e6
