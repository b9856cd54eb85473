"""Deterministic MicroDuck-like biped written in the `.duck` text format.

The real MicroDuck model is compiled from fetched MJCF and STL assets with
MuJoCo (scripts/prepare_standing.py:31-103, scripts/model_io.py:89-272), none
of which exist offline.  This module authors a synthetic biped with the same
topology and interface contract instead:

* 16 bodies: the static world plus 15 links (masses 0.02-0.4 kg), stored as
  centre-of-mass frames exactly as `Solver::load` reads them
  (src/solver.cpp:85-95);
* 14 hinges in the joint order the specialised backend checks
  (src/cuda/extension.cu:228-231), parent before child with `a < b`
  (src/cuda/model.hpp:54-65);
* one collision shape per link: boxes for most links, an 8-vertex convex hull
  for each foot (src/solver.cpp:115-147);
* the file state is the HOME pose of scripts/prepare_standing.py:13-28, lifted
  so the lowest foot vertex sits 0.1 mm above the ground
  (scripts/prepare_standing.py:74-75), with hinge tangents chosen so the
  measured angle of every joint equals its HOME value (the writer convention
  of scripts/model_io.py:144-148).

`write_model` also emits `metadata.json` with the keys `TensorEnv` reads
(python/duck_gym/tensor_env.py:94-139).
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

JOINT_NAMES = (
    "left_hip_yaw", "left_hip_roll", "left_hip_pitch", "left_knee", "left_ankle",
    "neck_pitch", "head_pitch", "head_yaw", "head_roll",
    "right_hip_yaw", "right_hip_roll", "right_hip_pitch", "right_knee", "right_ankle",
)

# STAND2 home frame (scripts/prepare_standing.py:13-28).
HOME = dict(
    left_hip_yaw=0.0, right_hip_yaw=0.0,
    left_hip_roll=-0.0873, right_hip_roll=0.0873,
    left_hip_pitch=-0.4579, right_hip_pitch=0.4579,
    left_knee=-0.0049, right_knee=0.0049,
    left_ankle=0.4530, right_ankle=-0.4530,
    neck_pitch=0.3491, head_pitch=0.3491,
    head_yaw=0.0, head_roll=0.0,
)

LIMITS = dict(
    left_hip_yaw=(-0.6, 0.6), right_hip_yaw=(-0.6, 0.6),
    left_hip_roll=(-0.5, 0.4), right_hip_roll=(-0.4, 0.5),
    left_hip_pitch=(-1.2, 0.8), right_hip_pitch=(-0.8, 1.2),
    left_knee=(-1.4, 1.4), right_knee=(-1.4, 1.4),
    left_ankle=(-1.0, 1.2), right_ankle=(-1.2, 1.0),
    neck_pitch=(-0.6, 1.1), head_pitch=(-0.6, 1.1),
    head_yaw=(-1.5, 1.5), head_roll=(-0.6, 0.6),
)


def qmul(a, b):
    aw, ax, ay, az = a
    bw, bx, by, bz = b
    return np.array([
        aw * bw - ax * bx - ay * by - az * bz,
        aw * bx + ax * bw + ay * bz - az * by,
        aw * by - ax * bz + ay * bw + az * bx,
        aw * bz + ax * by - ay * bx + az * bw,
    ])


def qconj(q):
    return np.array([q[0], -q[1], -q[2], -q[3]])


def qrot(q, v):
    u = np.asarray(q[1:], dtype=float)
    v = np.asarray(v, dtype=float)
    return v + 2.0 * np.cross(u, np.cross(u, v) + q[0] * v)


def axis_angle(axis, angle):
    axis = np.asarray(axis, dtype=float)
    axis = axis / np.linalg.norm(axis)
    return np.array([math.cos(angle / 2), *(math.sin(angle / 2) * axis)])


def _box_inertia(mass, half):
    x, y, z = (2.0 * h for h in half)
    return np.array([mass / 12 * (y * y + z * z), mass / 12 * (x * x + z * z),
                     mass / 12 * (x * x + y * y)])


# Body frames: principal axes of a few links are permuted relative to the
# world so that the rotation code paths are exercised at HOME.
_RZ90 = axis_angle([0, 0, 1], math.pi / 2)
_RX90 = axis_angle([1, 0, 0], math.pi / 2)


def _links(foot_friction=0.8):
    """Link table in the HOME pose, world coordinates, before the lift."""
    links = []

    def add(name, parent, joint, axis, anchor, mass, com, half, frame=None,
            hull=None):
        links.append(dict(name=name, parent=parent, joint=joint, axis=axis,
                          anchor=anchor, mass=mass, com=np.array(com, float),
                          half=np.array(half, float),
                          frame=np.array([1.0, 0, 0, 0]) if frame is None else frame,
                          hull=hull, friction=foot_friction))

    add("trunk", 0, None, None, None, 0.40, [0.0, 0.0, 0.222], [0.05, 0.045, 0.03],
        frame=_RZ90)
    foot_hull = np.array([[sx * (0.035 if sz < 0 else 0.030),
                           sy * (0.020 if sz < 0 else 0.016), sz * 0.006]
                          for sz in (-1, 1) for sy in (-1, 1) for sx in (-1, 1)])
    for side, sy, pitch_axis in (("left", 1.0, [0, 1, 0]), ("right", -1.0, [0, -1, 0])):
        y = 0.035 * sy
        base = len(links)  # index within `links`; body index = base + 1
        add(f"{side}_hip_yaw_link", 1, f"{side}_hip_yaw", [0, 0, 1], [0, y, 0.195],
            0.03, [0, y, 0.184], [0.012, 0.012, 0.008])
        add(f"{side}_hip_roll_link", base + 1, f"{side}_hip_roll", [1, 0, 0],
            [0, y, 0.174], 0.05, [0, y, 0.160], [0.013, 0.013, 0.012],
            frame=_RX90)
        add(f"{side}_thigh", base + 2, f"{side}_hip_pitch", pitch_axis, [0, y, 0.145],
            0.06, [0, y, 0.115], [0.012, 0.012, 0.027])
        add(f"{side}_shin", base + 3, f"{side}_knee", pitch_axis, [0, y, 0.085],
            0.05, [0, y, 0.055], [0.011, 0.011, 0.027])
        add(f"{side}_foot", base + 4, f"{side}_ankle", pitch_axis, [0.002, y, 0.022],
            0.04, [0.008, y, 0.006], [0.035, 0.02, 0.006],
            frame=_RZ90 if side == "left" else None, hull=foot_hull)
        if side == "left":
            add("neck", 1, "neck_pitch", [0, 1, 0], [0.02, 0, 0.252], 0.03,
                [0.02, 0, 0.266], [0.01, 0.01, 0.012])
            add("head_pitch_link", 7, "head_pitch", [0, 1, 0], [0.02, 0, 0.28], 0.02,
                [0.025, 0, 0.289], [0.01, 0.012, 0.008])
            add("head_yaw_link", 8, "head_yaw", [0, 0, 1], [0.025, 0, 0.298], 0.02,
                [0.025, 0, 0.304], [0.01, 0.01, 0.005])
            add("head", 9, "head_roll", [1, 0, 0], [0.025, 0, 0.31], 0.10,
                [0.035, 0, 0.332], [0.03, 0.035, 0.02])
    return links


def _fmt(values):
    out = []
    for v in values:
        if isinstance(v, (str, int, np.integer)):
            out.append(str(v))
        else:
            out.append(format(float(v), ".17g"))
    return " ".join(out)


def model_text(*, self_contact=False, frictionloss=0.0, armature=0.005,
               damping=0.2, kp=8.0, friction=0.8, lift=0.0001, torque_limit=0.0):
    """Return (.duck text, metadata dict) for the MicroDuck-like biped."""
    links = _links(friction)
    lowest = min((l["com"][2] + (l["hull"][:, 2].min() if l["hull"] is not None
                                 else -l["half"][2])) for l in links)
    dz = lift - lowest
    for l in links:
        l["com"] = l["com"] + [0, 0, dz]
        if l["anchor"] is not None:
            l["anchor"] = np.array(l["anchor"], float) + [0, 0, dz]
    joint_lines, lower, upper, home = [], [], [], []
    by_joint = {l["joint"]: (i + 1, l) for i, l in enumerate(links) if l["joint"]}
    for name in JOINT_NAMES:
        b, child = by_joint[name]
        a = child["parent"]
        parent = links[a - 1]
        qa, qb = parent["frame"], child["frame"]
        axis = np.array(child["axis"], float)
        t = np.cross(axis, [1, 0, 0] if abs(axis[0]) < 0.8 else [0, 1, 0])
        t /= np.linalg.norm(t)
        u = qrot(axis_angle(axis, HOME[name]), t)
        lo, hi = LIMITS[name]
        lower.append(lo)
        upper.append(hi)
        home.append(HOME[name])
        joint_lines.append(_fmt([
            name, a, b,
            *qrot(qconj(qa), child["anchor"] - parent["com"]),
            *qrot(qconj(qb), child["anchor"] - child["com"]),
            *qrot(qconj(qa), axis), *qrot(qconj(qb), axis),
            *qrot(qconj(qa), t), *qrot(qconj(qb), u),
            1, lo, hi, damping, armature, frictionloss,
            0, kp, HOME[name], torque_limit,
        ]))
    body_lines = [_fmt(["world", 0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0])]
    shape_lines = []
    for i, l in enumerate(links):
        inertia = _box_inertia(l["mass"], l["half"])
        frame = l["frame"]
        # Inertia is diagonal in the body frame: permute by the frame rotation.
        rot = np.array([qrot(frame, e) for e in np.eye(3)])  # rows: body axes in world
        inertia_body = np.array([rot[k] @ np.diag(inertia) @ rot[k] for k in range(3)])
        body_lines.append(_fmt([l["name"], l["mass"], *inertia_body, *l["com"], *frame,
                                0, 0, 0, 0, 0, 0]))
        centre = qrot(qconj(frame), [0.0, 0.0, 0.0])
        if l["hull"] is not None:
            row = [i + 1, 3, *centre, *qconj(frame), 0, 0, 0, l["friction"],
                   len(l["hull"]), *l["hull"].ravel()]
        else:
            row = [i + 1, 1, *centre, *qconj(frame), *l["half"], l["friction"], 0]
        if self_contact:
            row.append(1)
        shape_lines.append(_fmt(row))
    names = [l["name"] for l in links]
    pairs = []
    if self_contact:
        for left, right in (("left_foot", "right_foot"), ("left_shin", "right_shin"),
                            ("left_thigh", "right_thigh"), ("left_foot", "right_shin")):
            pairs.append((names.index(left), names.index(right), friction))
    header = f"DUCK_MODEL {2 if self_contact else 1} {len(links) + 1} {len(JOINT_NAMES)} {len(links)}"
    lines = [header, _fmt([0, 0, -9.81, 1]), *body_lines, *joint_lines, *shape_lines]
    if self_contact:
        lines.append(str(len(pairs)))
        lines += [_fmt([a, b, mu]) for a, b, mu in pairs]
    trunk = links[0]
    meta = dict(
        joint_names=list(JOINT_NAMES),
        home=home,
        lower=lower,
        upper=upper,
        root_iquat=[float(x) for x in trunk["frame"]],
        root_height=float(trunk["com"][2]),
        mass=float(sum(l["mass"] for l in links)),
        kp=kp,
        torque_limit=torque_limit,
        torque_limit_enabled=torque_limit > 0,
        physics_profile="microduck-like-synthetic",
        body_names=["world", *names],
        self_contact=self_contact,
    )
    return "\n".join(lines) + "\n", meta


def write_model(directory, **kw):
    """Write `microduck.duck` and `metadata.json` into `directory`."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    text, meta = model_text(**kw)
    (directory / "microduck.duck").write_text(text)
    (directory / "metadata.json").write_text(json.dumps(meta, indent=2) + "\n")
    return directory / "microduck.duck"


if __name__ == "__main__":
    import argparse

    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("output", type=Path)
    p.add_argument("--self-contact", action="store_true")
    p.add_argument("--frictionloss", type=float, default=0.0)
    args = p.parse_args()
    print(write_model(args.output, self_contact=args.self_contact,
                      frictionloss=args.frictionloss))
