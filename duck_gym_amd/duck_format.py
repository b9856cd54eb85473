"""The `.duck` model text format: reader, writer, v2 body-pair generation and an
importer for a subset of MJCF that needs no MuJoCo.

The format is the one `Solver::load` reads (src/solver.cpp:67-174) and the
reference's exporter writes (scripts/model_io.py:254-271):

    DUCK_MODEL <version 1|2> <bodies> <joints> <shapes>
    <gravity x y z> <ground 0|1>
    <name> <mass> <inertia 3> <com position 3> <principal frame quat wxyz> <v 3> <w 3>   per body
    <name> <a> <b> <anchor in a 3> <anchor in b 3> <axis in a 3> <axis in b 3>
        <tangent in a 3> <tangent in b 3> <limited> <lo> <hi> <damping> <armature>
        <frictionloss> <torque> <kp> <target> <max torque>                           per hinge
    <body> <kind 0 sphere|1 box|2 capsule|3 mesh> <center 3> <quat 4> <size 3>
        <friction> <n> <n vertices 3> [<ground 0|1> in version 2]                     per shape
    [version 2: <pair count>, then <shape a> <shape b> <friction> per pair]

`from_mjcf` follows the reference exporter's rules (scripts/model_io.py:89-272):
one hinge per non-root body (a root body: free, fixed or hinged to the world), the static z = 0 plane as the
only world geom, body frames at the centre of mass along the principal axes,
hinge tangents `axis x e_x` (or `x e_y`), shapes in the body's principal frame,
body-body pairs only with `self_contacts`.  What it computes from the MJCF itself
(forward kinematics at a keyframe, masses and inertias from geoms with MuJoCo's
solid-body formulas, principal axes) is done here in numpy.  Unsupported
elements raise `ValueError` rather than change the physics.
"""

from __future__ import annotations

import math
import xml.etree.ElementTree as ET
from dataclasses import dataclass, field, replace
from pathlib import Path

import numpy as np

SPHERE, BOX, CAPSULE, MESH = 0, 1, 2, 3


@dataclass
class Body:
    name: str
    mass: float
    inertia: list
    x: list
    q: list
    v: list = field(default_factory=lambda: [0.0, 0.0, 0.0])
    w: list = field(default_factory=lambda: [0.0, 0.0, 0.0])


@dataclass
class Joint:
    name: str
    a: int
    b: int
    anchor_a: list
    anchor_b: list
    axis_a: list
    axis_b: list
    tangent_a: list
    tangent_b: list
    limited: int = 0
    lo: float = 0.0
    hi: float = 0.0
    damping: float = 0.0
    armature: float = 0.0
    frictionloss: float = 0.0
    torque: float = 0.0
    kp: float = 0.0
    target: float = 0.0
    max_torque: float = 0.0


@dataclass
class Shape:
    body: int
    kind: int
    center: list
    q: list
    size: list
    friction: float
    points: list = field(default_factory=list)
    ground: int = 1


@dataclass
class DuckModel:
    gravity: list
    ground: int
    bodies: list
    joints: list
    shapes: list
    pairs: list | None = None  # None: version 1 (no body-body pairs)

    @property
    def version(self) -> int:
        return 1 if self.pairs is None else 2


# ------------------------------------------------------------------ text --

def read_duck(source) -> DuckModel:
    """Parse `.duck` text (a path or the text itself), with the loader's
    structural checks (src/solver.cpp:67-174)."""
    text = Path(source).read_text() if isinstance(source, Path) or (
        isinstance(source, str) and "\n" not in source and Path(source).is_file()) else str(source)
    tokens = text.split()
    pos = 0

    def take(n=1, kind=float):
        nonlocal pos
        if pos + n > len(tokens):
            raise ValueError("Truncated model")
        out = [kind(t) for t in tokens[pos:pos + n]]
        pos += n
        return out if n > 1 else out[0]

    if take(kind=str) != "DUCK_MODEL":
        raise ValueError("Invalid model header")
    version, nb, nj, ns = take(4, int)
    if version not in (1, 2) or nb < 1 or nj < 0 or ns < 0:
        raise ValueError("Invalid model header")
    gravity = take(3)
    ground = take(kind=int)
    bodies = []
    for _ in range(nb):
        name = take(kind=str)
        mass = take()
        inertia, x, q, v, w = take(3), take(3), take(4), take(3), take(3)
        if mass < 0 or (mass > 0 and min(inertia) <= 0):
            raise ValueError("Invalid mass/inertia")
        bodies.append(Body(name, mass, inertia, x, q, v, w))
    joints = []
    for _ in range(nj):
        name = take(kind=str)
        a, b = take(2, int)
        frames = [take(3) for _ in range(6)]
        limited = take(kind=int)
        rest = take(9)
        if not (0 <= a < nb and 0 <= b < nb and a != b) or min(rest[2], rest[3], rest[4]) < 0:
            raise ValueError("Invalid joint")
        joints.append(Joint(name, a, b, *frames, limited, *rest))
    shapes = []
    for _ in range(ns):
        body, kind = take(2, int)
        center, q, size = take(3), take(4), take(3)
        friction = take()
        n = take(kind=int)
        if not (0 <= body < nb and 0 <= kind <= 3 and n >= 0 and friction >= 0):
            raise ValueError("Invalid collision shape")
        points = [take(3) for _ in range(n)]
        flag = take(kind=int) if version == 2 else 1
        if kind == MESH and n < 4:
            raise ValueError("Convex mesh needs at least four vertices")
        shapes.append(Shape(body, kind, center, q, size, friction, points, flag))
    pairs = None
    if version == 2:
        count = take(kind=int)
        pairs = []
        for _ in range(count):
            a, b = take(2, int)
            mu = take()
            if not (0 <= a < b < ns) or shapes[a].body == shapes[b].body or mu < 0:
                raise ValueError("Invalid body collision pair")
            if any(p[0] == a and p[1] == b for p in pairs):
                raise ValueError("Duplicate body collision pair")
            pairs.append((a, b, mu))
    if pos != len(tokens):
        raise ValueError("Unexpected model data")
    return DuckModel(gravity, ground, bodies, joints, shapes, pairs)


def _line(values) -> str:
    return " ".join(str(v) if isinstance(v, (str, int, np.integer)) else format(float(v), ".17g")
                    for v in values)


def write_duck(model: DuckModel, path=None) -> str:
    """The model as `.duck` text (floats to 17 significant digits, as the
    reference's exporter writes them); also written to `path` when given."""
    m = model
    lines = [f"DUCK_MODEL {m.version} {len(m.bodies)} {len(m.joints)} {len(m.shapes)}",
             _line([*m.gravity, int(m.ground)])]
    for b in m.bodies:
        lines.append(_line([b.name, b.mass, *b.inertia, *b.x, *b.q, *b.v, *b.w]))
    for j in m.joints:
        lines.append(_line([j.name, int(j.a), int(j.b), *j.anchor_a, *j.anchor_b, *j.axis_a,
                            *j.axis_b, *j.tangent_a, *j.tangent_b, int(j.limited), j.lo, j.hi,
                            j.damping, j.armature, j.frictionloss, j.torque, j.kp, j.target,
                            j.max_torque]))
    for s in m.shapes:
        row = [int(s.body), int(s.kind), *s.center, *s.q, *s.size, s.friction, len(s.points),
               *np.asarray(s.points, dtype=float).ravel()]
        if m.version == 2:
            row.append(int(s.ground))
        lines.append(_line(row))
    if m.version == 2:
        lines.append(str(len(m.pairs)))
        lines += [_line([int(a), int(b), mu]) for a, b, mu in m.pairs]
    text = "\n".join(lines) + "\n"
    if path is not None:
        Path(path).parent.mkdir(parents=True, exist_ok=True)
        Path(path).write_text(text)
    return text


# ----------------------------------------------------------------- pairs --

def body_pairs(model: DuckModel, exclude=()):
    """Candidate body-body pairs of a model: every two shapes on different
    dynamic bodies that are not parent and child through a hinge, in shape
    order, friction the larger of the two (the exporter's rule without MJCF
    contype/priority, scripts/model_io.py:166-195).  `exclude` lists body
    index pairs to leave out."""
    linked = {(j.a, j.b) for j in model.joints} | {(j.b, j.a) for j in model.joints}
    skip = {tuple(p) for p in exclude} | {tuple(p)[::-1] for p in exclude}
    pairs = []
    for a, sa in enumerate(model.shapes):
        for b in range(a + 1, len(model.shapes)):
            sb = model.shapes[b]
            ba, bb = sa.body, sb.body
            if (ba == 0 or bb == 0 or ba == bb or model.bodies[ba].mass == 0
                    or model.bodies[bb].mass == 0 or (ba, bb) in linked or (ba, bb) in skip):
                continue
            pairs.append((a, b, max(sa.friction, sb.friction)))
    return pairs


def with_body_pairs(model: DuckModel, pairs=None) -> DuckModel:
    """A version-2 copy of the model with the given pairs (default
    `body_pairs(model)`); every shape keeps its ground flag (1 for a v1 model,
    whose shapes all touch the ground)."""
    pairs = body_pairs(model) if pairs is None else [tuple(p) for p in pairs]
    if len(pairs) > 32:
        raise ValueError(f"{len(pairs)} body pairs: the loader takes at most 32")
    return replace(model, shapes=[replace(s) for s in model.shapes], pairs=pairs)


# --------------------------------------------------------------- quaternions

def _qmul(a, b):
    aw, ax, ay, az = a
    bw, bx, by, bz = b
    return np.array([aw * bw - ax * bx - ay * by - az * bz, aw * bx + ax * bw + ay * bz - az * by,
                     aw * by - ax * bz + ay * bw + az * bx, aw * bz + ax * by - ay * bx + az * bw])


def _qinv(q):
    return np.array([q[0], -q[1], -q[2], -q[3]])


def _qrot(q, v):
    u = np.asarray(q[1:], dtype=float)
    v = np.asarray(v, dtype=float)
    return v + 2.0 * np.cross(u, np.cross(u, v) + q[0] * v)


def _qaxis(axis, angle):
    axis = np.asarray(axis, dtype=float)
    return np.r_[math.cos(angle / 2), math.sin(angle / 2) * axis]


def _qmatrix(q):
    return np.stack([_qrot(q, e) for e in np.eye(3)], axis=1)


def _matrix_quat(r):
    """Unit quaternion (w >= 0) of a proper rotation matrix."""
    t = np.trace(r)
    if t > 0:
        s = math.sqrt(t + 1.0) * 2
        q = [0.25 * s, (r[2, 1] - r[1, 2]) / s, (r[0, 2] - r[2, 0]) / s, (r[1, 0] - r[0, 1]) / s]
    elif r[0, 0] > r[1, 1] and r[0, 0] > r[2, 2]:
        s = math.sqrt(1.0 + r[0, 0] - r[1, 1] - r[2, 2]) * 2
        q = [(r[2, 1] - r[1, 2]) / s, 0.25 * s, (r[0, 1] + r[1, 0]) / s, (r[0, 2] + r[2, 0]) / s]
    elif r[1, 1] > r[2, 2]:
        s = math.sqrt(1.0 + r[1, 1] - r[0, 0] - r[2, 2]) * 2
        q = [(r[0, 2] - r[2, 0]) / s, (r[0, 1] + r[1, 0]) / s, 0.25 * s, (r[1, 2] + r[2, 1]) / s]
    else:
        s = math.sqrt(1.0 + r[2, 2] - r[0, 0] - r[1, 1]) * 2
        q = [(r[1, 0] - r[0, 1]) / s, (r[0, 2] + r[2, 0]) / s, (r[1, 2] + r[2, 1]) / s, 0.25 * s]
    q = np.asarray(q)
    q /= np.linalg.norm(q)
    return q if q[0] >= 0 else -q


# ------------------------------------------------------------------ MJCF --

_GEOM_TYPES = {"sphere": SPHERE, "box": BOX, "capsule": CAPSULE, "mesh": MESH}


def _floats(text, n=None):
    vals = [float(t) for t in text.split()] if text is not None else []
    if n is not None and len(vals) != n:
        raise ValueError(f"expected {n} numbers, got {text!r}")
    return np.array(vals)


class _Mjcf:
    """The parts of an MJCF document the importer reads, defaults resolved."""

    def __init__(self, root: ET.Element):
        if root.tag != "mujoco":
            raise ValueError("not an MJCF document (root element is not <mujoco>)")
        for tag in ("actuator", "tendon", "equality", "contact", "plugin", "deformable"):
            if root.find(tag) is not None:
                raise ValueError(f"<{tag}> is not supported (the exporter refuses it too)")
        compiler = root.find("compiler")
        self.degrees = True
        self.eulerseq = "xyz"
        self.inertia_from_geom = "auto"
        if compiler is not None:
            self.degrees = compiler.get("angle", "degree") == "degree"
            self.eulerseq = compiler.get("eulerseq", "xyz")
            self.inertia_from_geom = compiler.get("inertiafromgeom", "auto")
        option = root.find("option")
        self.gravity = np.array([0.0, 0.0, -9.81])
        if option is not None:
            if option.get("gravity") is not None:
                self.gravity = _floats(option.get("gravity"), 3)
            for attr in ("wind", "density", "viscosity"):
                if option.get(attr) is not None and np.any(_floats(option.get(attr)) != 0):
                    raise ValueError("Fluid forces are not supported")
        self.defaults = {}
        default = root.find("default")
        if default is not None:
            self._read_defaults(default, "main", {})
        self.meshes = {}
        asset = root.find("asset")
        if asset is not None:
            for mesh in asset.findall("mesh"):
                if mesh.get("vertex") is None:
                    raise ValueError(f"mesh {mesh.get('name')!r}: only inline vertex lists are supported")
                verts = _floats(mesh.get("vertex")).reshape(-1, 3)
                scale = _floats(mesh.get("scale"), 3) if mesh.get("scale") else np.ones(3)
                self.meshes[mesh.get("name")] = verts * scale
        self.root = root

    def _read_defaults(self, node, name, inherited):
        own = {tag: dict(attrs) for tag, attrs in inherited.items()}
        for child in node:
            if child.tag == "default":
                continue
            own.setdefault(child.tag, {}).update(child.attrib)
        self.defaults[name] = own
        for child in node.findall("default"):
            self._read_defaults(child, child.get("class"), own)

    def attrs(self, element, cls):
        cls = element.get("class", cls)
        out = dict(self.defaults.get(cls, {}).get(element.tag, {}))
        out.update(element.attrib)
        return out

    def angle(self, value):
        return math.radians(value) if self.degrees else value

    def orientation(self, a):
        """Quaternion of an element's quat / axisangle / euler / xyaxes / zaxis."""
        if "quat" in a:
            q = _floats(a["quat"], 4)
            return q / np.linalg.norm(q)
        if "axisangle" in a:
            v = _floats(a["axisangle"], 4)
            return _qaxis(v[:3] / np.linalg.norm(v[:3]), self.angle(v[3]))
        if "euler" in a:
            e = _floats(a["euler"], 3)
            q = np.array([1.0, 0, 0, 0])
            for axis_name, value in zip(self.eulerseq, e):
                axis = np.eye(3)["xyzXYZ".index(axis_name) % 3]
                step = _qaxis(axis, self.angle(value))
                # lower case: rotations about the moving axes; upper: fixed axes
                q = _qmul(q, step) if axis_name.islower() else _qmul(step, q)
            return q
        if "xyaxes" in a:
            v = _floats(a["xyaxes"], 6)
            x = v[:3] / np.linalg.norm(v[:3])
            y = v[3:] - x * np.dot(x, v[3:])
            y /= np.linalg.norm(y)
            return _matrix_quat(np.stack([x, y, np.cross(x, y)], axis=1))
        if "zaxis" in a:
            z = _floats(a["zaxis"], 3)
            z /= np.linalg.norm(z)
            axis = np.cross([0, 0, 1.0], z)
            s = np.linalg.norm(axis)
            if s < 1e-12:
                return np.array([1.0, 0, 0, 0]) if z[2] > 0 else np.array([0.0, 1, 0, 0])
            return _qaxis(axis / s, math.atan2(s, z[2]))
        return np.array([1.0, 0, 0, 0])


def _geom_frame(g):
    """pos, quat and size of a geom, with `fromto` resolved."""
    size = _floats(g.get("size", "0"))
    if "fromto" in g:
        ft = _floats(g["fromto"], 6)
        a, b = ft[:3], ft[3:]
        axis = b - a
        length = np.linalg.norm(axis)
        pos = (a + b) / 2
        z = axis / length
        rot = np.cross([0, 0, 1.0], z)
        s = np.linalg.norm(rot)
        if s < 1e-12:
            quat = np.array([1.0, 0, 0, 0]) if z[2] > 0 else np.array([0.0, 1, 0, 0])
        else:
            quat = _qaxis(rot / s, math.atan2(s, z[2]))
        size = np.array([size[0], length / 2])
        return pos, quat, size
    return None, None, size


def _solid(kind, size, vertices, density):
    """Volume, centre (geom frame) and inertia tensor per unit mass of a geom
    of uniform density, by MuJoCo's solid-body formulas (a capsule's two caps
    as one sphere, shifted by the parallel-axis term MuJoCo applies); a mesh
    by its convex hull."""
    if kind == SPHERE:
        r = size[0]
        vol = 4.0 / 3.0 * math.pi * r ** 3
        return vol, np.zeros(3), np.eye(3) * (0.4 * r * r)
    if kind == BOX:
        a, b, c = 2 * size[:3]
        vol = a * b * c
        return vol, np.zeros(3), np.diag([b * b + c * c, a * a + c * c, a * a + b * b]) / 12.0
    if kind == CAPSULE:
        r, h = size[0], 2 * size[1]
        v_sphere, v_cyl = 4.0 / 3.0 * math.pi * r ** 3, math.pi * r * r * h
        vol = v_sphere + v_cyl
        i_axial = v_cyl * r * r / 2 + v_sphere * 2 * r * r / 5
        i_cross = (v_cyl * (3 * r * r + h * h) / 12
                   + v_sphere * (2 * r * r / 5 + h * h / 4 + 3 * h * r / 8))
        return vol, np.zeros(3), np.diag([i_cross, i_cross, i_axial]) / vol
    if kind == MESH:
        from scipy.spatial import ConvexHull

        hull = ConvexHull(vertices)
        vol, first, second = 0.0, np.zeros(3), np.zeros((3, 3))
        origin = vertices[hull.vertices].mean(axis=0)  # inside the hull
        for simplex, plane in zip(hull.simplices, hull.equations):
            # tetrahedron (origin, face) with the face wound outwards
            p = vertices[simplex] - origin
            if np.dot(np.cross(p[1] - p[0], p[2] - p[0]), plane[:3]) < 0:
                p = p[[0, 2, 1]]
            det = np.dot(p[0], np.cross(p[1], p[2]))
            vol += det / 6.0
            first += det / 24.0 * p.sum(axis=0)
            s = p.sum(axis=0)
            second += det / 120.0 * (np.outer(s, s) + sum(np.outer(x, x) for x in p))
        com = first / vol
        second_c = second - vol * np.outer(com, com)
        tensor = np.trace(second_c) * np.eye(3) - second_c
        return vol, com + origin, tensor / vol
    raise ValueError(f"no solid formula for geom kind {kind}")


def from_mjcf(source, keyframe=0, self_contacts=False) -> DuckModel:
    """A `.duck` model from MJCF text or a file (no MuJoCo), in the pose of
    keyframe `keyframe` (index or name; the reference pose when the document
    has none).  See the module docstring for the supported subset."""
    text = Path(source).read_text() if not str(source).lstrip().startswith("<") else str(source)
    doc = _Mjcf(ET.fromstring(text))
    world = doc.root.find("worldbody")
    if world is None:
        raise ValueError("MJCF has no <worldbody>")

    # -- bodies in document (depth-first) order
    order = []  # (element, parent index, childclass)

    def walk(node, parent, cls):
        for child in node.findall("body"):
            order.append((child, parent, child.get("childclass", cls)))
            walk(child, len(order), child.get("childclass", cls))

    walk(world, 0, "main")
    nb = len(order) + 1

    # -- joints, qpos layout
    joints, qpos_size = [], 0
    for i, (body, parent, cls) in enumerate(order, start=1):
        js = [(j, doc.attrs(j, cls)) for j in body.findall("joint")]
        js += [(j, {"type": "free", **j.attrib}) for j in body.findall("freejoint")]
        if not js:
            if parent != 0:
                raise ValueError(f"Fixed child body must be fused before export: {body.get('name')}")
            joints.append((i, None, None, qpos_size))
            continue
        if len(js) != 1:
            raise ValueError("Only one hinge per body is supported")
        j, a = js[0]
        kind = a.get("type", "hinge")
        if kind == "free":
            if parent != 0:
                raise ValueError("A free joint is supported on root bodies only")
            joints.append((i, j, a, qpos_size))
            qpos_size += 7
        elif kind == "hinge":
            joints.append((i, j, a, qpos_size))
            qpos_size += 1
        else:
            raise ValueError("Only free and hinge joints are supported")

    # reference configuration (qpos0) and the keyframe
    qpos0 = np.zeros(qpos_size)
    for i, j, a, adr in joints:
        body = order[i - 1][0]
        if a is not None and a.get("type", "hinge") == "free":
            qpos0[adr:adr + 3] = _floats(body.get("pos", "0 0 0"), 3)
            qpos0[adr + 3:adr + 7] = doc.orientation(body.attrib)
        elif a is not None:
            qpos0[adr] = float(a.get("ref", 0.0))
            if qpos0[adr] != 0:
                raise ValueError("Nonzero hinge ref is not supported")
    qpos = qpos0.copy()
    keys = doc.root.find("keyframe")
    if keys is not None and len(keys.findall("key")):
        all_keys = keys.findall("key")
        key = (all_keys[keyframe] if isinstance(keyframe, int)
               else next(k for k in all_keys if k.get("name") == keyframe))
        if key.get("qpos") is not None:
            qpos = _floats(key.get("qpos"), qpos_size)
        if key.get("qvel") is not None and np.any(_floats(key.get("qvel")) != 0):
            raise ValueError("Keyframe velocities are not supported (export at rest)")

    # -- forward kinematics of body frames
    xpos, xquat = [np.zeros(3)], [np.array([1.0, 0, 0, 0])]
    anchors = {}
    for (body, parent, cls), (i, j, a, adr) in zip(order, joints):
        if a is not None and a.get("type", "hinge") == "free":
            p, q = qpos[adr:adr + 3], qpos[adr + 3:adr + 7] / np.linalg.norm(qpos[adr + 3:adr + 7])
        else:
            p = xpos[parent] + _qrot(xquat[parent], _floats(body.get("pos", "0 0 0"), 3))
            q = _qmul(xquat[parent], doc.orientation(body.attrib))
        if a is not None and a.get("type", "hinge") == "hinge":
            axis = _floats(a.get("axis", "0 0 1"), 3)
            axis = _qrot(q, axis / np.linalg.norm(axis))
            anchor = p + _qrot(q, _floats(a.get("pos", "0 0 0"), 3))
            angle = qpos[adr] - qpos0[adr]
            turn = _qaxis(axis, angle)
            q = _qmul(turn, q)
            p = anchor + _qrot(turn, p - anchor)
            anchors[i] = (anchor, axis, angle)
        xpos.append(p)
        xquat.append(q / np.linalg.norm(q))

    # -- geoms, mass properties, collision shapes
    ground = False
    planes = []
    for g in world.findall("geom"):
        a = doc.attrs(g, "main")
        if a.get("type", "sphere") == "plane":
            pos = _floats(a.get("pos", "0 0 0"), 3)
            if np.linalg.norm(pos) > 1e-10 or abs(_qrot(doc.orientation(a), [0, 0, 1])[2] - 1) > 1e-10:
                raise ValueError("Only the static z=0 ground plane is supported")
            planes.append(a)
            ground = True
        elif int(a.get("contype", 1)) or int(a.get("conaffinity", 1)):
            raise ValueError("Only a plane is supported as a static collision obstacle")

    def compatible(a1, a2):
        return bool((int(a1.get("contype", 1)) & int(a2.get("conaffinity", 1)))
                    or (int(a2.get("contype", 1)) & int(a1.get("conaffinity", 1))))

    bodies = [Body("world", 0.0, [0.0, 0.0, 0.0], [0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0])]
    frames = [(np.zeros(3), np.array([1.0, 0, 0, 0]))]  # (ipos, iquat) in the body frame
    body_geoms = []
    for i, (body, parent, cls) in enumerate(order, start=1):
        geoms = []
        for g in body.findall("geom"):
            a = doc.attrs(g, cls)
            kind_name = a.get("type", "sphere")
            if kind_name not in _GEOM_TYPES:
                raise ValueError(f"Unsupported collision geom type {kind_name}: {a.get('name')}")
            kind = _GEOM_TYPES[kind_name]
            pos, quat, size = _geom_frame(a)
            if pos is None:
                pos, quat = _floats(a.get("pos", "0 0 0"), 3), doc.orientation(a)
            verts = None
            if kind == MESH:
                verts = doc.meshes[a["mesh"]]
                size = np.zeros(3)
            if float(a.get("margin", 0)) or float(a.get("gap", 0)):
                raise ValueError("Nonzero collision margins/gaps are not supported")
            geoms.append(dict(a=a, kind=kind, pos=pos, quat=quat, size=size, verts=verts))
        body_geoms.append(geoms)
        inertial = body.find("inertial")
        given = None  # explicit principal moments and frame (diaginertia)
        if inertial is not None and doc.inertia_from_geom != "true":
            a = inertial.attrib
            mass = float(a["mass"])
            ipos = _floats(a.get("pos", "0 0 0"), 3)
            iq = doc.orientation(a)
            if "fullinertia" in a:
                f = _floats(a["fullinertia"], 6)
                tensor = np.array([[f[0], f[3], f[4]], [f[3], f[1], f[5]], [f[4], f[5], f[2]]])
                tensor = _qmatrix(iq) @ tensor @ _qmatrix(iq).T
                iq = np.array([1.0, 0, 0, 0])
            else:
                given = _floats(a["diaginertia"], 3)
        elif doc.inertia_from_geom != "false" and geoms:
            mass, first, tensor = 0.0, np.zeros(3), np.zeros((3, 3))
            parts = []
            for gm in geoms:
                vol, centre, per_unit = _solid(gm["kind"], gm["size"], gm["verts"], 1.0)
                a = gm["a"]
                m = float(a["mass"]) if "mass" in a else float(a.get("density", 1000.0)) * vol
                rot = _qmatrix(gm["quat"])
                c = gm["pos"] + rot @ centre
                parts.append((m, c, rot @ (per_unit * m) @ rot.T))
                mass += m
                first += m * c
            ipos = first / mass
            for m, c, t in parts:
                d = c - ipos
                tensor += t + m * (np.dot(d, d) * np.eye(3) - np.outer(d, d))
            iq = np.array([1.0, 0, 0, 0])
        else:
            raise ValueError(f"body {body.get('name')!r} has no mass")
        # principal axes, largest moment first (explicit diaginertia kept as
        # given); a diagonal tensor keeps its axes, permuted by a rotation
        # when out of order
        if given is not None:
            principal = given
        elif abs(tensor[0, 1]) + abs(tensor[0, 2]) + abs(tensor[1, 2]) <= 1e-12 * np.trace(tensor):
            moments = np.diag(tensor).copy()
            order_idx = np.argsort(-moments, kind="stable")
            axes = np.eye(3)[:, order_idx]
        else:
            moments, axes = np.linalg.eigh(tensor)
            order_idx = np.argsort(-moments, kind="stable")
            axes = axes[:, order_idx]
            # each axis with its largest component positive (a stable sign)
            for k in range(3):
                if axes[np.argmax(np.abs(axes[:, k])), k] < 0:
                    axes[:, k] = -axes[:, k]
        if given is None:
            if np.linalg.det(axes) < 0:
                axes[:, 2] = -axes[:, 2]
            principal = np.array([axes[:, k] @ tensor @ axes[:, k] for k in range(3)])
            iq = _qmul(iq, _matrix_quat(axes))
        frames.append((ipos, iq))
        x = xpos[i] + _qrot(xquat[i], ipos)
        q = _qmul(xquat[i], iq)
        name = body.get("name") or f"body_{i}"
        bodies.append(Body(name, mass, list(principal), list(x), list(q / np.linalg.norm(q))))

    # -- hinge rows (scripts/model_io.py:120-153)
    duck_joints = []
    for (body, parent, cls), (i, j, a, adr) in zip(order, joints):
        if a is None or a.get("type", "hinge") != "hinge":
            continue
        anchor, axis, angle = anchors[i]
        t = np.cross(axis, [1.0, 0, 0] if abs(axis[0]) < 0.8 else [0, 1.0, 0])
        t /= np.linalg.norm(t)
        u = _qrot(_qaxis(axis, angle), t)
        qa, qb = np.asarray(bodies[parent].q), np.asarray(bodies[i].q)
        xa, xb = np.asarray(bodies[parent].x), np.asarray(bodies[i].x)
        rng = _floats(a.get("range", "0 0"), 2)
        rng = np.array([doc.angle(v) for v in rng])
        limited = a.get("limited", "auto")
        limited = int(limited == "true" or (limited == "auto" and "range" in a))
        duck_joints.append(Joint(
            j.get("name") or f"joint_{len(duck_joints)}", parent, i,
            list(_qrot(_qinv(qa), anchor - xa)), list(_qrot(_qinv(qb), anchor - xb)),
            list(_qrot(_qinv(qa), axis)), list(_qrot(_qinv(qb), axis)),
            list(_qrot(_qinv(qa), t)), list(_qrot(_qinv(qb), u)),
            limited, *(rng - qpos0[adr]),
            float(a.get("damping", 0)), float(a.get("armature", 0)),
            float(a.get("frictionloss", 0))))

    # -- collision shapes in the principal frame (scripts/model_io.py:197-250)
    shapes, geom_ids = [], []
    for i, geoms in enumerate(body_geoms, start=1):
        ipos, iq = frames[i]
        for gm in geoms:
            a = gm["a"]
            if int(a.get("contype", 1)) == 0 and int(a.get("conaffinity", 1)) == 0:
                continue
            floor = any(compatible(a, p) for p in planes)
            if not self_contacts and planes and not floor:
                raise ValueError("Per-shape collision filters require self_contacts=True")
            size = np.zeros(3)
            size[:len(gm["size"])] = gm["size"][:3]
            points = []
            if gm["kind"] == MESH:
                points = np.unique(gm["verts"].astype(float), axis=0).tolist()
            friction = _floats(a.get("friction", "1"))[0]
            shapes.append(Shape(i, gm["kind"], list(_qrot(_qinv(iq), gm["pos"] - ipos)),
                                list(_qmul(_qinv(iq), gm["quat"])), list(size), float(friction),
                                points, int(floor)))
            geom_ids.append((i, a))

    pairs = None
    linked = {(j.a, j.b) for j in duck_joints} | {(j.b, j.a) for j in duck_joints}
    found = []
    for sa in range(len(shapes)):
        for sb in range(sa + 1, len(shapes)):
            (ba, aa), (bb, ab) = geom_ids[sa], geom_ids[sb]
            if ba == bb or (ba, bb) in linked or not compatible(aa, ab):
                continue
            if not self_contacts:
                raise ValueError("Body-body collision requires self_contacts=True")
            pa, pb = int(aa.get("priority", 0)), int(ab.get("priority", 0))
            mu = (shapes[sa] if pa > pb else shapes[sb]).friction if pa != pb else max(
                shapes[sa].friction, shapes[sb].friction)
            found.append((sa, sb, mu))
    if self_contacts:
        pairs = found
    return DuckModel(list(doc.gravity), int(ground), bodies, duck_joints, shapes, pairs)
