"""Small `.duck` models written as text for the tests: a chain of boxes
hinged to each other above the ground, with switches that break one rule of
the format or of the flattening checks at a time."""

from __future__ import annotations


def _body(name, mass, z, inertia=(1e-3, 1e-3, 1e-3), q=(1, 0, 0, 0)):
    return " ".join(str(v) for v in (name, mass, *inertia, 0, 0, z, *q, 0, 0, 0, 0, 0, 0))


def _hinge(name, a, b, axis=(0, 1, 0), damping=0.1, joint_a=None):
    tangent = (1, 0, 0)
    return " ".join(str(v) for v in (
        name, a if joint_a is None else joint_a, b, 0, 0, -0.05, 0, 0, 0.05, *axis, *axis,
        *tangent, *tangent, 1, -1.5, 1.5, damping, 0.01, 0, 0, 8, 0, 0))


def _box(body, ground=1, friction=0.8, version=2, kind=1, vertices=()):
    head = [body, kind, 0, 0, 0, 1, 0, 0, 0, 0.03, 0.02, 0.02, friction, len(vertices)]
    line = " ".join(str(v) for v in head)
    for v in vertices:
        line += " " + " ".join(str(c) for c in v)
    return line + (f" {ground}" if version == 2 else "")


def chain(bodies=4, shapes_per_body=1, version=2, pairs=(), header=None, edit=None,
          ground_flags=None, extra=""):
    """A world body and `bodies - 1` boxes in a hinged chain along -z.
    `edit(lines)` may change the list of lines (header first) before the
    text is joined."""
    nb, nj = bodies, bodies - 2
    ns = (bodies - 1) * shapes_per_body
    lines = [header or f"DUCK_MODEL {version} {nb} {nj} {ns}", "0 0 -9.81 1",
             _body("world", 0, 0)]
    for b in range(1, nb):
        lines.append(_body(f"link{b}", 0.1, 0.5 - 0.1 * b))
    for j in range(nj):
        lines.append(_hinge(f"hinge{j}", j + 1, j + 2))
    k = 0
    for b in range(1, nb):
        for _ in range(shapes_per_body):
            flag = 1 if ground_flags is None else ground_flags[k]
            lines.append(_box(b, ground=flag, version=version))
            k += 1
    if version == 2:
        lines.append(str(len(pairs)))
        for a, b, f in pairs:
            lines.append(f"{a} {b} {f}")
    if edit is not None:
        edit(lines)
    return "\n".join(lines) + "\n" + extra


def caterpillar(segments=24, pairs=True, length=0.04, width=0.03, height=0.02, mass=0.05,
                friction=0.8, shapes_per_segment=1):
    """`segments` boxes lying on the ground in a row along x, each hinged to
    the next about z (yaw: the row curls in the ground plane), every box a
    ground shape resting on its four bottom corners; with `pairs`, body
    contact between segments i and i + 2 (the neighbours a curl brings
    together).  Segment 1 is the free root.  `shapes_per_segment` > 1 stacks
    that many identical box shapes on each segment (each brings its own four
    ground contacts)."""
    hx, hy, hz = length / 2, width / 2, height / 2
    ix = mass * (4 * hy * hy + 4 * hz * hz) / 12
    iy = mass * (4 * hx * hx + 4 * hz * hz) / 12
    iz = mass * (4 * hx * hx + 4 * hy * hy) / 12
    nb, nj = segments + 1, segments - 1
    lines = [f"DUCK_MODEL {2 if pairs else 1} {nb} {nj} {segments * shapes_per_segment}",
             "0 0 -9.81 1",
             _body("world", 0, 0)]
    for s in range(segments):
        lines.append(" ".join(str(v) for v in (f"segment{s}", mass, ix, iy, iz,
                                               s * (length + 0.002), 0, hz + 0.001,
                                               1, 0, 0, 0, 0, 0, 0, 0, 0, 0)))
    for j in range(nj):
        gap = 0.001
        lines.append(" ".join(str(v) for v in (
            f"yaw{j}", j + 1, j + 2, hx + gap, 0, 0, -hx - gap, 0, 0, 0, 0, 1, 0, 0, 1,
            1, 0, 0, 1, 0, 0, 1, -1.2, 1.2, 0.02, 0.001, 0, 0, 8, 0, 0)))
    for s in range(segments):
        for _ in range(shapes_per_segment):
            line = f"{s + 1} 1 0 0 0 1 0 0 0 {hx} {hy} {hz} {friction} 0"
            lines.append(line + (" 1" if pairs else ""))
    if pairs:
        k = shapes_per_segment
        chosen = [(k * s, k * (s + 2)) for s in range(segments - 2)]
        lines.append(str(len(chosen)))
        lines += [f"{a} {b} 0.5" for a, b in chosen]
    return "\n".join(lines) + "\n"
