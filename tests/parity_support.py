"""Helpers shared by the GPU parity tests: run the CPU oracle beside the HIP
batch, seed the batch with oracle states, compare whole states."""

from __future__ import annotations

import numpy as np

from oracle.oracle import Oracle
from duck_gym_amd.state import ground_id, self_id


def oracle_envs(model, n, dt, iterations, fp64, mode=0):
    return [Oracle(model, dt, iterations, fp64, mode) for _ in range(n)]


def _contact_dicts(ints, reals):
    """Compacted contact lists (the oracle's / the reference probe's
    `contacts()` rows) in the decoded-blob vocabulary."""
    gc, sc = [], []
    for I, R in zip(ints, reals):
        body, shape, feature, other, other_shape, stick = (int(v) for v in I)
        if other < 0:
            gc.append(dict(id=int(ground_id(shape, body, feature, bool(stick))), local=R[0:3],
                           anchor=R[3:5], c0=R[19:20], **{"lambda": R[20:23]}, penalty=R[23:26],
                           body=body, shape=shape, feature=feature, stick=bool(stick)))
        else:
            sc.append(dict(id=int(self_id(body, other, shape, other_shape, bool(stick))),
                           local=R[0:3], localB=R[6:9], t1=R[9:12], t2=R[12:15], n=R[15:18],
                           c0=R[19:20], friction=R[18:19], **{"lambda": R[20:23]},
                           penalty=R[23:26], body=body, other=other, shape=shape,
                           otherShape=other_shape, stick=bool(stick)))
    return gc, sc


def state_dict(bodies, joints, diag, js, ints, reals, colors, count, failed):
    """A per-env solver state in the decoded-blob vocabulary from snapshot
    arrays: bodies [B,13], joints [J,2], diag [6], the 31-column joint state
    (lambda 0-6, penalty 7-13, c0 14-20, angle0, velocity0, lambdaF,
    penaltyF, target, kp, maxTorque, torque, frictionloss, damping), the
    contact rows and the colouring."""
    gc, sc = _contact_dicts(ints, reals)
    return dict(
        x=bodies[:, 0:3], q=bodies[:, 3:7], v=bodies[:, 7:10], w=bodies[:, 10:13],
        joints=joints, diag=diag,
        **{"lambda": js[:, 0:7]}, penalty=js[:, 7:14], lambdaF=js[:, 23], penaltyF=js[:, 24],
        target=js[:, 25], kp=js[:, 26], maxTorque=js[:, 27], torque=js[:, 28],
        frictionloss=js[:, 29], damping=js[:, 30],
        gc=gc, sc=sc, colors=np.asarray(colors), colorCount=int(count), failed=int(failed),
    )


def oracle_state(o):
    """The oracle's per-env state in the decoded-blob vocabulary."""
    bodies, joints, diag = o.snapshot()
    ints, reals = o.contacts()
    colors, count = o.colors()
    return state_dict(bodies, joints, diag, o.joint_state(), ints, reals, colors, count, o.failed)


def fixture_state(f, i):
    """Checkpoint i of a golden fixture (tests/golden/kernel_*.npz, written
    by the reference's own kernel.cuh) in the decoded-blob vocabulary."""
    n = int(f["contact_count"][i])
    return state_dict(f["bodies"][i], f["joints"][i], f["diag"][i], f["joint_state"][i],
                      f["contact_ints"][i][:n], f["contact_reals"][i][:n], f["colors"][i],
                      f["color_count"][i], f["diag"][i][5])


def seed_batch(batch, oracles):
    """Overwrite every env of `batch` with the matching oracle's state."""
    import torch

    codec = batch.codec()
    raw = batch.export_state().cpu().numpy()
    for e, o in enumerate(oracles):
        s = codec.decode(raw[e])
        ref = oracle_state(o)
        for key in ("x", "q", "v", "w", "lambda", "penalty", "lambdaF", "penaltyF", "target",
                    "kp", "maxTorque", "torque", "frictionloss", "damping", "gc", "sc",
                    "colors", "colorCount", "failed"):
            s[key] = ref[key]
        s["ngc"], s["nsc"] = len(ref["gc"]), len(ref["sc"])
        d = ref["diag"]
        s["diag"] = np.array([d[0], d[1], d[2], d[3], d[4], 0, 0, 0])
        codec.encode(raw[e], s)
    batch.import_state(torch.from_numpy(raw).to(batch.device))
    torch.cuda.synchronize()


def contact_keys(entries):
    """The discrete part of a compacted contact list, in list order: bodies,
    shapes, feature and the stick flag."""
    return [(c["body"], c["shape"], c.get("feature", -1), c.get("other", -1),
             c.get("otherShape", -1), bool(c["stick"])) for c in entries]


def stick_mismatches(gpu_list, ref_list):
    """Contacts of two lists with equal keys whose stick flags differ:
    (pressing, free) counts.  A contact presses when the reference's normal
    multiplier is negative.  A free contact (lambda_z = 0) has zero friction
    bound, so its stick test (kernel.cuh:1035-1037) is the exact comparison
    hypot(lambda_t + k C_t) <= 0, decided by whether C_t rounds to zero."""
    pressing = free = 0
    for a, b in zip(gpu_list, ref_list):
        if bool(a["stick"]) != bool(b["stick"]):
            if float(b["lambda"][2]) < 0:
                pressing += 1
            else:
                free += 1
    return pressing, free


def rotation_angle(qa, qb):
    """Angle (rad) of the rotation qa * conj(qb) per row of [n,4] (w x y z)
    quaternions: 2 atan2(|vec|, |w|), the smaller of the two covers."""
    qa, qb = np.atleast_2d(qa), np.atleast_2d(qb)
    w = np.sum(qa * qb, axis=1)
    aw, av = qa[:, :1], qa[:, 1:]
    bw, bv = qb[:, :1], qb[:, 1:]
    vec = bw * av - aw * bv - np.cross(av, bv)
    return 2.0 * np.arctan2(np.linalg.norm(vec, axis=1), np.abs(w))


def _rel(a, b, floor):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b) / np.maximum(floor, np.abs(b))))


# One float32 rounding of a constraint value formed from coordinates of
# order 0.1-1 (m or rad).
CONSTRAINT_EPS = 1e-8


def _rel_k(a, b, k):
    """Multiplier difference beyond what one rounding of the constraint
    moves it by (penalty k x CONSTRAINT_EPS), relative to max(1, |ref|)."""
    a, b, k = (np.asarray(v, dtype=np.float64) for v in (a, b, k))
    if a.size == 0:
        return 0.0
    excess = np.maximum(0.0, np.abs(a - b) - np.abs(k) * CONSTRAINT_EPS)
    return float(np.max(excess / np.maximum(1.0, np.abs(b))))


def _abs(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b), initial=0.0))


def differences(gpu, ref):
    """Worst differences between a decoded GPU env and a reference state.

    Absolute: x (m), rot (rad, rotation angle of q_gpu q_ref^-1), v (m/s),
    w (rad/s), contact geometry (local and anchor points, m; contact
    normals and tangents), c0 (m).  Relative to max(1, |ref|): the joint
    multipliers (lambda, lambdaF; N or N m) and every penalty (>= 1 by
    construction), the contact multipliers.  Also the discrete outputs'
    equality (contact keys, colours, colour count, failed flag)."""
    d = {}
    d["x"] = _abs(gpu["x"], ref["x"])
    d["q"] = _abs(gpu["q"], ref["q"])
    d["rot"] = float(np.max(rotation_angle(gpu["q"], ref["q"]), initial=0.0))
    d["v"] = _abs(gpu["v"], ref["v"])
    d["w"] = _abs(gpu["w"], ref["w"])
    d["joint_lambda"] = max(_rel(gpu["lambda"], ref["lambda"], 1.0),
                            _rel(gpu["lambdaF"], ref["lambdaF"], 1.0))
    d["joint_lambda_k"] = max(_rel_k(gpu["lambda"], ref["lambda"], ref["penalty"]),
                              _rel_k(gpu["lambdaF"], ref["lambdaF"], ref["penaltyF"]))
    d["joint_penalty"] = max(_rel(gpu["penalty"], ref["penalty"], 1.0),
                             _rel(gpu["penaltyF"], ref["penaltyF"], 1.0))
    same_g = [k[:5] for k in contact_keys(gpu["gc"])] == [k[:5] for k in contact_keys(ref["gc"])]
    same_s = [k[:5] for k in contact_keys(gpu["sc"])] == [k[:5] for k in contact_keys(ref["sc"])]
    stick_pressing = stick_free = 0
    for key in ("gc", "sc"):
        p, f = stick_mismatches(gpu[key], ref[key])
        stick_pressing += p
        stick_free += f
    geo, c0, lam, lamk, pen = 0.0, 0.0, 0.0, 0.0, 0.0
    if same_g:
        for a, b in zip(gpu["gc"], ref["gc"]):
            geo = max(geo, _abs(a["local"], b["local"]), _abs(a["anchor"], b["anchor"]))
            c0 = max(c0, _abs(a["c0"], b["c0"]))
            lam = max(lam, _rel(a["lambda"], b["lambda"], 1.0))
            lamk = max(lamk, _rel_k(a["lambda"], b["lambda"], b["penalty"]))
            pen = max(pen, _rel(a["penalty"], b["penalty"], 1.0))
    if same_s:
        for a, b in zip(gpu["sc"], ref["sc"]):
            geo = max(geo, *(_abs(a[k], b[k]) for k in ("local", "localB", "t1", "t2", "n")))
            c0 = max(c0, _abs(a["c0"], b["c0"]))
            lam = max(lam, _rel(a["lambda"], b["lambda"], 1.0))
            lamk = max(lamk, _rel_k(a["lambda"], b["lambda"], b["penalty"]))
            pen = max(pen, _rel(a["penalty"], b["penalty"], 1.0))
            assert abs(float(a["friction"][0]) - float(b["friction"][0])) <= 1e-7 * max(
                1.0, abs(float(b["friction"][0]))), "pair friction"
    d.update(contact_geometry=geo, contact_c0=c0, contact_lambda=lam, contact_lambda_k=lamk,
             contact_penalty=pen)
    gd, rd = np.asarray(gpu["diag"])[:5], np.asarray(ref["diag"])[:5]
    d["diag"] = float(np.max(np.abs(gd - rd)))
    d["stick_free"] = stick_free
    d["_discrete"] = dict(
        ground=same_g, body=same_s, stick=stick_pressing == 0,
        colors=list(gpu["colors"]) == list(ref["colors"]),
        colorCount=gpu["colorCount"] == ref["colorCount"], failed=gpu["failed"] == ref["failed"],
        diag_counts=bool(gd[2] == rd[2] and gd[3] == rd[3]))
    return d


# Tolerance classes of the parity gates.  `tol` is the pose tolerance (m
# and rad).  float64 runs evaluate the reference's operations (one lane per
# block solve: its accumulation order), so every quantity -- velocities,
# joint and contact multipliers, penalties, contact points -- is held to
# `tol` as well (absolute, or relative to max(1, |ref|)).  float32 runs use
# the hardware reciprocal/square root, fused multiply-adds and another
# summation order.  A multiplier moves by penalty x constraint (penalties up
# to 1e9 on positions, 1e7 on angles), so one float rounding of a
# constraint value (CONSTRAINT_EPS) moves it by k x CONSTRAINT_EPS; beyond
# that, after the ten augmented-Lagrangian iterations of one step from an
# identical state, multipliers agree within FLOAT_LAMBDA_RTOL of
# max(1, |lambda|).  Measured: 2.2e-3 on the biped, 2.0e-2 on a curled
# 24-segment chain with its hinge limits engaged -- where the reference's
# own float32 build differs from its float64 build by as much (2.0e-2 after
# 20 steps, poses within 7e-6).  A penalty ramps by beta |C| per iteration, so
# float rounding of an angle (~1e-7 rad) moves an angular penalty at its
# floor of 1 by beta_angular (1e5) x 1e-7 x 10 iterations = 0.1 relative:
# FLOAT_PENALTY_RTOL.  Velocities are pose differences over one step
# (v = (x - x0) / h), so a pose tolerance admits 2 tol / h.
FLOAT_LAMBDA_RTOL = 5e-2
FLOAT_PENALTY_RTOL = 1e-1


def default_gates(tol, dt, fp64):
    if fp64:
        return dict(x=tol, rot=tol, q=tol, v=tol, w=tol, joint_lambda=tol, joint_penalty=tol,
                    contact_geometry=tol, contact_c0=tol, contact_lambda=tol,
                    contact_penalty=tol, diag=tol)
    return dict(x=tol, rot=tol, q=tol, v=2 * tol / dt, w=2 * tol / dt,
                joint_lambda_k=FLOAT_LAMBDA_RTOL, joint_penalty=FLOAT_PENALTY_RTOL,
                contact_geometry=tol, contact_c0=tol, contact_lambda_k=FLOAT_LAMBDA_RTOL,
                contact_penalty=FLOAT_PENALTY_RTOL, diag=tol)


def compare_env(gpu, ref, tol, what="", dt=0.005, gates=None, fp64=None, strict_stick=False):
    """Assert that a decoded GPU env matches a reference state: every
    discrete output (contact lists in order, the stick flags of every
    pressing contact, colours, colour count, failed flag, contact count and
    converged flag) exactly; poses,
    rotation angles, velocities, joint and contact multipliers and
    penalties, contact points and the step diagnostics within the gates
    (default_gates(tol, dt, fp64), overridden per key by `gates`; `fp64`
    defaults to the decoded state's precision).  With `strict_stick` (runs
    from identical states) the stick flags of free contacts must match too.
    Returns the worst differences."""
    if fp64 is None:
        fp64 = np.asarray(gpu["x"]).dtype == np.float64
    d = differences(gpu, ref)
    disc = d.pop("_discrete")
    assert disc["ground"], (f"{what} ground contact set "
                            f"{contact_keys(gpu['gc'])} vs {contact_keys(ref['gc'])}")
    assert disc["body"], (f"{what} body contact set "
                          f"{contact_keys(gpu['sc'])} vs {contact_keys(ref['sc'])}")
    assert disc["stick"], f"{what} stick flag of a pressing contact"
    assert disc["colors"], f"{what} colours {list(gpu['colors'])} vs {list(ref['colors'])}"
    assert disc["colorCount"], f"{what} colour count"
    assert disc["failed"], f"{what} failed flag"
    assert disc["diag_counts"], f"{what} diag contact count / converged flag"
    g = default_gates(tol, dt, fp64)
    g.update(gates or {})
    if strict_stick:
        assert d["stick_free"] == 0, f"{what} stick flag of a free contact"
    for key, limit in g.items():
        assert d[key] <= limit, f"{what} {key} differs by {d[key]:.3g} > {limit:.3g}"
    return d
