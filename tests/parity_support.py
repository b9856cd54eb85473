"""Helpers shared by the GPU parity tests: run the CPU oracle beside the HIP
batch, seed the batch with oracle states, compare whole states."""

from __future__ import annotations

import numpy as np

from oracle.oracle import Oracle
from duck_gym_amd.state import ground_id, self_id


def oracle_envs(model, n, dt, iterations, fp64, mode=0):
    return [Oracle(model, dt, iterations, fp64, mode) for _ in range(n)]


def oracle_state(o):
    """The oracle's per-env state in the decoded-blob vocabulary."""
    bodies, joints, diag = o.snapshot()
    js = o.joint_state()
    ints, reals = o.contacts()
    colors, count = o.colors()
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
    return dict(
        x=bodies[:, 0:3], q=bodies[:, 3:7], v=bodies[:, 7:10], w=bodies[:, 10:13],
        joints=joints, diag=diag,
        **{"lambda": js[:, 0:7]}, penalty=js[:, 7:14], lambdaF=js[:, 23], penaltyF=js[:, 24],
        target=js[:, 25], kp=js[:, 26], maxTorque=js[:, 27], torque=js[:, 28],
        frictionloss=js[:, 29], damping=js[:, 30],
        gc=gc, sc=sc, colors=colors, colorCount=count, failed=int(o.failed),
    )


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
    return [(c["body"], c["shape"], c.get("feature", -1), c.get("other", -1),
             c.get("otherShape", -1)) for c in entries]


def compare_env(gpu, ref, tol, what=""):
    """Max abs differences between a decoded GPU env and an oracle state,
    asserting exact equality of every discrete output."""
    assert contact_keys(gpu["gc"]) == contact_keys(ref["gc"]), f"{what} ground contact set"
    assert contact_keys(gpu["sc"]) == contact_keys(ref["sc"]), f"{what} body contact set"
    assert list(gpu["colors"]) == list(ref["colors"]), f"{what} colours"
    assert gpu["colorCount"] == ref["colorCount"], f"{what} colour count"
    assert gpu["failed"] == ref["failed"], f"{what} failed flag"
    worst = {}
    for key in ("x", "q", "v", "w"):
        worst[key] = float(np.max(np.abs(gpu[key] - ref[key])))
    for key in ("lambda", "penalty"):
        scale = np.maximum(1.0, np.abs(ref[key]))
        worst[key] = float(np.max(np.abs(gpu[key] - ref[key]) / scale, initial=0.0))
    for key in ("x", "q"):
        assert worst[key] <= tol, f"{what} {key} differs by {worst[key]:.3g} > {tol:.3g}"
    # step diagnostics: max anchor error, penetration, contact count,
    # converged flag, max axis error (the decoded blob's first five slots)
    gd, rd = np.asarray(gpu["diag"])[:5], np.asarray(ref["diag"])[:5]
    assert gd[2] == rd[2] and gd[3] == rd[3], f"{what} diag counts/flags {gd} vs {rd}"
    worst["diag"] = float(np.max(np.abs(gd - rd)))
    assert worst["diag"] <= tol, f"{what} diag differs by {worst['diag']:.3g} > {tol:.3g}"
    return worst
