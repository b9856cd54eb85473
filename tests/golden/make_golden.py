"""Write the golden fixtures that pin the CPU oracle (tests/golden/*.npz).

Every expected value comes from the reference's own C++ compiled in place
from the reference tree by oracle/Makefile (`make -C oracle ref`):
  * oracle/_ref/ref_probe.so  -- src/cuda/kernel.cuh (the CudaBatch solver
    core) behind a small C driver: trajectories, compacted contact lists,
    colours, joint multipliers, generalized loads, contact forces;
  * oracle/_ref/duck_sim      -- src/main.cpp + src/solver.cpp (the
    independent FP64 solver) CSV trajectories.
Inputs are the MicroDuck-like models of duck_gym_amd/microduck.py (the model
text is stored in each fixture) and the reference's tests/fixtures/pendulum.duck
(copied as data into tests/golden/pendulum.duck).

Run in a container that has the reference tree:
    make -C oracle ref && python tests/golden/make_golden.py
(`--solver-pd` writes only the explicit-PD duck_sim fixtures.)
"""

from __future__ import annotations

import csv
import io
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from duck_gym_amd.microduck import HOME, JOINT_NAMES, model_text  # noqa: E402
from oracle.oracle import REF_DIR, ReferenceProbe  # noqa: E402

DT, ITER, KP = 0.005, 10, 8.0
CHECKPOINTS = (1, 2, 10, 40, 100, 200)


def home():
    return np.array([HOME[n] for n in JOINT_NAMES])


def legs_together(rng, n):
    t = home() + rng.uniform(-0.3, 0.3, (n, 14))
    t[:, 1] -= 0.4
    t[:, 10] += 0.4
    t[:, 0] += 0.3
    t[:, 9] -= 0.3
    return t


def probe_record(model_path, fp64, targets, steps, limit=0.0, motor=None, root=None,
                 iterations=ITER):
    """Run the reference core from reset(targets[0] pose) and record."""
    p = ReferenceProbe(model_path, DT, iterations, fp64)
    p.reset(targets, np.zeros(6) if root is None else root)
    rec = {k: [] for k in ("step", "bodies", "joints", "diag", "joint_state", "loads",
                           "forces", "stats", "counts", "colors", "color_count",
                           "contact_ints", "contact_reals", "contact_count")}
    offset = np.array([0.001, -0.002, 0.003])
    for s in range(1, steps + 1):
        if motor is not None:
            p.set_motor(motor[s - 1])
            p.advance(1)
        else:
            p.step(targets, None, 1, KP, limit)
        if s in CHECKPOINTS or s <= 3:
            b, j, d = p.snapshot()
            ints, reals = p.contacts(64)
            c, cc = p.colors()
            rec["step"].append(s)
            rec["bodies"].append(b)
            rec["joints"].append(j)
            rec["diag"].append(d)
            rec["joint_state"].append(p.joint_state())
            rec["loads"].append(p.generalized_loads(offset))
            rec["forces"].append(p.contact_forces())
            rec["stats"].append(p.self_contact_stats())
            rec["counts"].append(p.contact_counts())
            rec["colors"].append(c)
            rec["color_count"].append(cc)
            pad_i = np.full((64, 6), -9, np.int32)
            pad_r = np.zeros((64, 26))
            pad_i[: len(ints)] = ints
            pad_r[: len(reals)] = reals
            rec["contact_ints"].append(pad_i)
            rec["contact_reals"].append(pad_r)
            rec["contact_count"].append(len(ints))
    return {k: np.array(v) for k, v in rec.items()}


def duck_sim_record(model_path, steps, iterations=ITER, dt=DT, summary=False):
    out = subprocess.run([str(REF_DIR / "duck_sim"), str(model_path), "--steps", str(steps),
                          "--dt", str(dt), "--iterations", str(iterations), "--output",
                          "/dev/stdout"], capture_output=True, text=True, check=True).stdout
    rows = [r for r in csv.reader(io.StringIO(out)) if r and r[0].isdigit()]
    by_step = {}
    for r in rows:
        by_step.setdefault(int(r[0]), []).append([float(v) for v in r[3:]])
    trajectory = np.array([by_step[s] for s in range(steps + 1)])
    if summary:
        return trajectory, [line for line in out.splitlines() if line.startswith("{")][-1]
    return trajectory


SOLVER_CHECKPOINTS = (0, 1, 2, 3, 10, 50, 100, 150, 200)


def solver_pd_fixtures(tmp):
    """src/solver.cpp (duck_sim) with the explicit PD drive of the standing
    biped (kp = 8 from the file, HOME targets): 200 steps at the single-env
    workload's dt = 5 ms, where it diverges, and at dt = 1 ms, where it stays
    bounded; checkpoints of the trajectory and duck_sim's JSON summary."""
    text, _ = model_text()
    path = tmp / "standing_pd.duck"
    path.write_text(text)
    for dt, name in ((0.005, "solver_standing_kp8_dt5ms_fp64"),
                     (0.001, "solver_standing_kp8_dt1ms_fp64")):
        trajectory, summary = duck_sim_record(path, 200, dt=dt, summary=True)
        np.savez_compressed(HERE / f"{name}.npz", model=np.array(text), dt=dt,
                            step=np.array(SOLVER_CHECKPOINTS),
                            trajectory=trajectory[list(SOLVER_CHECKPOINTS)],
                            summary=np.array(summary))
        print("wrote", name, flush=True)


def main():
    if not (REF_DIR / "ref_probe.so").exists():
        raise SystemExit("oracle/_ref is not built: make -C oracle ref")
    if sys.argv[1:] == ["--solver-pd"]:
        with tempfile.TemporaryDirectory() as tmp:
            solver_pd_fixtures(Path(tmp))
        return
    rng = np.random.default_rng(20260927)
    with tempfile.TemporaryDirectory() as tmp:
        tmp = Path(tmp)
        cases = {}

        def model(name, **kw):
            text, _ = model_text(**kw)
            path = tmp / f"{name}.duck"
            path.write_text(text)
            return path, text

        standing, standing_text = model("standing")
        for fp64 in (False, True):
            cases[f"standing_home_fp{64 if fp64 else 32}"] = (standing_text, dict(
                fp64=fp64, targets=home(), limit=0.0, **probe_record(standing, fp64, home(), 200)))
        selfc, selfc_text = model("selfc", self_contact=True)
        t = legs_together(rng, 2)
        for i in range(2):
            cases[f"selfc_limits_fp64_{i}"] = (selfc_text, dict(
                fp64=True, targets=t[i], limit=0.5, **probe_record(selfc, True, t[i], 40, 0.5)))
        cases["selfc_limits_fp32_0"] = (selfc_text, dict(
            fp64=False, targets=t[0], limit=0.5, **probe_record(selfc, False, t[0], 40, 0.5)))
        friction, friction_text = model("friction", frictionloss=0.02)
        motor = np.stack([rng.uniform(-0.2, 0.2, (40, 14)), rng.uniform(0, 0.05, (40, 14)),
                          rng.uniform(0, 0.3, (40, 14))], -1)
        cases["friction_motor_fp64"] = (friction_text, dict(
            fp64=True, targets=home(), limit=0.0, motor=motor,
            **probe_record(friction, True, home(), 40, motor=motor)))
        tgt = home() + rng.uniform(-0.3, 0.3, 14)
        cases["friction_pd_fp32"] = (friction_text, dict(
            fp64=False, targets=tgt, limit=0.3, **probe_record(friction, False, tgt, 40, 0.3)))
        for name, (text, data) in cases.items():
            np.savez_compressed(HERE / f"kernel_{name}.npz", model=np.array(text), **data)
            print("wrote", name, flush=True)
        # Independent FP64 solver (solver.cpp) trajectories from the file state.
        limp, limp_text = model("limp", kp=0.0, frictionloss=0.01)
        np.savez_compressed(HERE / "solver_limp_fp64.npz", model=np.array(limp_text),
                            trajectory=duck_sim_record(limp, 150))
        pend = HERE / "pendulum.duck"
        np.savez_compressed(HERE / "solver_pendulum_fp64.npz", model=np.array(pend.read_text()),
                            trajectory=duck_sim_record(pend, 400))
        print("wrote solver trajectories", flush=True)


if __name__ == "__main__":
    main()
