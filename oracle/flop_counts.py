"""Exact floating-point work per environment-step of the benchmark workloads
(test infrastructure, not product code): oracle/op_count -- the oracle's
float64 step instantiated with an operation-counting number type -- driven
with each workload's seeded inputs (duck_gym_amd.workloads) for a sample of
environments, averaged over the steps of the benchmark's timed window.

    python oracle/flop_counts.py [--envs 8] [--steps 300] [--first 100]

prints one `flop_per_env_step.<workload>: N` line per workload (add, sub,
mul, div and sqrt; transcendental calls are listed apart), the figures
bench.py divides by the kernel time for its FP32-VALU roofline:

  home   fixed HOME, 10 iterations (the headline workload)
  sweep  HOME + U(-0.3, 0.3) targets redrawn every 4 steps, body contacts,
         ground friction U(0.5, 1.2), 10 iterations
  drop   drop/jump starts (height, rotation, velocity, mass scale), 15
         iterations, HOME targets
  servo  the BAM servo loop's motor channels (the servo oracle's XL330 model
         with a 2-substep delay on the sweep's targets, one draw per 4
         substeps), body contacts; the physics step only (the actuator and
         its Newton-Euler load pass are a few thousand more per substep)
"""

from __future__ import annotations

import argparse
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

DT, KP, SEED = 0.005, 8.0, 20260927


def count(model, iterations, start, controls, first):
    """op_count's per-step averages for one environment: `start` = (q, root,
    ext), `controls` = one ('T', targets) or ('M', motor[J,3]) per step."""
    q, root, ext = start
    lines = [" ".join(repr(float(v)) for v in (*q, *root, *ext))]
    for kind, values in controls:
        lines.append(kind + " " + " ".join(repr(float(v)) for v in np.ravel(values)))
    out = subprocess.run([str(ROOT / "oracle" / "op_count"), str(model), str(len(controls)),
                          str(iterations), str(DT), str(KP), "-", str(first)],
                         input="\n".join(lines) + "\n", capture_output=True, text=True,
                         check=True).stdout
    fields = dict(line.split() for line in out.splitlines())
    if int(fields["failed"]):
        raise RuntimeError(f"{model}: the counted environment failed")
    return {k: float(v) for k, v in fields.items() if k != "failed"}


def main():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--envs", type=int, default=8)
    p.add_argument("--steps", type=int, default=300)
    p.add_argument("--first", type=int, default=100)
    args = p.parse_args()
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "op_count"], check=True)
    from duck_gym_amd import workloads as W
    from duck_gym_amd.microduck import model_text, write_model

    meta = model_text()[1]
    home = np.array(meta["home"])
    envs = np.arange(args.envs)
    zero_root, keep = np.zeros(6), np.array([-1.0, 1.0, 0.0, 0.0, 0.0])
    results = {}
    with tempfile.TemporaryDirectory() as tmp:
        plain = write_model(Path(tmp) / "plain")
        pairs = write_model(Path(tmp) / "pairs", self_contact=True)
        runs = {"home": [], "sweep": [], "drop": [], "servo": []}
        for e in envs:
            runs["home"].append(count(plain, 10, (home, zero_root, keep),
                                      [("T", home)] * args.steps, args.first))
            ext = keep.copy()
            ext[0] = W.ground_friction(np.array([e]), SEED)[0]
            sweep = [("T", W.servo_targets(home, np.array([e]), s, SEED)[0])
                     for s in range(args.steps)]
            runs["sweep"].append(count(pairs, 10, (home, zero_root, ext), sweep, args.first))
            q, root, ext = W.drop_start(np.array([e]), SEED, home, meta["root_height"])
            runs["drop"].append(count(plain, 15, (q[0], root[0], ext[0]),
                                      [("T", home)] * args.steps, args.first))
        from oracle.oracle import Oracle
        from oracle.servo_oracle import ServoOracle

        from duck_gym_amd.servo import SYNTHETIC_SUPPLY, SYNTHETIC_XL330

        for e in envs:
            o = Oracle(pairs, DT, 10, True)
            o.reset(home)
            so = ServoOracle(o, home, [0.0, 0.0, 0.01], 2, parameters=SYNTHETIC_XL330,
                             **SYNTHETIC_SUPPLY)
            motors = [("M", so.substep(W.servo_targets(home, np.array([e]), 4 * (s // 4),
                                                       SEED)[0]))
                      for s in range(args.steps)]
            runs["servo"].append(count(pairs, 10, (home, zero_root, keep), motors, args.first))
        for name, rows in runs.items():
            results[name] = {k: float(np.mean([r[k] for r in rows])) for k in rows[0]}
    print(f"# op_count over {args.envs} envs, steps {args.first + 1}-{args.steps} "
          f"(python oracle/flop_counts.py --envs {args.envs} --steps {args.steps} "
          f"--first {args.first})")
    for name, r in results.items():
        print(f"flop_per_env_step.{name}: {r['flop_per_step']:.0f}  "
              f"(add/sub {r['add_sub']:.0f}, mul {r['mul']:.0f}, div {r['div']:.0f}, "
              f"sqrt {r['sqrt']:.0f}; transcendental calls {r['transcendental']:.0f})")


if __name__ == "__main__":
    main()
