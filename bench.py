"""Physics env-steps/s of the batched AVBD env step on one MI355X.

Workload: the MicroDuck-like biped (16 bodies, 14 hinges, kp 8, kd 0.2,
ground friction 0.8), 4096 environments in float32, held at the fixed HOME
pose with zero action, dt = 1/200 s, 10 AVBD iterations per step.  One
"step" is one physics step of every environment: one launch of the fused
step kernel (`CudaBatch.step(target, forces, 1, kp, 0)`), inputs resident in
HBM.  W untimed warm-up steps follow a reset, then exactly K steps are timed
between device synchronisations; the kernel's own duration is measured with
HIP events on the launch stream.

The JSON line also carries
  roofline      algorithmic HBM bytes per launch of the step kernel (the
                persistent state read and written once per step plus the
                controls read) over its measured duration, against 8 TB/s;
                `traffic` is the measured HBM bytes per launch from
                rocprofv3 FETCH_SIZE/WRITE_SIZE when recorded in profiles/.
                `bound` says what limits the kernel: neither HBM nor MFMA,
                but the latency of one wave's dependent FP32 VALU chain (one
                wave per SIMD, fixed by the LDS each workgroup stages);
                `valu` gives the exact floating-point work per env-step of
                the reference algorithm (oracle/op_count over the timed
                window, recorded in profiles/flop_counts.md) over the kernel
                time against the FP32 vector peak (157.3 TFLOP/s) and against
                the 78.6 TFLOP/s reachable without packed FP32; `occupancy`
                the step kernel's registers, LDS, scratch and resident waves
                as the runtime reports them
  cpu_baseline  the reference's own CPU build of the same solver core
                (src/cuda/kernel.cuh via src/cuda/cpu_bindings.cpp, compiled
                in place into oracle/_ref) on a bounded sample of the
                4096-env workload over the host's CPUs, plus the single-env
                float64 figure and src/solver.cpp's own CLI on that env
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "physics env-steps/s at 4096 envs on 1 MI355X; achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3          # MI355X dense FP32 vector, packed FP32 included
FP32_NONPACKED_PEAK_TFLOPS = 78.6  # one wave64 FMA per SIMD per quad-cycle
ENVS, DT, ITERATIONS, KP = 4096, 0.005, 10, 8.0
BOUND = ("latency: one wave per SIMD (the LDS each workgroup stages allows no second), "
         "whose dependent FP32 VALU chain and LDS round trips set the step time; neither "
         "HBM- nor MFMA-bound (profiles/advance_kernel_microduck_4096_counters.md)")


def state_bytes_per_env(contacts, bodies=15, joints=14):
    """Minimal persistent state of one env (float32): bodies (x, q, v, w),
    joint multipliers/penalties (lambda 7, penalty 7, lambdaF, penaltyF),
    the contact warm-start cache (13 words per live contact: shape and
    feature id, local point, ground anchor, c0, lambda 3, penalty 3) and
    count/flag."""
    return bodies * 13 * 4 + joints * 16 * 4 + 52 * contacts + 8


SELF_CONTACT_BYTES = 68  # normal, two local points, lambda 3, penalty 3, c0, ids


def algorithmic_bytes_per_launch(envs, contacts, model_bytes, self_contacts=0.0):
    """State read + written once (with `self_contacts` live body-contact cache
    entries per env), targets [J] + forces [3] read, model once."""
    per_env = 2 * (state_bytes_per_env(contacts) + SELF_CONTACT_BYTES * self_contacts) + \
        (14 + 3) * 4
    return envs * per_env + model_bytes


def servo_bytes_per_env(contacts, self_contacts, joints=14, feet=2):
    """One fused servo substep of one env: the persistent state read and
    written once, plus the actuator's buffers -- the ring slot written and the
    delayed one read, the targets and root offset read, previous raw/applied
    torques read and written, the motor channels and supply written, the
    self-contact maxima read and written, the refresh outputs written (root
    gravity, angular, linear and origin velocity; per foot the force, site
    position and velocity) and the air/contact timers read and written."""
    state = 2 * (state_bytes_per_env(contacts) + SELF_CONTACT_BYTES * self_contacts)
    actuator = (2 * joints + joints + 3 + 2 * 2 * joints + 3 * joints + 1 + 2 * 2
                + 4 * 3 + feet * 9 + 2 * 2 * feet) * 4 + 2  # + the initialized flag R/W
    return state + actuator


def measured_traffic():
    """HBM bytes per launch recorded from rocprofv3 counters, if present."""
    path = ROOT / "profiles" / "advance_kernel_microduck_4096_counters.md"
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text())
    return float(m.group(1)) if m else None


def measured_valu():
    """The step kernel's VALU counters recorded from rocprofv3 in profiles/
    (fixed HOME, 4096 envs): the fraction of the wave's life issuing VALU
    instructions, the active lanes per VALU instruction, and the FP32 lane
    operations it executes per env-step."""
    path = ROOT / "profiles" / "advance_kernel_microduck_4096_counters.md"
    if not path.exists():
        return None
    text, out = path.read_text(), {}
    for key in ("valu_busy_fraction", "valu_lanes_active", "executed_fp32_lane_flop_per_env_step"):
        m = re.search(rf"^{key}:\s*([0-9.eE+]+)", text, re.M)
        if m:
            out[key] = float(m.group(1))
    return out or None


def flop_per_env_step(workload):
    """Exact floating-point operations per env-step of the reference
    algorithm on `workload` (oracle/op_count over the timed window, recorded
    in profiles/flop_counts.md by oracle/flop_counts.py), or None."""
    path = ROOT / "profiles" / "flop_counts.md"
    if not path.exists():
        return None
    m = re.search(rf"flop_per_env_step\.{workload}:\s*([0-9.]+)", path.read_text())
    return float(m.group(1)) if m else None


def roofline(kernel_s, algo_bytes, env_steps_per_launch, flop_workload, occupancy,
             traffic=None, kernel="advanceKernel"):
    """The roofline object of a bench line for the dominant kernel: HBM
    (the metric's figures), the FP32-VALU fraction and the occupancy."""
    achieved = algo_bytes / kernel_s / 1e9
    out = {
        "bound": "latency",
        "bound_detail": BOUND,
        "achieved": achieved,
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": achieved / HBM_PEAK_GBS,
        "traffic": traffic,
        "kernel": kernel,
        "kernel_ms": kernel_s * 1e3,
        "algorithmic_bytes_per_launch": algo_bytes,
        "valu": None,
        "occupancy": occupancy,
    }
    flop = flop_per_env_step(flop_workload)
    if flop is not None:
        tflops = flop * env_steps_per_launch / kernel_s / 1e12
        out["valu"] = {
            "flop_per_env_step": flop,
            "flop_source": f"oracle/op_count on the {flop_workload} workload "
                           "(profiles/flop_counts.md)",
            "achieved_tflops": tflops,
            "peak_tflops": FP32_PEAK_TFLOPS,
            "frac": tflops / FP32_PEAK_TFLOPS,
            "peak_nonpacked_tflops": FP32_NONPACKED_PEAK_TFLOPS,
            "frac_nonpacked": tflops / FP32_NONPACKED_PEAK_TFLOPS,
        }
    return out


def host_facts():
    """The CPU the baseline ran on: logical CPUs, those this process may use,
    the model name, and the reference build's compiler and flags."""
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    info = ROOT / "oracle" / "_ref" / "BUILD_INFO"
    build = info.read_text().splitlines() if info.exists() else [None, None]
    return {"nproc": os.cpu_count(), "available_cpus": threads, "cpu_model": model,
            "compiler": build[0], "flags": build[1] if len(build) > 1 else None}


def cpu_baseline(model, home, seconds_budget=12.0):
    """The reference's own CPU build of the solver core, timed on this host:

    batch   kernel.cuh's CPU batch (CpuBatch32, src/cuda/cpu_bindings.cpp,
            compiled in place into oracle/_ref) on the same 4096-env workload,
            env-striped over every CPU this process may use (capped by
            OMP_NUM_THREADS where set: a GPU box grants 16 per GPU), for about
            `seconds_budget` seconds;
    single  one env in float64 on one thread for 200 steps (CpuBatch64),
            timed around step() only, as src/main.cpp:63-68 times its solver;
    solver  src/solver.cpp's own CLI (duck_sim) on the same env: its steps/s
            and where the root ends -- its explicit PD drive diverges at
            kp = 8, dt = 5 ms;
    port    the oracle's own threaded batch (oracle.OracleBatch, the same
            CpuBatch semantics over this repository's restatement) on the
            same workload and threads, for about a third of the budget.
    The reference build is required: without oracle/_ref this raises."""
    import json as _json
    import subprocess

    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle" / "_ref"))
    try:
        import _duck_reference
    except ImportError as e:
        raise RuntimeError("the reference CPU build is missing (make -C oracle ref): "
                           f"{e}") from e
    facts = host_facts()
    threads = facts["available_cpus"] or 1
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    threads = max(1, min(64, threads))  # CpuBatch accepts 1-64 threads
    envs = ENVS
    batch = _duck_reference.CpuBatch32(str(model), envs, DT, ITERATIONS, threads)
    q = np.tile(home, (envs, 1)).astype(np.float32)
    batch.reset(np.ones(envs, bool), q, np.zeros((envs, 6), np.float32))
    forces = np.zeros((envs, 3), np.float32)
    batch.step(q, forces, 1, KP, 1e9)  # warm; limit 1e9 = uncapped PD torques
    steps, start = 0, time.perf_counter()
    while time.perf_counter() - start < seconds_budget:
        batch.step(q, forces, 1, KP, 1e9)
        steps += 1
    elapsed = time.perf_counter() - start

    single = _duck_reference.CpuBatch64(str(model), 1, DT, ITERATIONS, 1)
    q1 = home[None].astype(np.float64)
    single.reset(np.ones(1, bool), q1, np.zeros((1, 6)))
    f1 = np.zeros((1, 3))
    spent = 0.0
    for _ in range(200):
        t0 = time.perf_counter()
        single.step(q1, f1, 1, KP, 1e9)
        spent += time.perf_counter() - t0

    from oracle.oracle import OracleBatch

    port = OracleBatch(model, envs, DT, ITERATIONS, threads=threads)
    port.reset(np.ones(envs, bool), np.tile(home, (envs, 1)), np.zeros((envs, 6)))
    q64, f64 = np.tile(home, (envs, 1)), np.zeros((envs, 3))
    port.step(q64, f64, 1, KP, 1e9)
    port_steps, start = 0, time.perf_counter()
    while time.perf_counter() - start < seconds_budget / 3:
        port.step(q64, f64, 1, KP, 1e9)
        port_steps += 1
    port_elapsed = time.perf_counter() - start
    del port

    run = subprocess.run([str(ROOT / "oracle" / "_ref" / "duck_sim"), str(model), "--steps", "200",
                          "--dt", str(DT), "--iterations", str(ITERATIONS), "--output",
                          "/dev/stdout"], capture_output=True, text=True, check=True).stdout
    summary = _json.loads([line for line in run.splitlines() if line.startswith("{")][-1])
    rows = [line.split(",") for line in run.splitlines() if line[:1].isdigit()]
    roots = {int(r[0]): np.array([float(v) for v in r[3:6]]) for r in rows if r[2] == "1"}
    return {
        "value": envs * steps / elapsed, "unit": "env-steps/s", "cores": threads,
        "kind": "reference",
        "sample": (f"{envs} envs x {steps} steps of src/cuda/kernel.cuh's CPU build (CpuBatch32, "
                   f"float32, {threads} threads), same model/HOME/dt/iterations"),
        "host": facts,
        "single_env_fp64": {
            "value": 200 / spent, "unit": "steps/s", "steps": 200, "threads": 1,
            "sample": "CpuBatch64 (kernel.cuh, float64), 1 env at HOME, timed around step()"},
        "solver_cpp": {
            "steps_per_second": summary["steps_per_second"], "steps": 200,
            "root_displacement_m": float(np.linalg.norm(roots[200] - roots[0])),
            "unconverged_steps": summary["unconverged_steps"],
            "note": "src/solver.cpp (duck_sim): its explicit PD drive diverges at kp 8, dt 5 ms"},
        "port": {
            "value": envs * port_steps / port_elapsed, "unit": "env-steps/s", "threads": threads,
            "sample": (f"{envs} envs x {port_steps} steps of oracle.OracleBatch (this repository's "
                       "restatement, CpuBatch semantics, float32)")},
    }


def other_workload(args):
    """env-steps/s of the non-headline workloads (same timing protocol)."""
    import numpy as np
    import torch

    from duck_gym_amd import CudaBatch
    from duck_gym_amd import workloads as W
    from duck_gym_amd.microduck import model_text, write_model

    seed, kp = 20260927, KP
    meta = model_text()[1]
    home = np.array(meta["home"])
    tmp = tempfile.TemporaryDirectory()
    dev = torch.device("cuda:0")
    config = {}
    if args.workload in ("sweep", "drop"):
        sweep = args.workload == "sweep"
        E = args.envs or (4096 if sweep else 16384)
        iterations = 10 if sweep else 15
        model = write_model(Path(tmp.name) / "m", self_contact=sweep)
        batch = CudaBatch(model, E, DT, iterations, 0, False)
        envs = np.arange(E)
        if sweep:
            q, root = np.tile(home, (E, 1)), np.zeros((E, 6))
            ext = np.zeros((E, 5))
            ext[:, 0], ext[:, 1] = W.ground_friction(envs, seed), 1.0
        else:
            q, root, ext = W.drop_start(envs, seed, home, meta["root_height"])
        t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)  # noqa: E731
        batch.reset(torch.ones(E, dtype=torch.bool, device=dev), t(q), t(root), t(ext))
        forces = torch.zeros(E, 3, device=dev)
        # Targets for every step, resident in HBM before timing.
        blocks = [t(W.servo_targets(home, envs, 4 * k, seed) if sweep else np.tile(home, (E, 1)))
                  for k in range((args.warmup + args.steps) // 4 + 1)]
        for s in range(args.warmup):
            batch.step(blocks[s // 4], forces, 1, kp, 0.0)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        begin.record(stream)
        for s in range(args.warmup, args.warmup + args.steps):
            batch.step(blocks[s // 4], forces, 1, kp, 0.0)
        end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        kernel_s = begin.elapsed_time(end) / 1000.0 / args.steps
        failed = int((batch.state()[2][:, 5] != 0).sum())
        value = E * args.steps / wall
        counts = batch.contact_counts().float().mean(0)
        algo = algorithmic_bytes_per_launch(E, float(counts[0]), 4 * 4096, float(counts[1]))
        line_roofline = roofline(kernel_s, algo, E, args.workload, batch.kernel_info())
        config = {"workload": "servo-target sweep, HOME + U(-0.3, 0.3) every 4 steps, body "
                              "contacts between the leg chains, friction U(0.5, 1.2)" if sweep
                  else "drop/jump stress: base height U(0.15, 0.35) m, rotation +-0.5 rad, "
                       "velocity N(0, 0.5), masses x U(0.9, 1.1)",
                  "envs": E, "iterations": iterations, "dt_s": DT, "failed_envs": failed,
                  "live_contacts_per_env_at_end": [float(counts[0]), float(counts[1])]}
        ms = wall / args.steps * 1e3
    elif args.workload == "rollout":
        from duck_gym_amd.tensor_env import TensorEnv

        write_model(Path(tmp.name))
        E, substeps = args.envs or 32768, 4
        env = TensorEnv(Path(tmp.name), E, ITERATIONS, DT, substeps, seed=seed, task="rollout",
                        episode_seconds=10.0)
        torch.manual_seed(seed)
        policy = torch.nn.Sequential(
            torch.nn.Linear(48, 256), torch.nn.ELU(), torch.nn.Linear(256, 128), torch.nn.ELU(),
            torch.nn.Linear(128, 14)).to(dev)
        obs, _ = env.get_observations()
        stream = torch.cuda.current_stream()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.no_grad():
            for _ in range(args.warmup):
                obs, _, _, _ = env.step(policy(obs))
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            begin.record(stream)
            for _ in range(args.steps):
                obs, _, _, _ = env.step(policy(obs))
            end.record(stream)
            torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        value = E * args.steps * substeps / wall
        ms = wall / args.steps * 1e3
        # the whole control step (policy, task kernels and the 4-substep step
        # launch) on the stream, per physics step; the step kernel alone is in
        # the rocprofv3 trace (profiles/rollout_32768.md)
        control_s = begin.elapsed_time(end) / 1000.0 / args.steps
        counts = env.native.contact_counts().float().mean(0)
        # one step launch of `substeps` physics steps moves the state once;
        # the task kernels add the observation, the actions and last action,
        # reward and done flags
        algo = algorithmic_bytes_per_launch(E, float(counts[0]), 4 * 4096) + \
            E * (48 * 4 + 2 * 14 * 4 + 4 * 4)
        line_roofline = roofline(control_s, algo, E * substeps, "home",
                                 env.native.kernel_info(), kernel="control step (all kernels)")
        line_roofline["valu"] and line_roofline["valu"].update(
            flop_source="oracle/op_count on the HOME workload (the rollout's targets stay "
                        "near HOME; its trajectory is not counted separately)")
        config = {"workload": "tensor-env rollout: 48-wide observation, locomotion reward, reset "
                              "below 0.08 m, random-init 48-256-128-14 ELU policy",
                  "envs": E, "iterations": ITERATIONS, "dt_s": DT,
                  "physics_steps_per_control_step": substeps,
                  "control_steps_per_s": E * args.steps / wall}
    elif args.workload == "servo":
        from duck_gym_amd.servo import SYNTHETIC_SUPPLY, ServoLoop, servo_params

        E, substeps, lag = args.envs or 4096, 4, 2
        meta = model_text(self_contact=True)[1]
        model = write_model(Path(tmp.name) / "m", self_contact=True)
        names = meta["body_names"]
        feet = [names.index("left_foot"), names.index("right_foot")]
        envs = np.arange(E)
        t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)  # noqa: E731
        targets = [t(W.servo_targets(home, envs, 4 * k, seed))
                   for k in range(args.warmup + args.steps + 1)]
        timing = {}
        for fused in (True, False):
            batch = CudaBatch(model, E, DT, ITERATIONS, 0, False)
            batch.reset(torch.ones(E, dtype=torch.bool, device=dev), t(np.tile(home, (E, 1))),
                        t(np.zeros((E, 6))))
            loop = ServoLoop(batch, servo_params(**SYNTHETIC_SUPPLY, lag=lag), home,
                             [0.0, 0.0, 0.01], root_principal_quat=meta["root_iquat"], feet=feet,
                             foot_sites=[[0.01, 0.0, -0.006]] * 2, fused=fused)
            for k in range(args.warmup):
                loop.substeps(targets[k], substeps)
            torch.cuda.synchronize()
            stream = torch.cuda.current_stream()
            begin = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            begin.record(stream)
            for k in range(args.warmup, args.warmup + args.steps):
                loop.substeps(targets[k], substeps)
            end.record(stream)
            torch.cuda.synchronize()
            timing[fused] = time.perf_counter() - t0
            if fused:
                kernel_s = begin.elapsed_time(end) / 1000.0 / (args.steps * substeps)
                counts = batch.contact_counts().float().mean(0)
                algo = E * servo_bytes_per_env(float(counts[0]), float(counts[1])) + 4 * 4096
                line_roofline = roofline(kernel_s, algo, E, "servo",
                                         batch.kernel_info("servo_substep"),
                                         kernel="servoStepKernel")
        wall = timing[True]
        value = E * args.steps * substeps / wall
        ms = wall / args.steps * 1e3
        config = {"workload": "BAM servo substeps: XL330 actuator with a 2-substep delay and "
                              "load-dependent friction, servo targets HOME + U(-0.3, 0.3) per "
                              "control step, body contacts between the leg chains, refresh "
                              "quantities (root frame, foot forces and sites, timers) per "
                              "substep; one launch per substep",
                  "envs": E, "iterations": ITERATIONS, "dt_s": DT,
                  "physics_steps_per_control_step": substeps,
                  "unfused_env_steps_per_s": E * args.steps * substeps / timing[False],
                  "unfused": "servo kernel, motor step, state/contact-force/self-contact "
                             "queries and torch refresh arithmetic per substep"}
    elif args.workload == "train":
        line_roofline = None
        from duck_gym_amd.on_policy import STANDING, OnPolicyRunner
        from duck_gym_amd.tensor_env import TensorEnv

        write_model(Path(tmp.name))
        E, substeps = args.envs or 4096, 4
        env = TensorEnv(Path(tmp.name), E, ITERATIONS, DT, substeps, seed=seed, task="standing")
        torch.manual_seed(seed)
        runner = OnPolicyRunner(env, STANDING, device="cuda:0")
        runner.learn(args.warmup, init_at_random_ep_len=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        runner.learn(args.steps)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        T = STANDING["num_steps_per_env"]
        value = E * T * args.steps * substeps / wall
        ms = wall / args.steps * 1e3
        timed = runner.history[-args.steps:]
        config = {"workload": "PPO training iterations (configs/standing.json: 24 control steps "
                              "per env, 4 epochs x 4 mini-batches, 64-64 ELU actor and critic, "
                              "empirical normalisation) on the standing tensor env",
                  "envs": E, "iterations": ITERATIONS, "dt_s": DT,
                  "physics_steps_per_control_step": substeps,
                  "control_steps_per_s": E * T * args.steps / wall,
                  "collection_s_per_iteration": sum(h["collection_s"] for h in timed) / len(timed),
                  "update_s_per_iteration": sum(h["learning_s"] for h in timed) / len(timed)}
    return {"metric": f"physics env-steps/s ({args.workload} workload)", "value": value,
            "unit": "env-steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp32", "data": "synthetic", "config": config, "roofline": line_roofline}


def main():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--envs", type=int, default=None,
                   help="environments (default: 4096; the other workloads' own sizes)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--device-warmup", type=float, default=0.25, metavar="SECONDS",
                   help="home workload: seconds of the same step on a second batch before the "
                        "warm-up steps, so that the timed steps do not run at idle clocks (0: off)")
    p.add_argument("--substeps", type=int, default=1,
                   help="physics steps per kernel launch (default 1, the tensor-env contract; "
                        "K > 1 runs K steps inside one launch, the reference's chunked form)")
    p.add_argument("--workload", choices=("home", "sweep", "drop", "rollout", "train", "servo"),
                   default="home",
                   help="home: fixed HOME, 4096 envs (default, the headline line); sweep: "
                        "servo-target sweep with body contacts and per-env friction; drop: "
                        "drop/jump stress, 16384 envs, 15 iterations; rollout: tensor-env "
                        "rollout with a random MLP policy, 32768 envs; train: PPO iterations "
                        "of configs/standing.json on the standing tensor env, 4096 envs "
                        "(--steps and --warmup count learning iterations)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB (three times): the "
                        "reference dispatch for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = p.parse_args()
    if args.copy_calibration:
        import torch

        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4}), flush=True)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X (use --gpus 1): environments shard across "
              "GPUs with no exchange, so an N-GPU run is N independent runs of E/N envs "
              "each (bench.py --envs E/N).", file=sys.stderr)
        sys.exit(2)

    if args.workload != "home":
        print(json.dumps(other_workload(args)), flush=True)
        return

    import numpy as np
    import torch

    from duck_gym_amd import CudaBatch
    from duck_gym_amd.microduck import HOME, JOINT_NAMES, write_model

    home = np.array([HOME[n] for n in JOINT_NAMES])
    tmp = tempfile.TemporaryDirectory()
    model = write_model(Path(tmp.name) / "standing")
    E = args.envs or ENVS
    dev = torch.device("cuda:0")
    batch = CudaBatch(model, E, DT, ITERATIONS, 0, False)
    target = torch.tensor(np.tile(home, (E, 1)), dtype=torch.float32, device=dev)
    forces = torch.zeros(E, 3, dtype=torch.float32, device=dev)
    batch.reset(torch.ones(E, dtype=torch.bool, device=dev), target.clone(),
                torch.zeros(E, 6, device=dev))
    K = args.substeps
    if K < 1 or args.steps % K:
        raise SystemExit("--steps must be a positive multiple of --substeps")
    launches = args.steps // K
    # Device warm-up: the same step on a second batch of the same workload for
    # --device-warmup seconds, then the warm-up steps of the timed batch, then
    # the timed steps, with no idle gap between them.  A GPU that was idle runs
    # its first ~100 launches at lower clocks (the same clocks per wave take
    # longer), which a short window would time; the reference's own protocol
    # warms up for at least 10 GPU-seconds (scripts/benchmark_engines.py:485-
    # 500).  The timed batch is exactly --warmup steps past its reset.
    warm_launches = 0
    if args.device_warmup > 0:
        spare = CudaBatch(model, E, DT, ITERATIONS, 0, False)
        spare.reset(torch.ones(E, dtype=torch.bool, device=dev), target.clone(),
                    torch.zeros(E, 6, device=dev))
        torch.cuda.synchronize()
        t_warm = time.perf_counter()
        while time.perf_counter() - t_warm < args.device_warmup:
            for _ in range(20):
                spare.step(target, forces, K, KP, 0.0)
            warm_launches += 20
            torch.cuda.synchronize()
    for _ in range(max(1, args.warmup // K)):
        batch.step(target, forces, K, KP, 0.0)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    begin.record(stream)
    for _ in range(launches):
        batch.step(target, forces, K, KP, 0.0)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_s = begin.elapsed_time(end) / 1000.0 / launches  # per launch

    counts = batch.contact_counts()
    _, _, diag = batch.state()
    contacts = float(counts[:, 0].float().mean())
    failed = int((diag[:, 5] != 0).sum())
    finite = bool(torch.isfinite(batch.state()[0]).all())
    if failed or not finite:
        raise RuntimeError(f"invalid benchmark state: {failed} failed envs, finite={finite}")

    value = E * args.steps / wall
    model_bytes = 4 * 4096  # read-only model tables streamed per launch (upper bound)
    algo = algorithmic_bytes_per_launch(E, round(contacts), model_bytes)  # one state round trip
    traffic = measured_traffic() if E == ENVS and K == 1 else None
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": "MicroDuck-like biped (16 bodies, 14 hinges), fixed HOME pose, zero "
                        "action, ground contact",
            "envs": E,
            "iterations": ITERATIONS,
            "dt_s": DT,
            "kp": KP,
            "launch": "one physics step per kernel launch" if K == 1 else
                      f"{K} physics steps per kernel launch",
            "live_ground_contacts_per_env": contacts,
            "device_warmup": {"seconds": args.device_warmup, "launches": warm_launches,
                              "on": "a second batch of the same workload, right before the "
                                    "timed batch's warm-up steps; the timed batch is exactly "
                                    "`warmup` steps past its reset"},
        },
        "roofline": roofline(kernel_s, algo, E * K, "home", batch.kernel_info(), traffic),
        "cpu_baseline": None,
    }
    valu = line["roofline"]["valu"]
    counters = measured_valu() if E == ENVS and K == 1 else None
    if valu is not None and counters is not None:
        # the rocprofv3 counters of the same kernel and workload: the executed
        # FP32 lane operations at this run's kernel time
        counters["executed_tflops"] = \
            counters["executed_fp32_lane_flop_per_env_step"] * E / kernel_s / 1e12
        counters["source"] = "profiles/advance_kernel_microduck_4096_counters.md"
        valu["counters"] = counters
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(model, home)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
