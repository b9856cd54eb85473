"""The C++ interface include/duck/{math,solver}.hpp over libduck_hip.so
(tests/native/solver_api_test.cpp, built by __graft_entry__.build()):

* on the CPU: the math invariants of the reference's tests/math_test.cpp
  (exp/log, rotations, the SPD solve and its rejection of a singular system,
  hinge Jacobians against central differences);
* on the GPU: the Batch invariants of tests/state_test.cpp (identical
  environments agree bit for bit, a perturbed one differs, reset restores
  the file state and replays bit for bit, reload clears the multipliers, an
  empty batch is rejected) on the pendulum fixture and the MicroDuck-like
  biped, and duck::Solver::step -- the CudaBatch step with the controls
  held in the state -- against the oracle's kernel.cuh step in float64."""

import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PROGRAM = ROOT / "tests" / "native" / "solver_api_test"
GOLDEN = ROOT / "tests" / "golden"


def _run(*args, timeout=120):
    if not PROGRAM.exists():
        pytest.fail(f"{PROGRAM} is not built (python -c 'import __graft_entry__ as g; g.build()')")
    return subprocess.run([str(PROGRAM), *map(str, args)], capture_output=True, text=True,
                          timeout=timeout)


def test_math_invariants():
    out = _run("math")
    assert out.returncode == 0, out.stdout + out.stderr
    assert "math checks passed" in out.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["pendulum", "standing"])
def test_batch_invariants_on_the_gpu(models, which):
    model = GOLDEN / "pendulum.duck" if which == "pendulum" else models["standing"]
    out = _run("gpu", model)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "gpu checks passed" in out.stdout


@pytest.mark.gpu
def test_solver_step_matches_the_oracle(models):
    """duck::Solver on the biped from its file state with the file's hinge
    controls (kp 8, HOME targets, uncapped): 40 steps within 1e-9 of the
    oracle's kernel.cuh step (set_controls, then advance) in float64."""
    from oracle.oracle import Oracle

    model = models["standing"]
    out = _run("trace", model, 40)
    assert out.returncode == 0, out.stdout + out.stderr
    rows = np.array([[float(v) for v in line.split()] for line in out.stdout.splitlines()])
    o = Oracle(model, 0.005, 10, True)
    text = Path(model).read_text().splitlines()
    nb, nj = (int(v) for v in text[0].split()[2:4])
    joints = [line.split() for line in text[2 + nb: 2 + nb + nj]]
    target = np.array([float(j[29]) for j in joints])
    kp = {float(j[28]) for j in joints}
    assert kp == {8.0} and {float(j[30]) for j in joints} == {0.0}
    worst = 0.0
    for step in range(1, 41):
        o.set_controls(target, None, 8.0, 0.0)
        o.advance(1)
        bodies = o.snapshot()[0]
        mine = rows[rows[:, 0] == step][:, 2:9]
        worst = max(worst, float(np.abs(mine - bodies[:, :7]).max()))
    assert worst < 1e-9, worst
    print(f"duck::Solver vs oracle over 40 steps: {worst:.2e}")


@pytest.mark.gpu
def test_advance_with_held_controls_equals_step(models, home):
    """CudaBatch.advance (duck_advance) after a step repeats that step's
    controls: bit-identical to a second step with the same inputs."""
    from duck_gym_amd import CudaBatch

    E, dev = 6, "cuda:0"
    rng = np.random.default_rng(2)
    target = torch.tensor(home + rng.uniform(-0.3, 0.3, (E, 14)), dtype=torch.float32, device=dev)
    forces = torch.tensor(rng.normal(0, 0.2, (E, 3)), dtype=torch.float32, device=dev)
    a = CudaBatch(models["selfc"], E, 0.005, 10, 0, False)
    b = CudaBatch(models["selfc"], E, 0.005, 10, 0, False)
    for batch in (a, b):
        batch.reset(torch.ones(E, dtype=torch.bool, device=dev), target.clone(),
                    torch.zeros(E, 6, device=dev))
        batch.step(target, forces, 1, 8.0, 0.4)
    a.step(target, forces, 1, 8.0, 0.4)
    b.advance(1)
    assert torch.equal(a.export_state(), b.export_state())
