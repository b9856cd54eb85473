"""The oracle's threaded batch driver (oracle/avbd_oracle.cpp `oracle_batch_*`,
oracle.OracleBatch): the reference's CPU batch semantics
(src/cuda/cpu_bindings.cpp:20-168, CpuBatch32/64) over the restatement.
Pinned against the single-environment oracle, across worker counts, and
against the reference's own CpuBatch32/64 compiled in place (oracle/_ref)
where that build exists; its parameter checks and failure rules follow
cpu_bindings.cpp:35-111."""

import sys
from pathlib import Path

import numpy as np
import pytest

from oracle.oracle import Oracle, OracleBatch

REF_DIR = Path(__file__).resolve().parents[1] / "oracle" / "_ref"
DT, ITER, KP, LIMIT = 0.005, 10, 8.0, 1e9


def _inputs(home, n, steps, seed):
    rng = np.random.default_rng(seed)
    return [home + rng.uniform(-0.3, 0.3, (n, 14)) for _ in range(steps)]


def _run(batch, home, plan):
    n = batch.num_envs
    batch.reset(np.ones(n, bool), np.tile(home, (n, 1)), np.zeros((n, 6)))
    for t in plan:
        batch.step(t, np.zeros((n, 3)), 1, KP, LIMIT)
    return batch.state()


@pytest.mark.parametrize("fp64", [False, True])
def test_batch_equals_single_envs_and_any_worker_count(models, home, fp64):
    n, plan = 6, _inputs(home, 6, 12, 3)
    one = _run(OracleBatch(models["selfc"], n, DT, ITER, threads=1, fp64=fp64), home, plan)
    four = _run(OracleBatch(models["selfc"], n, DT, ITER, threads=4, fp64=fp64), home, plan)
    for a, b in zip(one, four):
        assert np.array_equal(a, b)
    for e in range(n):
        o = Oracle(models["selfc"], DT, ITER, fp64=fp64)
        o.reset(home)
        for t in plan:
            o.step(t[e], np.zeros(3), 1, KP, LIMIT)
        b, j, d = o.snapshot()
        assert np.array_equal(b, one[0][e]) and np.array_equal(j, one[1][e])
        assert np.array_equal(d, one[2][e])


def test_motor_steps_equal_single_envs(models, home):
    n = 4
    rng = np.random.default_rng(8)
    batch = OracleBatch(models["friction"], n, DT, ITER, threads=2)
    batch.reset(np.ones(n, bool), np.tile(home, (n, 1)), np.zeros((n, 6)))
    singles = []
    for _ in range(n):
        o = Oracle(models["friction"], DT, ITER)
        o.reset(home)
        singles.append(o)
    for _ in range(5):
        motor = np.stack([rng.uniform(-0.1, 0.1, (n, 14)), rng.uniform(0, 0.02, (n, 14)),
                          rng.uniform(0, 0.05, (n, 14))], axis=-1)
        batch.step_motor(motor, np.zeros((n, 3)))
        for e, o in enumerate(singles):
            o.set_motor(motor[e])
            if not o.failed:
                o.advance(1)
    b, j, d = batch.state()
    for e, o in enumerate(singles):
        sb, sj, sd = o.snapshot()
        assert np.array_equal(sb, b[e]) and np.array_equal(sj, j[e]) and np.array_equal(sd, d[e])


def test_parameter_checks_and_failures(models, home):
    for n, threads in ((0, 1), (4097, 1), (2, 0), (2, 65)):
        with pytest.raises(ValueError, match="Invalid batch parameters"):
            OracleBatch(models["standing"], n, DT, ITER, threads=threads)
    batch = OracleBatch(models["standing"], 3, DT, ITER, threads=3)
    batch.reset(np.ones(3, bool), np.tile(home, (3, 1)), np.zeros((3, 6)))
    target, forces = np.tile(home, (3, 1)), np.zeros((3, 3))
    for substeps, kp, limit in ((0, KP, LIMIT), (1, -1.0, LIMIT), (1, KP, 0.0), (1, KP, np.inf)):
        with pytest.raises(ValueError, match="Invalid controls"):
            batch.step(target, forces, substeps, kp, limit)
    # a non-finite target fails its environment only; a masked reset with a
    # non-finite pose fails it too, and a finite one revives it
    target[1, 4] = np.nan
    batch.step(target, forces, 1, KP, LIMIT)
    before = batch.state()[0].copy()
    batch.step(np.tile(home, (3, 1)), forces, 1, KP, LIMIT)
    after = batch.state()[0]
    assert np.array_equal(after[1], before[1])                   # failed: no step
    assert not np.array_equal(after[0], before[0])               # the others step
    root = np.zeros((3, 6))
    root[2, 0] = np.nan
    batch.reset(np.array([False, True, True]), np.tile(home, (3, 1)), root)
    moved = batch.state()[0]
    batch.step(np.tile(home, (3, 1)), forces, 1, KP, LIMIT)
    after = batch.state()[0]
    assert not np.array_equal(after[1], moved[1])                # revived: steps
    assert np.array_equal(after[2], moved[2])                    # failed by reset


@pytest.mark.skipif(not any(REF_DIR.glob("_duck_reference*.so")), reason="reference build absent")
@pytest.mark.parametrize("fp64", [False, True])
def test_batch_equals_the_reference_cpu_batch(models, home, fp64):
    """Bit for bit against the reference's own CpuBatch32/64 on the same
    inputs (body contacts included)."""
    sys.path.insert(0, str(REF_DIR))
    import _duck_reference

    n, plan = 5, _inputs(home, 5, 15, 11)
    dtype = np.float64 if fp64 else np.float32
    ref = (_duck_reference.CpuBatch64 if fp64 else _duck_reference.CpuBatch32)(
        str(models["selfc"]), n, DT, ITER, 2)
    ref.reset(np.ones(n, bool), np.tile(home, (n, 1)).astype(dtype), np.zeros((n, 6), dtype))
    for t in plan:
        ref.step(t.astype(dtype), np.zeros((n, 3), dtype), 1, KP, LIMIT)
    ours = _run(OracleBatch(models["selfc"], n, DT, ITER, threads=2, fp64=fp64), home,
                [t.astype(dtype).astype(np.float64) for t in plan])
    for a, b in zip(ref.state(), ours):
        assert np.array_equal(np.asarray(a, dtype=np.float64), b)
