"""The seeded workload inputs: deterministic, subset-consistent (an oracle
env sees exactly what the same env of the full batch sees) and in range."""

import numpy as np

from duck_gym_amd import workloads as W
from duck_gym_amd.microduck import HOME, JOINT_NAMES, model_text

HOME_V = np.array([HOME[n] for n in JOINT_NAMES])


def test_uniform_is_deterministic_subset_consistent_and_uniform():
    envs = np.arange(4096)
    a = W.uniform(7, envs, 3, 5)
    assert np.array_equal(a, W.uniform(7, envs, 3, 5))
    assert np.array_equal(a[[5, 17, 4000]], W.uniform(7, np.array([5, 17, 4000]), 3, 5))
    assert not np.array_equal(a, W.uniform(8, envs, 3, 5))
    assert not np.array_equal(a, W.uniform(7, envs, 4, 5))
    assert 0 <= a.min() and a.max() < 1
    counts = np.histogram(a, bins=8, range=(0, 1))[0]
    assert counts.min() > 4096 / 8 * 0.8  # roughly flat
    z = W.normal(7, envs, 0, 1)
    assert abs(z.mean()) < 0.08 and abs(z.std() - 1) < 0.06


def test_servo_targets_hold_for_a_period():
    envs = np.arange(64)
    t0 = W.servo_targets(HOME_V, envs, 0, 1)
    assert np.array_equal(t0, W.servo_targets(HOME_V, envs, 3, 1))
    assert not np.array_equal(t0, W.servo_targets(HOME_V, envs, 4, 1))
    assert np.abs(t0 - HOME_V).max() <= 0.3


def test_drop_start_ranges():
    meta = model_text()[1]
    envs = np.arange(16384)
    q, root, ext = W.drop_start(envs, 3, HOME_V, meta["root_height"])
    height = root[:, 2] + meta["root_height"]
    assert 0.15 <= height.min() and height.max() <= 0.35
    assert np.abs(root[:, 3:6]).max() <= 0.5 and np.all(root[:, :2] == 0)
    assert np.all(ext[:, 0] == -1) and 0.9 <= ext[:, 1].min() and ext[:, 1].max() <= 1.1
    assert abs(ext[:, 2:5].std() - 0.5) < 0.02
    mu = W.ground_friction(envs, 3)
    assert 0.5 <= mu.min() and mu.max() <= 1.2
