"""Seeded synthetic inputs for the benchmark and parity workloads.

Every draw is a pure function of (seed, env, block, index) through a
splitmix64 counter hash, so a host oracle and the GPU batch see identical
inputs for any subset of environments and any step, without sharing a
generator state:

  servo_targets   HOME + U(-a, a) per hinge, redrawn every `period` steps
  ground_friction U(0.5, 1.2) per environment
  drop_start      base height U(0.15, 0.35) m, base rotation vector
                  U(-0.5, 0.5)^3 rad, base velocity N(0, 0.5^2)^3 m/s and a
                  mass/inertia scale U(0.9, 1.1) per environment
"""

from __future__ import annotations

import numpy as np

_MASK = (1 << 64) - 1


def uniform(seed, env, block, index):
    """U[0, 1) for broadcastable integer arrays env, block, index (float64)."""
    env, block, index = np.broadcast_arrays(np.asarray(env, np.uint64),
                                            np.asarray(block, np.uint64),
                                            np.asarray(index, np.uint64))
    with np.errstate(over="ignore"):
        key = np.uint64(seed & _MASK)
        x = _vsplit(key ^ _vsplit(env + np.uint64(0x1000193)))
        x = _vsplit(x ^ _vsplit(block + np.uint64(0x2545F491)))
        x = _vsplit(x ^ _vsplit(index + np.uint64(0x61C88647)))
    return (x >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def _vsplit(x):
    x = np.asarray(x, np.uint64)
    x = x + np.uint64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def normal(seed, env, block, index):
    """N(0, 1) by Box-Muller from two counter draws."""
    u1 = uniform(seed, env, block, 2 * np.asarray(index))
    u2 = uniform(seed, env, block, 2 * np.asarray(index) + 1)
    return np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2 * np.pi * u2)


def servo_targets(home, envs, step, seed, amplitude=0.3, period=4):
    """[len(envs), J] targets HOME + U(-amplitude, amplitude), constant over
    each block of `period` steps."""
    envs = np.asarray(envs)
    J = len(home)
    u = uniform(seed, envs[:, None], step // period, np.arange(J)[None, :])
    return np.asarray(home)[None, :] + (2 * u - 1) * amplitude


def ground_friction(envs, seed, lo=0.5, hi=1.2):
    return lo + (hi - lo) * uniform(seed, np.asarray(envs), 0, 1000)


def drop_start(envs, seed, home, root_height):
    """(q [E,J], root [E,6], ext [E,5]) for the drop/jump stress start: the
    root offset puts the base COM at U(0.15, 0.35) m; ext keeps the shape
    friction (-1), scales masses and inertias by U(0.9, 1.1) and gives the
    whole body a linear velocity N(0, 0.5^2) per axis."""
    envs = np.asarray(envs)
    E = len(envs)
    q = np.tile(np.asarray(home, float), (E, 1))
    root = np.zeros((E, 6))
    root[:, 2] = 0.15 + 0.2 * uniform(seed, envs, 1, 0) - root_height
    root[:, 3:6] = 2 * uniform(seed, envs[:, None], 1, np.arange(1, 4)[None, :]) - 1
    root[:, 3:6] *= 0.5
    ext = np.zeros((E, 5))
    ext[:, 0] = -1.0
    ext[:, 1] = 0.9 + 0.2 * uniform(seed, envs, 1, 10)
    ext[:, 2:5] = 0.5 * normal(seed, envs[:, None], 1, np.arange(20, 23)[None, :])
    return q, root, ext
