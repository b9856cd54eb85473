"""The generic state (models beyond the MicroDuck layout: up to 32 bodies and
hinges, 4 ground contacts per shape and one contact per body pair) against
the oracle, on a 24-segment caterpillar (25 bodies, 23 yaw hinges, 24 box
shapes lying on the ground, 22 body-contact pairs between segments i and
i + 2).  Every box rests on four corners, so an environment holds 96 ground
contacts -- past the 64 of one mask word -- and curling the hinges brings up
to 8 body contacts and 7 colours on top.  The reference's own generic state
(BasicState<32, 32, 160>, kernel.cuh:365) reproduces the oracle on this
model bit for bit (tests/test_oracle.py)."""

import numpy as np
import pytest
import torch

from duck_gym_amd import CudaBatch
from model_text import caterpillar
from parity_support import compare_env, oracle_envs, oracle_state, seed_batch

pytestmark = pytest.mark.gpu
DT, ITER, KP, DEV = 0.005, 10, 8.0, "cuda:0"
E = 4


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("generic") / "caterpillar.duck"
    path.write_text(caterpillar())
    return path


def _targets():
    rng = np.random.default_rng(20260927)
    base = np.array([1.05, 0.9, 1.15, -1.05])[:, None]
    return base + rng.uniform(-0.1, 0.1, (E, 23))


@pytest.mark.parametrize("split", [False, True], ids=["one-lane", "split"])
def test_fp64_generic_trajectory_matches_oracle(model, split):
    """float64, 40 steps from rest: contact lists (96 ground contacts plus
    body contacts), stick flags, colours and counts exact; poses,
    velocities, multipliers, penalties and contact points within 1e-9 --
    one lane per block solve and four (the float layout)."""
    targets = _targets()
    batch = CudaBatch(model, E, DT, ITER, 0, True, split_solve=split)
    assert batch.num_bodies == 25 and batch.contact_capacity == 96 + 22
    codec = batch.codec()
    assert codec.L["CG"] == 128 and codec.L["CS"] == 32
    oracles = oracle_envs(model, E, DT, ITER, True)
    for o in oracles:
        o.reset(np.zeros(23))
    seed_batch(batch, oracles)
    tg = torch.tensor(targets, device=DEV)
    fg = torch.zeros(E, 3, dtype=torch.float64, device=DEV)
    most_ground = most_body = most_colours = 0
    worst = 0.0
    for step in range(40):
        batch.step(tg, fg, 1, KP, 0.0)
        for o, t in zip(oracles, targets):
            o.step(t, None, 1, KP, 0.0)
        raw = batch.export_state().cpu().numpy()
        for e, o in enumerate(oracles):
            gpu, ref = codec.decode(raw[e]), oracle_state(o)
            d = compare_env(gpu, ref, 1e-9, f"step {step + 1} env {e}")
            worst = max(worst, d["x"], d["rot"])
            most_ground = max(most_ground, len(ref["gc"]))
            most_body = max(most_body, len(ref["sc"]))
            most_colours = max(most_colours, ref["colorCount"])
    assert most_ground > 64 and most_body > 0 and most_colours > 2, (most_ground, most_body,
                                                                     most_colours)
    print(f"generic fp64 split={split}: {most_ground} ground, {most_body} body contacts, "
          f"{most_colours} colours, worst pose difference {worst:.2e}")


def test_fp32_generic_seeded_steps(model):
    """float32: the batch seeded with oracle states along the trajectory and
    stepped once agrees within 1e-5, with identical contact lists (stick
    flags included) and colours."""
    targets = _targets()
    oracles = oracle_envs(model, E, DT, ITER, False)
    for o in oracles:
        o.reset(np.zeros(23))
    batch = CudaBatch(model, E, DT, ITER, 0, False)
    codec = batch.codec()
    tg = torch.tensor(targets, dtype=torch.float32, device=DEV)
    fg = torch.zeros(E, 3, device=DEV)
    checked = body = 0
    for round_ in range(8):
        for _ in range(4):
            for o, t in zip(oracles, targets):
                o.step(t, None, 1, KP, 0.0)
        seed_batch(batch, oracles)
        batch.step(tg, fg, 1, KP, 0.0)
        for o, t in zip(oracles, targets):
            o.step(t, None, 1, KP, 0.0)
        raw = batch.export_state().cpu().numpy()
        for e, o in enumerate(oracles):
            ref = oracle_state(o)
            compare_env(codec.decode(raw[e]), ref, 1e-5, f"round {round_} env {e}", strict_stick=True)
            body += len(ref["sc"])
            checked += 1
    assert checked == 8 * E and body > 0
