"""Bodies with more ground contacts than the float assembly's straight-line
block takes (two per lane): a five-segment caterpillar whose segments each
carry three stacked box shapes, so a resting segment holds twelve ground
contacts.  The model fits the MicroDuck-sized state (6 bodies, 15 shapes,
60 ground contacts: one mask word), whose float assembly stamps a lane's
further contacts in ballot-counted rounds; a body on two lanes takes four
such rounds, the body lent the colour's free slot (four lanes) one.  The
float32 batch is seeded with the oracle's states along a trajectory and
stepped once at each checkpoint, to the float32 gates of the other parity
tests, with the contact lists (stick flags included) and colours exact."""

import numpy as np
import pytest
import torch

from duck_gym_amd import CudaBatch
from model_text import caterpillar
from parity_support import compare_env, oracle_envs, oracle_state, seed_batch

pytestmark = pytest.mark.gpu
DT, ITER, KP, DEV = 0.005, 10, 8.0, "cuda:0"
E, SEGMENTS, STACK = 4, 5, 3


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("stacked") / "stacked.duck"
    path.write_text(caterpillar(segments=SEGMENTS, pairs=False, shapes_per_segment=STACK))
    return path


def _targets():
    rng = np.random.default_rng(20261202)
    return rng.uniform(-0.8, 0.8, (E, SEGMENTS - 1))


def test_fp32_stacked_contacts_seeded_steps(model):
    targets = _targets()
    oracles = oracle_envs(model, E, DT, ITER, False)
    for o in oracles:
        o.reset(np.zeros(SEGMENTS - 1))
    batch = CudaBatch(model, E, DT, ITER, 0, False)
    codec = batch.codec()
    # the MicroDuck-sized instance (one 64-bit mask word per body)
    assert codec.L["CG"] == 64 and codec.L["B"] == 16
    tg = torch.tensor(targets, dtype=torch.float32, device=DEV)
    fg = torch.zeros(E, 3, device=DEV)
    checked, most_per_body = 0, 0
    for round_ in range(8):
        for _ in range(3):
            for o, t in zip(oracles, targets):
                o.step(t, None, 1, KP, 0.0)
        seed_batch(batch, oracles)
        batch.step(tg, fg, 1, KP, 0.0)
        for o, t in zip(oracles, targets):
            o.step(t, None, 1, KP, 0.0)
        raw = batch.export_state().cpu().numpy()
        for e, o in enumerate(oracles):
            ref = oracle_state(o)
            compare_env(codec.decode(raw[e]), ref, 1e-5, f"round {round_} env {e}",
                        strict_stick=True)
            bodies = [c["body"] for c in ref["gc"]]
            most_per_body = max([most_per_body] + [bodies.count(b) for b in set(bodies)])
            checked += 1
    assert checked == 8 * E
    # more than the straight-line block's two contacts on each of four lanes
    assert most_per_body > 8, most_per_body
    print(f"stacked shapes: up to {most_per_body} ground contacts on one body")
