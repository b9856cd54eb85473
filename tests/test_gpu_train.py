"""PPO training over the tensor env on the GPU (duck_gym_amd/on_policy.py,
the OnPolicyRunner that scripts/train_cuda.py:119-173 drives): a few
learning iterations of configs/standing.json with the reference's
zero-initialised last actor layer, rollout buffers on the device, finite
losses, a policy that moved, the observation normaliser fed every control
step, and a checkpoint that restores the same deterministic policy."""

import math
import sys
from pathlib import Path

import pytest
import torch

from duck_gym_amd.microduck import write_model
from duck_gym_amd.on_policy import PPO, STANDING, ActorCritic, OnPolicyRunner
from duck_gym_amd.tensor_env import TensorEnv

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT, ITER = 0.005, 10


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("train_model")
    write_model(d)
    return d


def test_ppo_iterations_on_the_standing_env(model_dir, tmp_path):
    E, iterations = 256, 3
    torch.manual_seed(0)
    env = TensorEnv(model_dir, E, ITER, DT, 4, seed=2, task="standing")
    runner = OnPolicyRunner(env, STANDING, log_dir=tmp_path, device=DEV)
    torch.nn.init.zeros_(runner.alg.policy.actor[-1].weight)
    torch.nn.init.zeros_(runner.alg.policy.actor[-1].bias)
    before = [p.detach().clone() for p in runner.alg.policy.actor.parameters()]
    assert runner.alg.storage.observations.device.type == "cuda"
    assert runner.alg.storage.observations.shape == (24, E, env.obs_dim)
    history = runner.learn(iterations, init_at_random_ep_len=True)
    assert len(history) == iterations
    for h in history:
        for key in ("loss/value_function", "loss/surrogate", "loss/entropy"):
            assert math.isfinite(h[key]), (key, h)
        assert 1e-5 <= h["learning_rate"] <= 1e-2
    change = sum(float((a - b.detach()).square().sum())
                 for a, b in zip(before, runner.alg.policy.actor.parameters())) ** 0.5
    assert change > 0
    assert int(runner.obs_normalizer.count) == E * 24 * iterations
    assert bool(torch.isfinite(runner.obs_normalizer._mean).all())
    b, _, d = env.native.state()
    assert bool(torch.isfinite(b).all())
    saved = tmp_path / f"model_{iterations - 1}.pt"
    assert saved.is_file()
    again = OnPolicyRunner(TensorEnv(model_dir, 8, ITER, DT, 4, seed=3), STANDING, device=DEV)
    again.load(saved)
    obs, _ = env.get_observations()
    with torch.no_grad():
        assert torch.equal(again.get_inference_policy()(obs), runner.get_inference_policy()(obs))


def test_device_learning_rate_follows_the_host_schedule():
    """On the GPU the KL-adaptive rate is updated in device memory; it takes
    the host schedule's decisions, to float32 rounding."""
    sys.path.insert(0, str(Path(__file__).parent))
    from test_on_policy import KL_SEQUENCE, expected_rates

    ppo = PPO(ActorCritic(3, 3, 2, [8], [8]), learning_rate=3e-4, schedule="adaptive",
              device=DEV)
    assert torch.is_tensor(ppo.optimizer.param_groups[0]["lr"])
    got = []
    for kl in KL_SEQUENCE:
        ppo._adapt_learning_rate(torch.tensor(kl, device=DEV))
        got.append(ppo.learning_rate)
    assert got == pytest.approx(expected_rates(3e-4, KL_SEQUENCE), rel=1e-5)
