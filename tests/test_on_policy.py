"""PPO runner (duck_gym_amd/on_policy.py) on the CPU: returns, normaliser, KL,
time-out bootstrap and mini-batching against closed forms and
torch.distributions, and a small learning problem that the runner must
solve.  The algorithm is rsl-rl-lib 2.3.3's (requirements-training.txt:5),
which this image does not hold; these checks pin the restatement."""

import numpy as np
import pytest
import torch

from duck_gym_amd.on_policy import (PPO, STANDING, ActorCritic, EmpiricalNormalization,
                                    OnPolicyRunner, RolloutStorage)



def _storage(T, E, seed, done_rate=0.25):
    g = torch.Generator().manual_seed(seed)
    s = RolloutStorage(E, T, [3], [3], [2], "cpu")
    s.rewards = torch.randn(T, E, 1, generator=g, dtype=torch.float64)
    s.values = torch.randn(T, E, 1, generator=g, dtype=torch.float64)
    s.dones = (torch.rand(T, E, 1, generator=g) < done_rate).to(torch.uint8)
    s.returns = torch.zeros(T, E, 1, dtype=torch.float64)
    last = torch.randn(E, 1, generator=g, dtype=torch.float64)
    return s, last


@pytest.mark.parametrize("lam", [0.0, 0.7, 1.0])
def test_gae_is_the_explicit_sum_of_discounted_residuals(lam):
    """A_t = sum_k (gamma lam)^k delta_{t+k}, truncated at the first done,
    with delta_t = r_t + gamma (1 - d_t) V_{t+1} - V_t."""
    T, E, gamma = 9, 6, 0.9
    s, last = _storage(T, E, 3)
    s.compute_returns(last, gamma, lam, normalize_advantage=False)
    r, v, d = s.rewards[..., 0].numpy(), s.values[..., 0].numpy(), s.dones[..., 0].numpy()
    nv = np.concatenate([v[1:], last.numpy().T], 0)
    delta = r + gamma * (1 - d) * nv - v
    for e in range(E):
        for t in range(T):
            a, w = 0.0, 1.0
            for k in range(t, T):
                a += w * delta[k, e]
                if d[k, e]:
                    break
                w *= gamma * lam
            assert s.advantages[t, e, 0].item() == pytest.approx(a, abs=1e-12)
            assert s.returns[t, e, 0].item() == pytest.approx(a + v[t, e], abs=1e-12)


def test_gae_with_lambda_one_is_the_bootstrapped_discounted_return():
    """lam = 1: R_t is the discounted reward sum to the episode's end, plus
    gamma^n V_T when the rollout ends first (values cancel)."""
    T, E, gamma = 8, 5, 0.95
    s, last = _storage(T, E, 5)
    s.compute_returns(last, gamma, 1.0, normalize_advantage=False)
    r, d = s.rewards[..., 0].numpy(), s.dones[..., 0].numpy()
    for e in range(E):
        for t in range(T):
            ret, w, k = 0.0, 1.0, t
            while True:
                ret += w * r[k, e]
                if d[k, e]:
                    break
                w *= gamma
                if k == T - 1:
                    ret += w * last[e, 0].item()
                    break
                k += 1
            assert s.returns[t, e, 0].item() == pytest.approx(ret, abs=1e-12)


def test_advantages_are_normalised_over_the_rollout():
    s, last = _storage(6, 7, 9)
    s.compute_returns(last, 0.99, 0.95)
    a = s.advantages.numpy().ravel()
    assert abs(a.mean()) < 1e-12 and a.std(ddof=1) == pytest.approx(1.0, abs=1e-8)


def test_normaliser_holds_the_moments_of_everything_seen():
    g = torch.Generator().manual_seed(1)
    norm = EmpiricalNormalization([4]).double()
    seen = []
    for n in (5, 1, 17, 3, 40):
        x = torch.randn(n, 4, generator=g, dtype=torch.float64) * torch.tensor([1, 3, 0.1, 7.0]) + 2
        seen.append(x.numpy())
        y = norm(x)
        all_ = np.concatenate(seen)
        np.testing.assert_allclose(norm._mean.numpy()[0], all_.mean(0), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(norm._var.numpy()[0], all_.var(0), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(y.numpy(), (x.numpy() - all_.mean(0)) / (all_.std(0) + 1e-2),
                                   rtol=1e-9, atol=1e-12)
    assert int(norm.count) == 66
    frozen = EmpiricalNormalization([4], until=10)
    frozen(torch.randn(12, 4, generator=g))
    before = frozen._mean.clone()
    frozen(torch.randn(12, 4, generator=g) + 5)
    assert torch.equal(frozen._mean, before) and int(frozen.count) == 12
    frozen.eval()
    frozen(torch.randn(3, 4, generator=g))
    assert int(frozen.count) == 12


def test_kl_matches_torch_distributions():
    g = torch.Generator().manual_seed(4)
    mu0, mu1 = torch.randn(50, 3, generator=g), torch.randn(50, 3, generator=g)
    s0, s1 = torch.rand(50, 3, generator=g) + 0.1, torch.rand(50, 3, generator=g) + 0.1
    ppo = PPO(ActorCritic(3, 3, 3, [8], [8]))
    ref = torch.distributions.kl_divergence(torch.distributions.Normal(mu0, s0),
                                            torch.distributions.Normal(mu1, s1)).sum(-1)
    # the 1e-5 inside the logarithm shifts each term by at most 1e-5 s0/s1
    np.testing.assert_allclose(ppo.kl(mu0, s0, mu1, s1).numpy(), ref.numpy(), atol=3e-4)
    assert torch.all(ppo.kl(mu0, s0, mu0, s0).abs() < 1e-4)


KL_SEQUENCE = [0.05, 0.001, 0.0, 0.01, 0.02, 0.0051, 0.0049] + [1.0] * 12 + [1e-4] * 20


def expected_rates(lr, kls, target=0.01):
    out = []
    for kl in kls:
        if kl > 2 * target:
            lr = lr / 1.5 if lr / 1.5 > 1e-5 else 1e-5
        elif 0 < kl < target / 2:
            lr = lr * 1.5 if lr * 1.5 < 1e-2 else 1e-2
        out.append(lr)
    return out


def test_adaptive_learning_rate_schedule():
    """Divide by 1.5 above twice the target KL, multiply by 1.5 for a positive
    KL below half of it, hold otherwise, within [1e-5, 1e-2]."""
    ppo = PPO(ActorCritic(3, 3, 2, [8], [8]), learning_rate=3e-4, schedule="adaptive")
    got = []
    for kl in KL_SEQUENCE:
        ppo._adapt_learning_rate(torch.tensor(kl))
        got.append(ppo.learning_rate)
    want = expected_rates(3e-4, KL_SEQUENCE)
    assert got[:7] == pytest.approx([2e-4, 3e-4, 3e-4, 3e-4, 3e-4, 3e-4, 4.5e-4], rel=1e-12)
    assert got == pytest.approx(want, rel=1e-12)
    assert min(got) == 1e-5 and max(got) == 1e-2


def test_timeouts_bootstrap_the_value_into_the_reward():
    torch.manual_seed(0)
    ppo = PPO(ActorCritic(3, 3, 2, [8], [8]), gamma=0.9)
    ppo.init_storage(4, 2, [3], [3], [2])
    obs = torch.randn(4, 3)
    ppo.act(obs, obs)
    values = ppo.policy.evaluate(obs).detach()[:, 0]
    rewards = torch.tensor([1.0, 2.0, 3.0, 4.0])
    timeouts = torch.tensor([False, True, False, True])
    ppo.process_env_step(rewards, timeouts, {"time_outs": timeouts})
    want = rewards + 0.9 * values * timeouts
    assert torch.allclose(ppo.storage.rewards[0, :, 0], want)
    assert ppo.storage.dones[0, :, 0].tolist() == [0, 1, 0, 1]
    ppo.act(obs, obs)
    ppo.process_env_step(rewards, timeouts, {})
    assert torch.equal(ppo.storage.rewards[1, :, 0], rewards)
    with pytest.raises(OverflowError):
        ppo.act(obs, obs)
        ppo.process_env_step(rewards, timeouts, {})


def test_mini_batches_visit_every_sample_once_per_epoch():
    T, E = 4, 6
    s = RolloutStorage(E, T, [1], [1], [1], "cpu")
    s.observations = torch.arange(T * E, dtype=torch.float32).view(T, E, 1)
    batches = list(s.mini_batches(3, 2))
    assert len(batches) == 6
    for epoch in range(2):
        ids = torch.cat([b[0][:, 0] for b in batches[3 * epoch:3 * epoch + 3]])
        assert sorted(ids.tolist()) == list(range(T * E))
    assert all(torch.equal(batches[i][0], batches[i + 3][0]) for i in range(3))


def test_surrogate_gradient_stops_outside_the_clip_range():
    """The clipped surrogate has no policy gradient for a sample whose ratio
    is already past 1 + clip in the direction its advantage favours."""
    torch.manual_seed(2)
    policy = ActorCritic(2, 2, 1, [], [], init_noise_std=1.0)
    ppo = PPO(policy, clip_param=0.2, value_loss_coef=0.0, entropy_coef=0.0, max_grad_norm=1e9,
              learning_rate=0.0)
    ppo.init_storage(1, 1, [2], [2], [1])
    obs = torch.tensor([[1.0, 0.5]])
    mean = policy.actor(obs).detach()
    action = mean + 1.0
    s = ppo.storage
    s.observations[0] = obs
    s.critic_observations[0] = obs
    s.actions[0] = action
    s.advantages = torch.ones(1, 1, 1)
    s.returns = torch.zeros(1, 1, 1)
    s.values = torch.zeros(1, 1, 1)
    s.mu[0], s.sigma[0] = mean, torch.ones(1, 1)
    for old_log_prob, moving in ((-10.0, False), (float(
            torch.distributions.Normal(mean, 1.0).log_prob(action).sum()), True)):
        s.actions_log_prob = torch.full((1, 1, 1), old_log_prob)
        ppo.update()
        grad = policy.actor[-1].bias.grad.abs().sum().item()
        assert (grad > 0) == moving


class _LinearTarget:
    """VecEnv of the TensorEnv contract on the CPU: observation x ~ N(0, 1)^4,
    reward -mean((a - W x)^2), episodes of 8 steps ended by time-outs."""

    def __init__(self, n=64, seed=0):
        self.num_envs, self.num_actions, self.max_episode_length, self.device = n, 2, 8, "cpu"
        self.g = torch.Generator().manual_seed(seed)
        self.W = torch.randn(2, 4, generator=self.g)
        self.obs = torch.randn(n, 4, generator=self.g)
        self.episode_length_buf = torch.zeros(n, dtype=torch.long)

    def get_observations(self):
        return self.obs.clone(), {"observations": {}}

    def step(self, actions):
        reward = -(actions - self.obs @ self.W.T).square().mean(-1)
        self.episode_length_buf += 1
        timeout = self.episode_length_buf >= self.max_episode_length
        self.episode_length_buf[timeout] = 0
        self.obs = torch.randn(self.num_envs, 4, generator=self.g)
        return self.obs.clone(), reward, timeout, {"observations": {}, "time_outs": timeout}

    def greedy_error(self, policy):
        x = torch.randn(2048, 4, generator=torch.Generator().manual_seed(99))
        with torch.no_grad():
            return float((policy(x) - x @ self.W.T).square().mean())


def test_runner_learns_a_linear_target(tmp_path):
    torch.manual_seed(0)
    env = _LinearTarget()
    cfg = {**STANDING, "num_steps_per_env": 16, "save_interval": 10,
           "policy": {**STANDING["policy"], "init_noise_std": 0.5},
           "algorithm": {**STANDING["algorithm"], "learning_rate": 3e-3}}
    runner = OnPolicyRunner(env, cfg, log_dir=tmp_path, device="cpu")
    before = env.greedy_error(runner.get_inference_policy())
    history = runner.learn(60)
    after = env.greedy_error(runner.get_inference_policy())
    assert len(history) == 60 and runner.current_learning_iteration == 59
    assert all(np.isfinite(h["loss/value_function"]) and np.isfinite(h["loss/surrogate"])
               for h in history)
    assert after < 0.1 * before, (before, after)
    assert history[-1]["mean_episode_length"] == 8
    assert (tmp_path / "log.jsonl").read_text().count("\n") == 60
    saved = tmp_path / "model_59.pt"
    assert saved.is_file() and (tmp_path / "model_50.pt").is_file()
    again = OnPolicyRunner(_LinearTarget(), cfg, device="cpu")
    again.load(saved)
    assert again.current_learning_iteration == 59
    x = torch.randn(5, 4)
    assert torch.equal(again.get_inference_policy()(x), runner.get_inference_policy()(x))


def test_runner_rejects_unknown_configuration():
    env = _LinearTarget(8)
    with pytest.raises(ValueError):
        OnPolicyRunner(env, {**STANDING, "policy": {**STANDING["policy"],
                                                     "class_name": "ActorCriticRecurrent"}},
                       device="cpu")
    with pytest.raises(ValueError):
        OnPolicyRunner(env, {**STANDING, "algorithm": {**STANDING["algorithm"],
                                                        "schedule": "cosine"}}, device="cpu")
    with pytest.raises(ValueError):
        OnPolicyRunner(env, {**STANDING, "algorithm": {**STANDING["algorithm"], "lr": 1.0}},
                       device="cpu")


class _WithCritic(_LinearTarget):
    """The same problem with a 6-wide privileged critic observation."""

    def _critic(self):
        return torch.cat((self.obs, self.obs[:, :2] * 2), -1)

    def get_observations(self):
        return self.obs.clone(), {"observations": {"critic": self._critic()}}

    def step(self, actions):
        obs, reward, timeout, info = super().step(actions)
        info["observations"]["critic"] = self._critic()
        return obs, reward, timeout, info


def test_runner_critic_observations_and_random_episode_start():
    torch.manual_seed(1)
    env = _WithCritic(32)
    runner = OnPolicyRunner(env, {**STANDING, "num_steps_per_env": 8}, device="cpu")
    assert runner.alg.policy.critic[0].in_features == 6
    assert runner.alg.policy.actor[0].in_features == 4
    assert runner.alg.storage.critic_observations.shape == (8, 32, 6)
    runner.learn(2, init_at_random_ep_len=True)
    # both normalisers saw every control step: the critic's its own 6 columns
    assert int(runner.obs_normalizer.count) == 32 * 8 * 2
    assert int(runner.critic_obs_normalizer.count) == 32 * 8 * 2
    assert runner.critic_obs_normalizer._mean.shape == (1, 6)
    assert runner.current_learning_iteration == 1
    starts = OnPolicyRunner(_WithCritic(256), {**STANDING, "num_steps_per_env": 1},
                            device="cpu")
    starts.env.episode_length_buf.zero_()
    starts.learn(1, init_at_random_ep_len=True)
    lengths = starts.env.episode_length_buf
    assert int(lengths.min()) >= 0 and int(lengths.max()) < 8
    assert len(set(lengths.tolist())) > 4
