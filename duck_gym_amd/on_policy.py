"""PPO training loop over the device-resident `TensorEnv`.

scripts/train_cuda.py:119-173 trains the tensor env with rsl-rl-lib 2.3.3's
`OnPolicyRunner` (requirements-training.txt:5), which this image does not
hold.  This module restates that runner's published algorithm (rsl-rl-lib
2.3.3: rsl_rl/runners/on_policy_runner.py, algorithms/ppo.py,
modules/actor_critic.py, modules/normalizer.py, storage/rollout_storage.py)
under the same names, so that train_cuda.py's uses of it read the same:
`OnPolicyRunner(env, cfg, log_dir, device)`, `runner.learn(n)`,
`runner.alg.policy.actor[-1]`, `runner.alg.policy.std`,
`runner.alg.optimizer`, `runner.save/load`, `runner.current_learning_iteration`.
The train config is the reference's JSON (configs/standing.json): policy
`ActorCritic`, algorithm `PPO`, `num_steps_per_env`, `save_interval`,
`empirical_normalization`.

Everything stays on the GPU: the rollout tensors are preallocated
[steps, envs, ...] buffers, the env step is the HIP control step, and the
update is plain torch.  Logging is a JSON-lines file (`log.jsonl` in
`log_dir`) instead of tensorboard.
"""

from __future__ import annotations

import json
import time
from pathlib import Path

import torch
from torch import nn
from torch.distributions import Normal

# configs/standing.json: the reference's standing-task training configuration
STANDING = {
    "num_steps_per_env": 24, "save_interval": 50, "empirical_normalization": True,
    "logger": "tensorboard",
    "policy": {"class_name": "ActorCritic", "init_noise_std": 0.1,
               "actor_hidden_dims": [64, 64], "critic_hidden_dims": [64, 64],
               "activation": "elu"},
    "algorithm": {"class_name": "PPO", "value_loss_coef": 1.0, "use_clipped_value_loss": True,
                  "clip_param": 0.2, "entropy_coef": 0.001, "num_learning_epochs": 4,
                  "num_mini_batches": 4, "learning_rate": 0.0003, "schedule": "adaptive",
                  "gamma": 0.99, "lam": 0.95, "desired_kl": 0.01, "max_grad_norm": 1.0},
}

_ACTIVATIONS = {"elu": nn.ELU, "relu": nn.ReLU, "selu": nn.SELU, "tanh": nn.Tanh,
                "sigmoid": nn.Sigmoid, "lrelu": nn.LeakyReLU}


def _mlp(inputs, hidden, outputs, activation):
    layers, width = [], inputs
    for h in hidden:
        layers += [nn.Linear(width, h), _ACTIVATIONS[activation]()]
        width = h
    layers.append(nn.Linear(width, outputs))
    return nn.Sequential(*layers)


class ActorCritic(nn.Module):
    """Gaussian policy with a state-independent standard deviation and a
    separate value network (rsl_rl/modules/actor_critic.py, 2.3.3)."""

    is_recurrent = False

    def __init__(self, num_actor_obs, num_critic_obs, num_actions, actor_hidden_dims=(256, 256, 256),
                 critic_hidden_dims=(256, 256, 256), activation="elu", init_noise_std=1.0,
                 noise_std_type="scalar", **unused):
        super().__init__()
        if unused:
            raise ValueError(f"Unknown ActorCritic arguments: {sorted(unused)}")
        if noise_std_type not in ("scalar", "log"):
            raise ValueError(f"Unknown noise_std_type {noise_std_type}")
        self.actor = _mlp(num_actor_obs, actor_hidden_dims, num_actions, activation)
        self.critic = _mlp(num_critic_obs, critic_hidden_dims, 1, activation)
        self.noise_std_type = noise_std_type
        if noise_std_type == "scalar":
            self.std = nn.Parameter(init_noise_std * torch.ones(num_actions))
        else:
            self.log_std = nn.Parameter(torch.log(init_noise_std * torch.ones(num_actions)))
        self.distribution = None

    def reset(self, dones=None):
        pass

    def update_distribution(self, observations):
        mean = self.actor(observations)
        std = self.std if self.noise_std_type == "scalar" else torch.exp(self.log_std)
        self.distribution = Normal(mean, std.expand_as(mean), validate_args=False)

    def act(self, observations):
        self.update_distribution(observations)
        return self.distribution.sample()

    def act_inference(self, observations):
        return self.actor(observations)

    def evaluate(self, critic_observations):
        return self.critic(critic_observations)

    def get_actions_log_prob(self, actions):
        return self.distribution.log_prob(actions).sum(dim=-1)

    @property
    def action_mean(self):
        return self.distribution.mean

    @property
    def action_std(self):
        return self.distribution.stddev

    @property
    def entropy(self):
        return self.distribution.entropy().sum(dim=-1)


class EmpiricalNormalization(nn.Module):
    """Running mean and variance of the observation stream, merged batch by
    batch with the exact pooled-moments update; `(x - mean) / (std + eps)`
    (rsl_rl/modules/normalizer.py, 2.3.3).  Stops updating once `until`
    samples have been seen."""

    def __init__(self, shape, eps=1e-2, until=None):
        super().__init__()
        self.eps, self.until = eps, until
        self.register_buffer("_mean", torch.zeros(shape).unsqueeze(0))
        self.register_buffer("_var", torch.ones(shape).unsqueeze(0))
        self.register_buffer("_std", torch.ones(shape).unsqueeze(0))
        self.register_buffer("count", torch.tensor(0, dtype=torch.long))

    def forward(self, x):
        if self.training:
            self.update(x)
        return (x - self._mean) / (self._std + self.eps)

    def update(self, x):
        if self.until is not None and self.count >= self.until:
            return
        n = x.shape[0]
        self.count += n
        rate = n / self.count.to(self._mean.dtype)
        var_x = torch.var(x, dim=0, unbiased=False, keepdim=True)
        mean_x = torch.mean(x, dim=0, keepdim=True)
        delta = mean_x - self._mean
        self._mean += rate * delta
        self._var += rate * (var_x - self._var + delta * (mean_x - self._mean))
        self._std = torch.sqrt(self._var)


class RolloutStorage:
    """[steps, envs, ...] buffers of one rollout and its returns
    (rsl_rl/storage/rollout_storage.py, 2.3.3)."""

    def __init__(self, num_envs, steps, obs_shape, critic_obs_shape, actions_shape, device):
        z = lambda *s, **k: torch.zeros(steps, num_envs, *s, device=device, **k)  # noqa: E731
        self.num_envs, self.steps, self.device = num_envs, steps, device
        self.observations = z(*obs_shape)
        self.critic_observations = z(*critic_obs_shape)
        self.actions = z(*actions_shape)
        self.rewards = z(1)
        self.dones = z(1, dtype=torch.uint8)
        self.values = z(1)
        self.actions_log_prob = z(1)
        self.mu = z(*actions_shape)
        self.sigma = z(*actions_shape)
        self.returns = z(1)
        self.advantages = z(1)
        self.step = 0

    def add(self, obs, critic_obs, actions, rewards, dones, values, log_prob, mu, sigma):
        if self.step >= self.steps:
            raise OverflowError("Rollout buffer overflow")
        s = self.step
        self.observations[s].copy_(obs)
        self.critic_observations[s].copy_(critic_obs)
        self.actions[s].copy_(actions)
        self.rewards[s].copy_(rewards.view(-1, 1))
        self.dones[s].copy_(dones.view(-1, 1))
        self.values[s].copy_(values)
        self.actions_log_prob[s].copy_(log_prob.view(-1, 1))
        self.mu[s].copy_(mu)
        self.sigma[s].copy_(sigma)
        self.step += 1

    def clear(self):
        self.step = 0

    def compute_returns(self, last_values, gamma, lam, normalize_advantage=True):
        """Generalised advantage estimation: delta_t = r_t + gamma (1 - d_t)
        V_{t+1} - V_t, A_t = delta_t + gamma lam (1 - d_t) A_{t+1}, R_t = A_t +
        V_t, with V_T the value of the observation after the last step."""
        advantage = 0
        for s in reversed(range(self.steps)):
            next_values = last_values if s == self.steps - 1 else self.values[s + 1]
            alive = 1.0 - self.dones[s].to(self.rewards.dtype)
            delta = self.rewards[s] + alive * gamma * next_values - self.values[s]
            advantage = delta + alive * gamma * lam * advantage
            self.returns[s] = advantage + self.values[s]
        self.advantages = self.returns - self.values
        if normalize_advantage:
            self.advantages = (self.advantages - self.advantages.mean()) / (
                self.advantages.std() + 1e-8)

    def mini_batches(self, num_mini_batches, num_epochs):
        """One permutation of the flattened rollout, cut into
        `num_mini_batches` slices, visited `num_epochs` times."""
        batch = self.num_envs * self.steps
        size = batch // num_mini_batches
        order = torch.randperm(num_mini_batches * size, device=self.device)
        flat = [t.flatten(0, 1) for t in (self.observations, self.critic_observations,
                                          self.actions, self.values, self.advantages,
                                          self.returns, self.actions_log_prob, self.mu,
                                          self.sigma)]
        for _ in range(num_epochs):
            for i in range(num_mini_batches):
                idx = order[i * size:(i + 1) * size]
                yield [t[idx] for t in flat]


class PPO:
    """Clipped-surrogate PPO with clipped value loss, entropy bonus, global
    gradient-norm clipping and the KL-adaptive learning rate
    (rsl_rl/algorithms/ppo.py, 2.3.3)."""

    def __init__(self, policy, num_learning_epochs=1, num_mini_batches=1, clip_param=0.2,
                 gamma=0.998, lam=0.95, value_loss_coef=1.0, entropy_coef=0.0,
                 learning_rate=1e-3, max_grad_norm=1.0, use_clipped_value_loss=True,
                 schedule="fixed", desired_kl=0.01, normalize_advantage_per_mini_batch=False,
                 device="cpu", **unused):
        if unused:
            raise ValueError(f"Unknown PPO arguments: {sorted(unused)}")
        if schedule not in ("fixed", "adaptive"):
            raise ValueError(f"Unknown schedule {schedule}")
        self.device = device
        self.policy = policy.to(device)
        # On the GPU the learning rate lives in device memory (Adam with
        # capturable=True takes a tensor rate): the KL-adaptive schedule then
        # makes no host round trip per mini-batch.
        self._device_lr = torch.device(device).type == "cuda"
        if self._device_lr:
            self.optimizer = torch.optim.Adam(
                self.policy.parameters(), capturable=True,
                lr=torch.tensor(float(learning_rate), dtype=torch.float32, device=device))
        else:
            self.optimizer = torch.optim.Adam(self.policy.parameters(), lr=learning_rate)
        self.learning_rate = learning_rate
        self.num_learning_epochs, self.num_mini_batches = num_learning_epochs, num_mini_batches
        self.clip_param, self.gamma, self.lam = clip_param, gamma, lam
        self.value_loss_coef, self.entropy_coef = value_loss_coef, entropy_coef
        self.max_grad_norm = max_grad_norm
        self.use_clipped_value_loss = use_clipped_value_loss
        self.schedule, self.desired_kl = schedule, desired_kl
        self.normalize_advantage_per_mini_batch = normalize_advantage_per_mini_batch
        self.storage = None
        self._pending = None

    def init_storage(self, num_envs, steps, obs_shape, critic_obs_shape, actions_shape):
        self.storage = RolloutStorage(num_envs, steps, obs_shape, critic_obs_shape,
                                      actions_shape, self.device)

    def act(self, obs, critic_obs):
        p = self.policy
        actions = p.act(obs).detach()
        values = p.evaluate(critic_obs).detach()
        self._pending = (obs, critic_obs, actions, values,
                         p.get_actions_log_prob(actions).detach(), p.action_mean.detach(),
                         p.action_std.detach())
        return actions

    def process_env_step(self, rewards, dones, infos):
        obs, critic_obs, actions, values, log_prob, mu, sigma = self._pending
        rewards = rewards.clone().to(self.device)
        if "time_outs" in infos:
            # bootstrap the value of an episode cut by the time limit
            rewards += self.gamma * (values * infos["time_outs"].unsqueeze(1).to(self.device)
                                     ).squeeze(1)
        self.storage.add(obs, critic_obs, actions, rewards, dones, values, log_prob, mu, sigma)
        self._pending = None
        self.policy.reset(dones)

    def compute_returns(self, last_critic_obs):
        last_values = self.policy.evaluate(last_critic_obs).detach()
        self.storage.compute_returns(last_values, self.gamma, self.lam,
                                     not self.normalize_advantage_per_mini_batch)

    def kl(self, old_mu, old_sigma, mu, sigma):
        """KL(old || new) of diagonal Gaussians, summed over actions."""
        return torch.sum(torch.log(sigma / old_sigma + 1e-5)
                         + (old_sigma.square() + (old_mu - mu).square()) / (2 * sigma.square())
                         - 0.5, dim=-1)

    @property
    def learning_rate(self):
        return float(self.optimizer.param_groups[0]["lr"])

    @learning_rate.setter
    def learning_rate(self, value):
        for group in self.optimizer.param_groups:
            if torch.is_tensor(group["lr"]):
                group["lr"].fill_(float(value))
            else:
                group["lr"] = float(value)

    def _adapt_learning_rate(self, kl_mean):
        """lr / 1.5 (not below 1e-5) when the mean KL exceeds twice the target,
        lr * 1.5 (not above 1e-2) when it is positive and below half of it."""
        high, low = self.desired_kl * 2.0, self.desired_kl / 2.0
        if self._device_lr:
            lr = self.optimizer.param_groups[0]["lr"]
            lr.copy_(torch.where(kl_mean > high, (lr / 1.5).clamp(min=1e-5),
                                 torch.where((kl_mean > 0.0) & (kl_mean < low),
                                             (lr * 1.5).clamp(max=1e-2), lr)))
            return
        lr = self.learning_rate
        if kl_mean > high:
            self.learning_rate = max(1e-5, lr / 1.5)
        elif 0.0 < kl_mean < low:
            self.learning_rate = min(1e-2, lr * 1.5)

    def _mini_batch(self, batch, sums):
        """One mini-batch: losses, KL-adaptive rate, backward, clipped Adam
        step; adds (value loss, surrogate, entropy) to `sums`."""
        p = self.policy
        (obs, critic_obs, actions, target_values, advantages, returns, old_log_prob, old_mu,
         old_sigma) = batch
        if self.normalize_advantage_per_mini_batch:
            with torch.no_grad():
                advantages = (advantages - advantages.mean()) / (advantages.std() + 1e-8)
        p.update_distribution(obs)
        log_prob = p.get_actions_log_prob(actions)
        values = p.evaluate(critic_obs)
        mu, sigma, entropy = p.action_mean, p.action_std, p.entropy
        if self.desired_kl is not None and self.schedule == "adaptive":
            with torch.no_grad():
                self._adapt_learning_rate(self.kl(old_mu, old_sigma, mu, sigma).mean())
        ratio = torch.exp(log_prob - old_log_prob.squeeze(-1))
        adv = advantages.squeeze(-1)
        surrogate = torch.max(-adv * ratio, -adv * ratio.clamp(1.0 - self.clip_param,
                                                               1.0 + self.clip_param)).mean()
        if self.use_clipped_value_loss:
            clipped = target_values + (values - target_values).clamp(-self.clip_param,
                                                                     self.clip_param)
            value_loss = torch.max((values - returns).square(),
                                   (clipped - returns).square()).mean()
        else:
            value_loss = (returns - values).square().mean()
        loss = surrogate + self.value_loss_coef * value_loss - self.entropy_coef * entropy.mean()
        self.optimizer.zero_grad()
        loss.backward()
        nn.utils.clip_grad_norm_(p.parameters(), self.max_grad_norm)
        self.optimizer.step()
        with torch.no_grad():
            sums += torch.stack((value_loss.detach(), surrogate.detach(),
                                 entropy.mean().detach()))

    def update(self):
        # loss sums stay on the device until the update ends
        sums = torch.zeros(3, device=self.device)
        n = 0
        for batch in self.storage.mini_batches(self.num_mini_batches, self.num_learning_epochs):
            self._mini_batch(batch, sums)
            n += 1
        self.storage.clear()
        value, surrogate, entropy = (sums / n).tolist()
        return {"value_function": value, "surrogate": surrogate, "entropy": entropy}


class OnPolicyRunner:
    """Rollout + PPO update per learning iteration over a VecEnv
    (rsl_rl/runners/on_policy_runner.py, 2.3.3).  The env provides
    `num_envs`, `num_actions`, `max_episode_length`, `episode_length_buf`,
    `get_observations() -> (obs, {"observations": {...}})` and
    `step(actions) -> (obs, rewards, dones, infos)` with `infos["time_outs"]`."""

    def __init__(self, env, train_cfg, log_dir=None, device="cuda:0"):
        cfg = json.loads(json.dumps(train_cfg))
        self.cfg, self.env, self.device = cfg, env, device
        policy_cfg, alg_cfg = dict(cfg["policy"]), dict(cfg["algorithm"])
        if policy_cfg.pop("class_name", "ActorCritic") != "ActorCritic":
            raise ValueError("Only the ActorCritic policy is provided")
        if alg_cfg.pop("class_name", "PPO") != "PPO":
            raise ValueError("Only the PPO algorithm is provided")
        obs, extras = env.get_observations()
        num_obs = obs.shape[1]
        critic = extras["observations"].get("critic")
        num_critic_obs = critic.shape[1] if critic is not None else num_obs
        policy = ActorCritic(num_obs, num_critic_obs, env.num_actions, **policy_cfg)
        self.alg = PPO(policy, device=device, **alg_cfg)
        self.num_steps_per_env = int(cfg["num_steps_per_env"])
        self.save_interval = int(cfg.get("save_interval", 50))
        if cfg.get("empirical_normalization", False):
            self.obs_normalizer = EmpiricalNormalization([num_obs], until=1.0e8).to(device)
            self.critic_obs_normalizer = EmpiricalNormalization([num_critic_obs],
                                                                until=1.0e8).to(device)
        else:
            self.obs_normalizer = nn.Identity().to(device)
            self.critic_obs_normalizer = nn.Identity().to(device)
        self.alg.init_storage(env.num_envs, self.num_steps_per_env, [num_obs],
                              [num_critic_obs], [env.num_actions])
        self.log_dir = Path(log_dir) if log_dir is not None else None
        self.current_learning_iteration = 0
        self.history = []

    def train_mode(self):
        self.alg.policy.train()
        self.obs_normalizer.train()
        self.critic_obs_normalizer.train()

    def eval_mode(self):
        self.alg.policy.eval()
        self.obs_normalizer.eval()
        self.critic_obs_normalizer.eval()

    def learn(self, num_learning_iterations, init_at_random_ep_len=False):
        env, alg = self.env, self.alg
        if init_at_random_ep_len:
            env.episode_length_buf = torch.randint_like(env.episode_length_buf,
                                                        high=int(env.max_episode_length))
        obs, extras = env.get_observations()
        critic_obs = extras["observations"].get("critic", obs)
        obs, critic_obs = obs.to(self.device), critic_obs.to(self.device)
        self.train_mode()
        episode_return = torch.zeros(env.num_envs, device=self.device)
        episode_length = torch.zeros(env.num_envs, device=self.device)
        start = self.current_learning_iteration
        for it in range(start, start + num_learning_iterations):
            t0 = time.perf_counter()
            # episode statistics stay on the device until the iteration ends
            ended = torch.zeros(3, device=self.device)
            with torch.inference_mode():
                for _ in range(self.num_steps_per_env):
                    actions = alg.act(obs, critic_obs)
                    obs, rewards, dones, infos = env.step(actions.to(env.device))
                    obs, rewards, dones = (obs.to(self.device), rewards.to(self.device),
                                           dones.to(self.device))
                    obs = self.obs_normalizer(obs)
                    critic = infos["observations"].get("critic")
                    critic_obs = self.critic_obs_normalizer(critic.to(self.device)) \
                        if critic is not None else obs
                    alg.process_env_step(rewards, dones, infos)
                    episode_return += rewards
                    episode_length += 1
                    d = dones.bool()
                    ended += torch.stack((torch.where(d, episode_return, 0).sum(),
                                          torch.where(d, episode_length, 0).sum(), d.sum()))
                    episode_return.masked_fill_(d, 0)
                    episode_length.masked_fill_(d, 0)
                if torch.device(self.device).type == "cuda":
                    torch.cuda.synchronize(self.device)  # time the phases, once per iteration
                collected = time.perf_counter() - t0
                alg.compute_returns(critic_obs)
            losses = alg.update()
            finished_return, finished_length, finished = ended.tolist()
            learned = time.perf_counter() - t0 - collected
            self.current_learning_iteration = it
            record = dict(iteration=it, collection_s=collected, learning_s=learned,
                          learning_rate=alg.learning_rate,
                          mean_noise_std=float(alg.policy.std.detach().mean())
                          if alg.policy.noise_std_type == "scalar"
                          else float(torch.exp(alg.policy.log_std.detach()).mean()),
                          mean_episode_return=finished_return / finished if finished else None,
                          mean_episode_length=finished_length / finished if finished else None,
                          steps_per_s=env.num_envs * self.num_steps_per_env / (collected + learned),
                          **{f"loss/{k}": v for k, v in losses.items()})
            self.history.append(record)
            if self.log_dir is not None:
                self.log_dir.mkdir(parents=True, exist_ok=True)
                with open(self.log_dir / "log.jsonl", "a") as f:
                    f.write(json.dumps(record) + "\n")
                if it % self.save_interval == 0:
                    self.save(self.log_dir / f"model_{it}.pt")
        if self.log_dir is not None:
            self.save(self.log_dir / f"model_{self.current_learning_iteration}.pt")
        return self.history

    def save(self, path):
        torch.save({"model_state_dict": self.alg.policy.state_dict(),
                    "optimizer_state_dict": self.alg.optimizer.state_dict(),
                    "obs_norm_state_dict": self.obs_normalizer.state_dict(),
                    "critic_obs_norm_state_dict": self.critic_obs_normalizer.state_dict(),
                    "iter": self.current_learning_iteration}, path)

    def load(self, path, load_optimizer=True):
        state = torch.load(path, map_location=self.device, weights_only=True)
        self.alg.policy.load_state_dict(state["model_state_dict"])
        self.obs_normalizer.load_state_dict(state["obs_norm_state_dict"])
        self.critic_obs_normalizer.load_state_dict(state["critic_obs_norm_state_dict"])
        if load_optimizer:
            self.alg.optimizer.load_state_dict(state["optimizer_state_dict"])
        self.current_learning_iteration = state["iter"]
        return state

    def get_inference_policy(self, device=None):
        """Deterministic policy: the actor's mean on normalised observations."""
        self.eval_mode()
        if device is not None:
            self.alg.policy.to(device)
            self.obs_normalizer.to(device)
        policy, norm = self.alg.policy, self.obs_normalizer
        return lambda x: policy.act_inference(norm(x))
