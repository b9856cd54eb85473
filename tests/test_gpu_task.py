"""The tensor-env control step on the GPU (duck_gym_amd.tensor_env.TensorEnv,
kernels taskTargetsKernel / taskKernel) against the CPU oracle of
oracle/task_oracle.py on the same post-step states: servo targets
bit-exact in float32, observations/rewards within float32 rounding, failure /
timeout / done flags exact, counters and returns, the reset bookkeeping, and
the reference's random reset draws (tensor_env.py:178-219, 279-391)."""

import numpy as np
import pytest
import torch

from duck_gym_amd.microduck import write_model
from duck_gym_amd.tensor_env import TensorEnv
from oracle import task_oracle as T

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT, ITER = 0.005, 10


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("task_model")
    write_model(d)
    return d


def _np(t):
    return t.detach().cpu().double().numpy()


def _check_step(env, kind, actions, tol, **extra):
    """One env.step() against the oracle on the state it produced.  `tol`
    bounds quantities kept in the batch dtype; observations and rewards are
    float32 outputs, so they get at least float32 rounding room."""
    out_tol = max(tol, 1e-6)
    last = _np(env.actions)
    episode = env.episode_length_buf.cpu().numpy()
    filtered = _np(env.filtered_velocity) if env.velocity_filter_seconds > 0 else None
    commands = _np(env.commands)
    returns = env.returns.clone()
    obs, reward, done, info = env.step(actions)
    b, j, d = [_np(x) for x in env.native.state()]
    meta = env.meta
    # Servo targets: the float32 arithmetic of tensor_env.py:331-335 exactly.
    f = np.float32 if env.dtype == torch.float32 else np.float64
    a = np.clip(actions.cpu().numpy().astype(f), f(-1), f(1))
    target = np.clip(np.asarray(meta["home"], f) + f(env.action_scale) * a,
                     np.asarray(meta["lower"], f), np.asarray(meta["upper"], f))
    assert np.array_equal(info["applied_targets"].cpu().numpy(), target)
    assert np.array_equal(env.actions.cpu().numpy(), a)
    failed, rew, ep, timeout, dn, filt = T.step_outputs(
        kind, b, j, d, a.astype(float), last, meta, control_dt=env.control_dt,
        episode=episode, max_episode_length=env.max_episode_length, commands=commands,
        filtered=filtered, alpha=env.velocity_alpha, tracking_weight=env.tracking_weight,
        heading_weight=env.heading_weight, tracking_sigma=env.tracking_sigma, **extra)
    assert np.array_equal(info["failed"].cpu().numpy(), failed)
    assert np.array_equal(info["time_outs"].cpu().numpy(), timeout)
    assert np.array_equal(done.cpu().numpy(), dn)
    np.testing.assert_allclose(reward.cpu().numpy(), rew, rtol=out_tol,
                               atol=out_tol * env.control_dt)
    np.testing.assert_allclose(env.returns.cpu().numpy(),
                               returns.cpu().numpy() + rew.astype(np.float32), rtol=1e-6,
                               atol=1e-7)
    np.testing.assert_array_equal(info["diagnostics"].cpu().numpy(), d)
    if filt is not None:
        np.testing.assert_allclose(_np(env.filtered_velocity), filt, rtol=tol, atol=tol)
    expect = T.observe(kind, b, j, a.astype(float), meta, commands=commands, episode=ep,
                       control_dt=env.control_dt, gait_period=0.8, filtered=filt)
    np.testing.assert_allclose(info["terminal_observation"].cpu().numpy(), expect,
                               rtol=out_tol, atol=out_tol)
    return obs, done, info


def test_standing_steps_match_oracle(model_dir):
    env = TensorEnv(model_dir, 64, ITER, DT, 1, seed=3, auto_reset=False)
    assert env.obs_dim == 52
    gen = torch.Generator().manual_seed(0)
    for _ in range(25):
        actions = (torch.rand(64, 14, generator=gen) * 3 - 1.5).to(DEV)
        _check_step(env, T.STANDING, actions, 2e-5)


def test_locomotion_filter_fp64_matches_oracle(model_dir):
    env = TensorEnv(model_dir, 32, ITER, DT, 2, seed=5, task="locomotion", auto_reset=False,
                    fp64=True, velocity_filter_seconds=0.05)
    assert env.obs_dim == 60
    gen = torch.Generator().manual_seed(1)
    for _ in range(15):
        actions = (torch.rand(32, 14, generator=gen, dtype=torch.float64) - 0.5).to(DEV)
        _check_step(env, T.LOCOMOTION, actions, 1e-9)


def test_rollout_task_resets_on_timeout(model_dir):
    # 4 control steps per episode: every env times out at step 4 and is reset.
    env = TensorEnv(model_dir, 48, ITER, DT, 1, seed=7, task="rollout", episode_seconds=0.02)
    assert env.obs_dim == 48 and env.max_episode_length == 4
    gen = torch.Generator().manual_seed(2)
    for step in range(1, 7):
        actions = (torch.rand(48, 14, generator=gen) - 0.5).to(DEV)
        before = env.returns.clone()
        obs, done, info = _check_step_rollout(env, actions)
        if step % 4 == 0:
            assert bool(done.all())
            assert int(env.episode_length_buf.abs().sum()) == 0
            assert float(env.returns.abs().sum()) == 0.0
            assert float(env.actions.abs().sum()) == 0.0
            b, j, d = [_np(x) for x in env.native.state()]
            expect = T.observe(T.ROLLOUT, b, j, np.zeros((48, 14)), env.meta)
            np.testing.assert_allclose(obs.cpu().numpy(), expect, rtol=2e-5, atol=2e-5)
        else:
            assert not bool(done.any()) and bool((env.returns != before).all())


def _check_step_rollout(env, actions):
    saved = env.auto_reset
    env.auto_reset = False
    try:
        obs, done, info = _check_step(env, T.ROLLOUT, actions, 2e-5, fall_height=0.08)
    finally:
        env.auto_reset = saved
    env.reset(done)
    return env._obs, done, info


def test_reset_draws_follow_the_reference_generator(model_dir):
    """tensor_env.py:178-197: q = HOME + (U - 0.5) 0.02, root rotation vector
    x/y = (U - 0.5) 0.02, +1 mm height, drawn from Generator(seed) on the env
    device in this order; the reset state equals the oracle's reset from the
    same draws."""
    from oracle.oracle import Oracle

    env = TensorEnv(model_dir, 16, ITER, DT, 1, seed=11)
    g = torch.Generator(device=DEV).manual_seed(11)
    q = env.home + (torch.rand((16, 14), generator=g, device=DEV) - 0.5) * 0.02
    roots = torch.zeros(16, 6, device=DEV)
    roots[:, 3:5] = (torch.rand((16, 2), generator=g, device=DEV) - 0.5) * 0.02
    roots[:, 2] = 0.001
    b = _np(env.native.state()[0])
    for e in range(16):
        o = Oracle(model_dir / "microduck.duck", DT, ITER, False)
        o.reset(q[e].cpu().double().numpy(), roots[e].cpu().double().numpy())
        np.testing.assert_allclose(b[e], o.snapshot()[0], atol=1e-6)
    obs, info = env.get_observations()
    assert obs.shape == (16, 52) and info == {"observations": {}}


@pytest.mark.parametrize("fp64", [False, True])
def test_reset_inputs_equal_the_torch_expressions(model_dir, fp64):
    """duck_task_reset_inputs against the reference's torch expressions
    (tensor_env.py:196-217) on the same draws, bit for bit: q, the root
    offsets, and the commands for drawn directions, one fixed direction and
    none; a TensorEnv's commands after a reset equal the expression on its
    generator's draws."""
    E, J = 64, 14
    dtype = torch.float64 if fp64 else torch.float32
    env = TensorEnv(model_dir, E, ITER, DT, 1, seed=5, task="locomotion", fp64=fp64)
    g = torch.Generator(device=DEV).manual_seed(123)
    u = torch.rand((E, J), generator=g, device=DEV, dtype=dtype)
    v = torch.rand((E, 2), generator=g, device=DEV, dtype=dtype)
    sel = torch.randint(4, (E,), generator=g, device=DEV)
    mask = torch.rand(E, generator=g, device=DEV) < 0.5
    old = torch.rand((E, 2), generator=g, device=DEV, dtype=dtype)
    table = torch.tensor([[1.0, 0], [-1, 0], [0, 1], [0, -1]], device=DEV, dtype=dtype)
    home = torch.tensor(env.meta["home"], device=DEV, dtype=dtype)
    speed = env.command_speed

    q_ref = home.expand(E, -1).clone()
    q_ref += (u - 0.5) * 0.02
    roots_ref = torch.zeros(E, 6, device=DEV, dtype=dtype)
    roots_ref[:, 3:5] = (v - 0.5) * 0.02
    roots_ref[:, 2] = 0.001
    for selected, direction in ((sel, -1), (None, 2), (None, -1)):
        q, roots = torch.empty(E, J, device=DEV, dtype=dtype), torch.empty(E, 6, device=DEV, dtype=dtype)
        commands = torch.full((E, 2), 7.0, device=DEV, dtype=dtype)
        draw = selected is not None or direction >= 0
        env.native.task_reset_inputs(env.spec, mask, u, v, selected, direction, speed,
                                     old if draw else None, q, roots, commands if draw else None)
        assert torch.equal(q, q_ref) and torch.equal(roots, roots_ref)
        if draw:
            chosen = selected if selected is not None else torch.full((E,), direction, device=DEV)
            expected = torch.where(mask[:, None], table[chosen] * speed, old)
            assert torch.equal(commands, expected)
        else:
            assert bool((commands == 7.0).all())
    # without draws: HOME and zero offsets
    q, roots = torch.empty(E, J, device=DEV, dtype=dtype), torch.empty(E, 6, device=DEV, dtype=dtype)
    env.native.task_reset_inputs(env.spec, mask, None, None, None, -1, speed, None, q, roots, None)
    assert torch.equal(q, home.expand(E, -1)) and bool((roots == 0).all())
    # a TensorEnv reset: the generator's draws in the reference's order
    g = torch.Generator(device=DEV).manual_seed(5)
    torch.rand((E, J), generator=g, device=DEV, dtype=dtype)
    torch.rand((E, 2), generator=g, device=DEV, dtype=dtype)
    first = torch.randint(4, (E,), generator=g, device=DEV)
    assert torch.equal(env.commands, table[first] * speed)
    with pytest.raises(RuntimeError, match="reset mask"):
        env.native.task_reset_inputs(env.spec, None, u, v, sel, -1, speed, old, q, roots, commands)
    with pytest.raises(RuntimeError, match="direction"):
        env.native.task_reset_inputs(env.spec, mask, u, v, None, 4, speed, old, q, roots, commands)


def test_task_argument_checks(model_dir):
    env = TensorEnv(model_dir, 8, ITER, DT, 1)
    with pytest.raises(RuntimeError):
        env.step(torch.zeros(8, 13, device=DEV))
    with pytest.raises(ValueError):
        TensorEnv(model_dir, 8, ITER, DT, 1, task="jumping")
    with pytest.raises(ValueError):
        TensorEnv(model_dir, 8, ITER, DT, 1, backend="cpu")
    with pytest.raises(ValueError):
        TensorEnv(model_dir, 8, ITER, DT, 0)


@pytest.mark.parametrize("task,kw", [("standing", {}), ("locomotion", {"velocity_filter_seconds": 0.2}),
                                     ("rollout", {})])
def test_observations_from_state_equal_the_kernel(model_dir, task, kw):
    """`observations(state())` (torch, tensor_env.py:238-258) and
    `get_observations()` (the task kernel) give the same rows."""
    env = TensorEnv(model_dir, 16, iterations=ITER, dt=DT, substeps=4, seed=3, task=task,
                    auto_reset=False, **kw)
    rng = np.random.default_rng(6)
    for _ in range(6):
        env.step(torch.tensor(rng.uniform(-0.5, 0.5, (16, 14)), dtype=torch.float32, device=DEV))
        torch_rows = env.observations(env.state())
        kernel_rows, _ = env.get_observations()
        assert torch_rows.shape == kernel_rows.shape
        np.testing.assert_allclose(_np(torch_rows), _np(kernel_rows), rtol=1e-5, atol=2e-6)
