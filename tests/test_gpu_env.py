"""ZenoEnv, make and the Gymnasium-style environments on the GPU: the reference's
TestGymnasiumAPI, TestMultiEnvBatching and TestResetMasking behaviours
(tests/test_python_integration.py:270-570) for zeno_amd."""
import numpy as np
import pytest

from tests.test_gpu_api import PENDULUM_MJCF
from zeno_amd import ZenoEnv, make
from zeno_amd.gym import ZenoGymnasiumEnv, ZenoVectorEnv, check_env, make_vec

pytestmark = pytest.mark.gpu


def test_single_env_reset_step():
    env = ZenoGymnasiumEnv(mjcf_path="pendulum")
    obs, info = env.reset(seed=3)
    assert isinstance(obs, np.ndarray) and obs.dtype == np.float32
    assert obs.shape == env.observation_space.shape and isinstance(info, dict)
    obs, reward, terminated, truncated, info = env.step(env.action_space.sample())
    assert obs.shape == env.observation_space.shape
    assert isinstance(reward, float) and isinstance(terminated, bool) and isinstance(truncated, bool)
    assert env.observation_space.contains(obs)
    for _ in range(10):
        assert env.action_space.contains(env.action_space.sample())
    env.close()


def test_single_env_truncates_at_limit():
    env = ZenoGymnasiumEnv(mjcf_path="pendulum", max_episode_steps=3)
    env.reset()
    flags = [env.step(np.zeros(1, np.float32))[3] for _ in range(3)]
    assert flags == [False, False, True]
    assert env.render() is None
    env.close()
    env = ZenoGymnasiumEnv(mjcf_path="ant", render_mode="rgb_array")
    env.reset()
    frame = env.render()
    assert frame.shape == (480, 640, 3) and frame.dtype == np.uint8
    env.close()


def test_vector_env_reset_step_and_autoreset():
    env = ZenoVectorEnv(mjcf_path="pendulum", num_envs=8, max_episode_steps=4)
    obs, info = env.reset(seed=1)
    assert obs.shape == (8, 2) and obs.dtype == np.float32
    actions = env.action_space.sample()
    assert actions.shape == (8, 1)
    result = env.step(actions)
    assert len(result) == 5
    obs, rewards, terminated, truncated, info = result
    assert obs.shape[0] == 8 and rewards.shape == (8,) and rewards.dtype == np.float32
    assert terminated.dtype == bool and truncated.dtype == bool
    for _ in range(3):
        obs, rewards, terminated, truncated, info = env.step(np.ones((8, 1), np.float32))
    assert truncated.all() and info["final_observation"][0] is not None
    # The next step first resets every env (auto-reset), then steps once.
    env.step(np.zeros((8, 1), np.float32))
    assert np.all(info["_elapsed_steps"] == 4) and np.all(env.elapsed_steps == 1)
    assert info["_final_observation"].all() and info["final_info"][3] == {"episode_step": 4}
    assert check_env(env) is True
    env.step_async(np.zeros((8, 1), np.float32))
    assert len(env.step_wait()) == 5
    env.reset_async(seed=2)
    assert env.reset_wait()[0].shape == (8, 2)
    assert env.get_attr("num_envs") == (8,) * 8
    env.close()


def test_check_env_single():
    env = ZenoGymnasiumEnv(mjcf_path="pendulum")
    assert check_env(env) is True
    env.close()


def test_batched_env_and_make():
    with ZenoEnv(mjcf_string=PENDULUM_MJCF, num_envs=1024) as env:
        obs = env.reset()
        assert obs.shape == (1024, env.observation_dim)
        obs, rewards, dones, info = env.step(np.random.default_rng(0).uniform(-1, 1, (1024, env.action_dim)))
        assert obs.shape == (1024, env.observation_dim) and rewards.shape == (1024,) and dones.shape == (1024,)
        assert dones.dtype == bool and info["step_count"] == 1 and not info["truncated"].any()
    env = make("ant", num_envs=16)
    assert env.observation_shape == (16, 29) and env.action_shape == (16, 8)
    assert env.timestep == pytest.approx(0.01)
    env.close()
    venv = make_vec("humanoid", num_envs=4)
    assert venv.reset()[0].shape == (4, 39)
    venv.close()


def test_high_level_env_reset_with_mask():
    env = ZenoEnv(mjcf_string=PENDULUM_MJCF, num_envs=8)
    env.reset()
    for _ in range(20):
        env.step(np.ones((8, 1), np.float32))
    before = env.get_body_positions().copy()
    mask = np.zeros(8, np.uint8)
    mask[:4] = 1
    obs = env.reset(mask=mask)
    assert obs.shape == (8, env.observation_dim)
    after = env.get_body_positions()
    assert all(not np.array_equal(before[i], after[i]) for i in range(4))
    np.testing.assert_array_equal(before[4:], after[4:])
    env.close()
