"""Gymnasium-style single and vector environments, the counterpart of
python/zeno/gym/registration.py.

ZenoGymnasiumEnv wraps one environment (registration.py:90-328) and ZenoVectorEnv the whole
batch with auto-reset of finished envs (registration.py:331-612); make_vec, make_sb3_env,
check_env and register_envs follow registration.py:615-779. When gymnasium is importable
the classes derive from gymnasium.Env / gymnasium.vector.VectorEnv and use its Box spaces
and registry; without it (as in this image) they use the small Box below and keep the same
methods, shapes and dtypes, where the reference would raise ImportError.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from .env import ZenoEnv, find_model

try:  # pragma: no cover - gymnasium is not part of this image
    import gymnasium as _gymnasium
    from gymnasium import spaces as _spaces
    from gymnasium.vector import VectorEnv as _VectorEnv
    HAS_GYMNASIUM = True
except ImportError:
    _gymnasium = None
    _spaces = None
    _VectorEnv = object
    HAS_GYMNASIUM = False

ENV_CONFIGS = {
    "Pendulum": {"mjcf_file": "pendulum.xml", "max_episode_steps": 200, "reward_threshold": -200.0},
    "Cartpole": {"mjcf_file": "cartpole.xml", "max_episode_steps": 500, "reward_threshold": 475.0},
    "Ant": {"mjcf_file": "ant.xml", "max_episode_steps": 1000, "reward_threshold": 6000.0},
    "Humanoid": {"mjcf_file": "humanoid.xml", "max_episode_steps": 1000, "reward_threshold": 6000.0},
    "HalfCheetah": {"mjcf_file": "cheetah.xml", "max_episode_steps": 1000, "reward_threshold": 4800.0},
    "Hopper": {"mjcf_file": "hopper.xml", "max_episode_steps": 1000, "reward_threshold": 3800.0},
    "Walker2d": {"mjcf_file": "walker.xml", "max_episode_steps": 1000, "reward_threshold": 5000.0},
    "Swimmer": {"mjcf_file": "swimmer.xml", "max_episode_steps": 1000, "reward_threshold": 360.0},
    "Reacher": {"mjcf_file": "reacher.xml", "max_episode_steps": 50, "reward_threshold": -3.75},
    "Pusher": {"mjcf_file": "pusher.xml", "max_episode_steps": 100, "reward_threshold": 0.0},
}


class Box:
    """A bounded (or unbounded) float box: the part of gymnasium.spaces.Box these envs use."""

    def __init__(self, low: float, high: float, shape: Tuple[int, ...], dtype=np.float32, seed: Optional[int] = None):
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.low = np.full(self.shape, low, dtype=self.dtype)
        self.high = np.full(self.shape, high, dtype=self.dtype)
        self._rng = np.random.default_rng(seed)

    def seed(self, seed: Optional[int] = None) -> None:
        self._rng = np.random.default_rng(seed)

    def sample(self) -> np.ndarray:
        bounded = np.isfinite(self.low) & np.isfinite(self.high)
        out = self._rng.standard_normal(self.shape)
        u = self._rng.uniform(np.where(bounded, self.low, 0.0), np.where(bounded, self.high, 1.0))
        return np.where(bounded, u, out).astype(self.dtype)

    def contains(self, x) -> bool:
        x = np.asarray(x)
        return (x.shape == self.shape and np.can_cast(x.dtype, self.dtype)
                and bool(np.all(x >= self.low)) and bool(np.all(x <= self.high)))

    def __repr__(self) -> str:
        return f"Box({float(self.low.flat[0]) if self.low.size else 0}, {float(self.high.flat[0]) if self.high.size else 0}, {self.shape}, {self.dtype})"


def _box(low: float, high: float, shape: Tuple[int, ...]):
    if HAS_GYMNASIUM:  # pragma: no cover
        return _spaces.Box(low=low, high=high, shape=shape, dtype=np.float32)
    return Box(low, high, shape)


class ZenoGymnasiumEnv(_gymnasium.Env if HAS_GYMNASIUM else object):
    """One environment with the Gymnasium reset/step API (registration.py:90-328)."""

    metadata = {"render_modes": ["rgb_array", "human"], "render_fps": 60}

    def __init__(self, mjcf_path: str, render_mode: Optional[str] = None, max_episode_steps: int = 1000, **kwargs):
        if HAS_GYMNASIUM:  # pragma: no cover
            super().__init__()
        kwargs["num_envs"] = 1
        self._env = ZenoEnv(mjcf_path=str(find_model(mjcf_path)), **kwargs)
        self._mjcf_path = mjcf_path
        self.render_mode = render_mode
        self._max_episode_steps = max_episode_steps
        self._elapsed_steps = 0
        self.observation_space = _box(-np.inf, np.inf, (self._env.observation_dim,))
        self.action_space = _box(-1.0, 1.0, (self._env.action_dim,))

    @property
    def unwrapped(self) -> "ZenoGymnasiumEnv":
        return self

    def reset(self, *, seed: Optional[int] = None, options: Optional[Dict[str, Any]] = None):
        if HAS_GYMNASIUM:  # pragma: no cover
            super().reset(seed=seed)
        if seed is not None:
            self._np_random = np.random.default_rng(seed)
            self.action_space.seed(seed)
        obs = self._env.reset()
        self._elapsed_steps = 0
        return obs[0].astype(np.float32), {"TimeLimit.truncated": False}

    def step(self, action: np.ndarray):
        action = np.asarray(action, dtype=np.float32)
        if action.shape != (self._env.action_dim,):
            action = action.reshape(self._env.action_dim)
        obs, rewards, dones, env_info = self._env.step(action.reshape(1, -1))
        self._elapsed_steps += 1
        terminated = bool(dones[0])
        truncated = self._elapsed_steps >= self._max_episode_steps
        info = {"TimeLimit.truncated": truncated and not terminated, "episode_step": self._elapsed_steps}
        if "truncated" in env_info:
            info["env_truncated"] = env_info["truncated"][0]
        return obs[0].astype(np.float32), float(rewards[0]), terminated, truncated, info

    def render(self) -> Optional[np.ndarray]:
        """rgb_array: body positions of the env projected on the x-z plane as dots
        (registration.py:277-317); human: nothing."""
        if self.render_mode != "rgb_array":
            return None
        positions = self._env.get_body_positions()[0]
        width, height = 640, 480
        frame = np.empty((height, width, 3), dtype=np.uint8)
        frame[:] = (135, 206, 235)
        yy, xx = np.mgrid[-5:6, -5:6]
        disk = xx * xx + yy * yy <= 25
        for pos in positions:
            x = int(width / 2 + pos[0] * 100)
            y = int(height / 2 - pos[2] * 100)
            if 0 <= x < width and 0 <= y < height:
                px, py = x + xx[disk], y + yy[disk]
                ok = (px >= 0) & (px < width) & (py >= 0) & (py < height)
                frame[py[ok], px[ok]] = (255, 100, 100)
        return frame

    def close(self) -> None:
        self._env.close()

    def get_wrapper_attr(self, name: str) -> Any:
        return getattr(self, name)


class ZenoVectorEnv(_VectorEnv):
    """The whole batch with the Gymnasium vector API and auto-reset (registration.py:331-612):
    an env that terminated or hit max_episode_steps is reset at the start of the next step."""

    def __init__(self, mjcf_path: str, num_envs: int = 1, max_episode_steps: int = 1000, **kwargs):
        self._env = ZenoEnv(mjcf_path=str(find_model(mjcf_path)), num_envs=num_envs, **kwargs)
        self._mjcf_path = mjcf_path
        self._max_episode_steps = max_episode_steps
        self._elapsed_steps = np.zeros(num_envs, dtype=np.int32)
        obs_dim, act_dim = self._env.observation_dim, self._env.action_dim
        single_obs = _box(-np.inf, np.inf, (obs_dim,))
        single_act = _box(-1.0, 1.0, (act_dim,))
        if HAS_GYMNASIUM:  # pragma: no cover
            super().__init__(num_envs=num_envs, observation_space=single_obs, action_space=single_act)
        else:
            self.num_envs = num_envs
            self.single_observation_space = single_obs
            self.single_action_space = single_act
            self.observation_space = Box(-np.inf, np.inf, (num_envs, obs_dim))
            self.action_space = Box(-1.0, 1.0, (num_envs, act_dim))
        self._autoreset_envs = np.zeros(num_envs, dtype=bool)
        self._pending_actions = None
        self._pending_reset = False

    @property
    def unwrapped(self) -> "ZenoVectorEnv":
        return self

    def reset(self, *, seed: Optional[Union[int, List[int]]] = None, options: Optional[Dict[str, Any]] = None):
        if seed is not None:
            seeds = [seed + i for i in range(self.num_envs)] if isinstance(seed, int) else list(seed)
            self._np_random = np.random.default_rng(seeds[0])
            self.action_space.seed(seeds[0])
        obs = self._env.reset()
        self._elapsed_steps[:] = 0
        self._autoreset_envs[:] = False
        return obs.astype(np.float32), {"TimeLimit.truncated": np.zeros(self.num_envs, dtype=bool),
                                        "_elapsed_steps": self._elapsed_steps.copy()}

    def step(self, actions: np.ndarray):
        actions = np.asarray(actions, dtype=np.float32)
        if np.any(self._autoreset_envs):
            self._env.reset(self._autoreset_envs.astype(np.uint8))
            self._elapsed_steps[self._autoreset_envs] = 0
            self._autoreset_envs[:] = False
        obs, rewards, dones, _ = self._env.step(actions)
        self._elapsed_steps += 1
        terminated = dones.astype(bool)
        truncated = self._elapsed_steps >= self._max_episode_steps
        self._autoreset_envs = terminated | truncated
        infos = {
            "TimeLimit.truncated": truncated & ~terminated,
            "_elapsed_steps": self._elapsed_steps.copy(),
            "final_observation": np.array([None] * self.num_envs, dtype=object),
            "final_info": np.array([{}] * self.num_envs, dtype=object),
        }
        for i in np.where(self._autoreset_envs)[0]:
            infos["final_observation"][i] = obs[i].copy()
            infos["final_info"][i] = {"episode_step": int(self._elapsed_steps[i])}
        return obs.astype(np.float32), rewards.astype(np.float32), terminated, truncated, infos

    def reset_async(self, seed=None, options=None) -> None:
        self._pending_reset = True
        self._reset_seed = seed
        self._reset_options = options

    def reset_wait(self, timeout: Optional[float] = None, seed=None, options=None):
        seed = seed or getattr(self, "_reset_seed", None)
        options = options or getattr(self, "_reset_options", None)
        self._pending_reset = False
        return self.reset(seed=seed, options=options)

    def step_async(self, actions: np.ndarray) -> None:
        self._pending_actions = np.asarray(actions, dtype=np.float32)

    def step_wait(self, timeout: Optional[float] = None):
        if self._pending_actions is None:
            raise RuntimeError("step_async must be called before step_wait")
        result = self.step(self._pending_actions)
        self._pending_actions = None
        return result

    def call(self, name: str, *args, **kwargs) -> Tuple[Any, ...]:
        method = getattr(self._env, name, None)
        if method is None:
            raise AttributeError(f"Environment has no method '{name}'")
        if callable(method):
            result = method(*args, **kwargs)
            return (result,) * self.num_envs if not isinstance(result, np.ndarray) else tuple(result)
        raise TypeError(f"'{name}' is not callable")

    def get_attr(self, name: str) -> Tuple[Any, ...]:
        return (getattr(self._env, name),) * self.num_envs

    def set_attr(self, name: str, values: Union[Any, Sequence[Any]]) -> None:
        setattr(self._env, name, values[0] if isinstance(values, (list, tuple)) else values)

    def close_extras(self, **kwargs) -> None:
        self._env.close()

    def close(self) -> None:
        self.close_extras()

    def get_body_positions(self, zero_copy: bool = True) -> np.ndarray:
        return self._env.world.get_body_positions(zero_copy=zero_copy)

    def get_body_quaternions(self, zero_copy: bool = True) -> np.ndarray:
        return self._env.world.get_body_quaternions(zero_copy=zero_copy)

    def get_state(self) -> Dict[str, np.ndarray]:
        return self._env.world.get_state()

    def set_state(self, state: Dict[str, np.ndarray]) -> None:
        self._env.world.set_state(state)


def register_envs() -> None:
    """Registers Zeno/<Name>-v0 with gymnasium when it is importable (registration.py:615-639)."""
    if not HAS_GYMNASIUM:
        return
    for name, cfg in ENV_CONFIGS.items():  # pragma: no cover
        try:
            _gymnasium.register(id=f"Zeno/{name}-v0", entry_point="zeno_amd.gym:ZenoGymnasiumEnv",
                                kwargs={"mjcf_path": cfg["mjcf_file"]}, max_episode_steps=cfg["max_episode_steps"],
                                reward_threshold=cfg.get("reward_threshold"))
        except _gymnasium.error.Error:
            pass


def make_vec(model: str, num_envs: int = 1, **kwargs) -> ZenoVectorEnv:
    """ZenoVectorEnv for a model name or MJCF path (registration.py:642-699)."""
    return ZenoVectorEnv(mjcf_path=str(find_model(model)), num_envs=num_envs, **kwargs)


def make_sb3_env(model: str, num_envs: int = 1, **kwargs) -> ZenoVectorEnv:
    return make_vec(model, num_envs=num_envs, **kwargs)


def check_env(env: Union[ZenoGymnasiumEnv, ZenoVectorEnv]) -> bool:
    """reset, one sampled step, five return values, observation inside the space
    (registration.py:739-779)."""
    try:
        obs, info = env.reset()
        assert obs is not None, "Reset returned None observation"
        if isinstance(env, ZenoVectorEnv):
            assert obs.shape[0] == env.num_envs, "Wrong batch size"
        result = env.step(env.action_space.sample())
        assert len(result) == 5, "Step should return 5 values"
        obs = result[0]
        assert obs is not None, "Step returned None observation"
        space = env.single_observation_space if isinstance(env, ZenoVectorEnv) else env.observation_space
        assert space.contains(obs if obs.ndim == 1 else obs[0]), "Observation not in space"
        return True
    except Exception as e:  # noqa: BLE001 - reported, as in the reference
        print(f"Environment check failed: {e}")
        return False


try:
    register_envs()
except ImportError:  # pragma: no cover
    pass
