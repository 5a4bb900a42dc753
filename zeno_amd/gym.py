"""Gymnasium-style environments over the batched ZenoEnv: the counterpart of
python/zeno/gym/registration.py (ZenoGymnasiumEnv :90-328, ZenoVectorEnv :331-612,
register_envs / make_vec / make_sb3_env / check_env :615-779).

Design. The whole batch lives in one ZenoEnv, so the vector environment needs no worker
processes: episode bookkeeping is a numpy array per environment (EpisodeClock), auto-reset
is one masked device reset issued before the next step, and the async calls only queue the
request that the matching *_wait call runs. The single environment is the same machinery at
batch size one. Both render the first environment with SideView, an orthographic x-z
rasteriser of the scene's geoms.

Interface kept from the reference (the names a user's code reads): the environment ids and
episode limits in ENV_CONFIGS; the info keys "TimeLimit.truncated", "_elapsed_steps",
"episode_step", "env_truncated", "final_observation" and "final_info"; observation space
(-inf, inf) and action space [-1, 1] in float32; auto-reset at the start of the step after an
episode ends. When gymnasium is importable the classes derive from gymnasium.Env /
gymnasium.vector.VectorEnv and use its Box; without it (as in this image) they use the Box
below with the same methods, shapes and dtypes, where the reference raises ImportError.
"""
from __future__ import annotations

import warnings
from typing import Any, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from .env import ZenoEnv, find_model

try:  # pragma: no cover - gymnasium is not part of this image
    import gymnasium as _gymnasium
    from gymnasium import spaces as _spaces
    from gymnasium.vector import VectorEnv as _VectorEnv
    from gymnasium.vector.utils import batch_space as _batch_space
    HAS_GYMNASIUM = True
except ImportError:
    _gymnasium = None
    _spaces = None
    _VectorEnv = object
    _batch_space = None
    HAS_GYMNASIUM = False

# Environment ids registered as Zeno/<name>-v0: asset file, episode limit, reward threshold.
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


class EpisodeClock:
    """Per-environment episode bookkeeping for a batch: steps taken since each env's last
    reset, the step limit, and which envs must be reset before the next step."""

    def __init__(self, num_envs: int, limit: int):
        self.limit = int(limit)
        self.steps = np.zeros(num_envs, dtype=np.int32)
        self.due = np.zeros(num_envs, dtype=bool)

    def restart(self, which: Optional[np.ndarray] = None) -> None:
        sel = slice(None) if which is None else which
        self.steps[sel] = 0
        self.due[sel] = False

    def collect_due(self) -> Optional[np.ndarray]:
        """The envs whose episode ended last step (then clears them), or None."""
        if not self.due.any():
            return None
        mask = self.due.copy()
        self.restart(mask)
        return mask

    def tick(self, terminated: np.ndarray) -> np.ndarray:
        """Counts one step; returns the truncation flags and marks ended episodes due."""
        self.steps += 1
        truncated = self.steps >= self.limit
        self.due = terminated | truncated
        return truncated


class SideView:
    """Orthographic side view of one environment: x to the right, z up, looking along +y.

    Every geom is drawn at its pose (body position plus the body-rotated local offset):
    spheres as discs, capsules as rounded segments, boxes as the rectangle bounding their
    rotated outline, planes as ground below their height. Geoms farther along +y are drawn
    first, so nearer ones cover them. The frame fits the non-plane geoms with a 15% margin
    on every side."""

    BACKGROUND = np.array([236, 240, 244], np.uint8)
    GROUND = np.array([92, 98, 108], np.uint8)
    PALETTE = np.array([[214, 96, 77], [67, 147, 195], [120, 170, 90], [230, 171, 2], [141, 106, 184],
                        [27, 158, 119], [217, 95, 2], [102, 102, 102]], np.uint8)

    def __init__(self, model: Dict[str, Any], width: int = 640, height: int = 480):
        g = model["geoms"]
        self.kind = g["type_body"][:, 0].astype(np.int64)
        self.body = g["type_body"][:, 1].astype(np.int64)
        self.local = g["pos_size0"][:, :3].astype(np.float64)
        self.radius = g["pos_size0"][:, 3].astype(np.float64)
        self.half = np.stack([g["pos_size0"][:, 3], g["params"][:, 0], g["params"][:, 1]], 1).astype(np.float64)
        self.gquat = g["quat"].astype(np.float64)
        self.width, self.height = int(width), int(height)

    @staticmethod
    def _rot(q: np.ndarray) -> np.ndarray:
        x, y, z, w = q / max(float(np.linalg.norm(q)), 1e-12)
        return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                         [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                         [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])

    def _shapes(self, positions: np.ndarray, quaternions: np.ndarray) -> List[Dict[str, Any]]:
        out = []
        for i in range(len(self.kind)):
            R = self._rot(quaternions[self.body[i]])
            centre = positions[self.body[i], :3] + R @ self.local[i]
            if not np.all(np.isfinite(centre)):
                continue
            s = {"kind": int(self.kind[i]), "c": centre, "colour": self.PALETTE[self.body[i] % len(self.PALETTE)]}
            if s["kind"] == 1:        # capsule: half segment along the rotated z axis
                s["seg"] = (R @ self._rot(self.gquat[i]))[:, 2] * self.half[i, 1]
                s["reach"] = np.abs(s["seg"]) + self.radius[i]
            elif s["kind"] == 2:      # box: half extents of its rotated outline's bounding box
                s["reach"] = np.abs(R @ self._rot(self.gquat[i])) @ self.half[i]
            else:
                s["reach"] = np.full(3, self.radius[i])
            s["r"] = self.radius[i]
            out.append(s)
        return out

    def draw(self, positions: np.ndarray, quaternions: np.ndarray) -> np.ndarray:
        """The rgb frame (height, width, 3) uint8 for one env's body poses."""
        shapes = self._shapes(np.asarray(positions, np.float64), np.asarray(quaternions, np.float64))
        solid = [s for s in shapes if s["kind"] != 3]
        if solid:
            lo = np.min([s["c"] - s["reach"] for s in solid], axis=0)
            hi = np.max([s["c"] + s["reach"] for s in solid], axis=0)
        else:
            lo, hi = np.full(3, -1.0), np.full(3, 1.0)
        extent = max(hi[0] - lo[0], hi[2] - lo[2], 1e-3) * 1.3
        px = min(self.width, self.height) / extent                 # pixels per metre
        xs = 0.5 * (lo[0] + hi[0]) + (np.arange(self.width) + 0.5 - 0.5 * self.width) / px
        zs = 0.5 * (lo[2] + hi[2]) - (np.arange(self.height) + 0.5 - 0.5 * self.height) / px
        X, Z = np.meshgrid(xs, zs)
        frame = np.empty((self.height, self.width, 3), np.uint8)
        frame[:] = self.BACKGROUND
        for s in sorted(shapes, key=lambda s: -s["c"][1]):
            c = s["c"]
            if s["kind"] == 3:
                frame[Z <= c[2]] = self.GROUND
                continue
            if s["kind"] == 1:
                a = c - s["seg"]
                d = 2.0 * s["seg"][[0, 2]]
                t = np.clip(((X - a[0]) * d[0] + (Z - a[2]) * d[1]) / max(float(d @ d), 1e-12), 0.0, 1.0)
                inside = (X - a[0] - t * d[0]) ** 2 + (Z - a[2] - t * d[1]) ** 2 <= s["r"] ** 2
            elif s["kind"] == 2:
                inside = (np.abs(X - c[0]) <= s["reach"][0]) & (np.abs(Z - c[2]) <= s["reach"][2])
            else:
                inside = (X - c[0]) ** 2 + (Z - c[2]) ** 2 <= s["r"] ** 2
            frame[inside] = s["colour"]
        return frame


def _per_env(value: Any, n: int) -> Tuple[Any, ...]:
    """One entry per env: an array whose first axis is the batch is split along it, anything
    else (a scalar, a method's single result) is repeated."""
    if isinstance(value, np.ndarray) and value.ndim >= 1 and value.shape[0] == n:
        return tuple(value)
    return tuple(value for _ in range(n))


def _same(a: Any, b: Any) -> bool:
    if isinstance(a, np.ndarray) or isinstance(b, np.ndarray):
        return np.array_equal(np.asarray(a), np.asarray(b))
    return a is b or a == b


class ZenoGymnasiumEnv(_gymnasium.Env if HAS_GYMNASIUM else object):
    """One environment with the Gymnasium reset/step API: a batch of one, its episode clock,
    and a side-view renderer. It does not reset itself; truncation is reported once the
    episode reaches max_episode_steps."""

    metadata = {"render_modes": ["rgb_array", "human"], "render_fps": 60}

    def __init__(self, mjcf_path: str, render_mode: Optional[str] = None, max_episode_steps: int = 1000, **kwargs):
        if HAS_GYMNASIUM:  # pragma: no cover
            super().__init__()
        kwargs.pop("num_envs", None)
        self.mjcf_path = str(find_model(mjcf_path))
        self.batch = ZenoEnv(mjcf_path=self.mjcf_path, num_envs=1, **kwargs)
        self.clock = EpisodeClock(1, max_episode_steps)
        self.render_mode = render_mode
        self.observation_space = _box(-np.inf, np.inf, (self.batch.observation_dim,))
        self.action_space = _box(-1.0, 1.0, (self.batch.action_dim,))
        self._side_view: Optional[SideView] = None

    @property
    def unwrapped(self) -> "ZenoGymnasiumEnv":
        return self

    @property
    def elapsed_steps(self) -> int:
        return int(self.clock.steps[0])

    @property
    def max_episode_steps(self) -> int:
        return self.clock.limit

    def reset(self, *, seed: Optional[int] = None, options: Optional[Dict[str, Any]] = None):
        if HAS_GYMNASIUM:  # pragma: no cover
            super().reset(seed=seed)
        if seed is not None:
            self.action_space.seed(seed)
        first = self.batch.reset()[0]
        self.clock.restart()
        return first.astype(np.float32, copy=False), {"TimeLimit.truncated": False}

    def step(self, action: np.ndarray):
        batch_action = np.asarray(action, dtype=np.float32).reshape(1, self.batch.action_dim)
        obs, rewards, dones, batch_info = self.batch.step(batch_action)
        terminated = bool(dones[0])
        truncated = bool(self.clock.tick(np.asarray(dones, bool))[0])
        info = {"TimeLimit.truncated": truncated and not terminated, "episode_step": self.elapsed_steps,
                "env_truncated": bool(batch_info["truncated"][0])}
        return obs[0].astype(np.float32, copy=False), float(rewards[0]), terminated, truncated, info

    def render(self) -> Optional[np.ndarray]:
        """rgb_array: the SideView frame of the environment; other modes draw nothing."""
        if self.render_mode != "rgb_array":
            return None
        if self._side_view is None:
            self._side_view = SideView(self.batch.world.model_view())
        w = self.batch.world
        return self._side_view.draw(w.get_body_positions(zero_copy=False)[0], w.get_body_quaternions(zero_copy=False)[0])

    def close(self) -> None:
        self.batch.close()

    def get_wrapper_attr(self, name: str) -> Any:
        return getattr(self, name)


class ZenoVectorEnv(_VectorEnv):
    """The whole batch with the Gymnasium vector API. An env whose episode ended (terminated,
    or max_episode_steps reached) is reset at the start of the next step call, in one masked
    device reset for all such envs; the step that ends an episode reports the observation it
    ended with under info["final_observation"]."""

    metadata = {"render_modes": ["rgb_array"], "autoreset_mode": "next_step"}

    def __init__(self, mjcf_path: str, num_envs: int = 1, max_episode_steps: int = 1000,
                 render_mode: Optional[str] = None, **kwargs):
        self.mjcf_path = str(find_model(mjcf_path))
        self.batch = ZenoEnv(mjcf_path=self.mjcf_path, num_envs=num_envs, **kwargs)
        self.clock = EpisodeClock(num_envs, max_episode_steps)
        self.render_mode = render_mode
        obs_dim, act_dim = self.batch.observation_dim, self.batch.action_dim
        # The spaces are set as attributes, which both gymnasium's older VectorEnv (whose
        # constructor takes them) and its newer one (whose constructor takes nothing) read.
        self.num_envs = num_envs
        self.single_observation_space = _box(-np.inf, np.inf, (obs_dim,))
        self.single_action_space = _box(-1.0, 1.0, (act_dim,))
        if HAS_GYMNASIUM:  # pragma: no cover
            self.observation_space = _batch_space(self.single_observation_space, num_envs)
            self.action_space = _batch_space(self.single_action_space, num_envs)
        else:
            self.observation_space = Box(-np.inf, np.inf, (num_envs, obs_dim))
            self.action_space = Box(-1.0, 1.0, (num_envs, act_dim))
        self.closed = False
        self._request: Optional[Tuple[Any, ...]] = None    # queued by *_async, run by *_wait
        self._side_view: Optional[SideView] = None

    @property
    def unwrapped(self) -> "ZenoVectorEnv":
        return self

    @property
    def elapsed_steps(self) -> np.ndarray:
        """Steps since each env's last reset (a copy)."""
        return self.clock.steps.copy()

    @property
    def max_episode_steps(self) -> int:
        return self.clock.limit

    # ---- reset / step ---------------------------------------------------------------------
    def reset(self, *, seed: Optional[Union[int, List[int]]] = None, options: Optional[Dict[str, Any]] = None):
        """Resets every env, or those in options["reset_mask"] (a bool per env). A seed (one
        int, or one per env of which the first is used) seeds the action spaces' sampling;
        the simulation itself is deterministic."""
        if seed is not None:
            first = int(seed) if np.isscalar(seed) else int(list(seed)[0])
            self.action_space.seed(first)
            self.single_action_space.seed(first)
        mask = None
        if options and options.get("reset_mask") is not None:
            mask = np.asarray(options["reset_mask"], dtype=bool).reshape(self.num_envs)
        obs = self.batch.reset(None if mask is None else mask.astype(np.uint8))
        self.clock.restart(mask)
        info = {"TimeLimit.truncated": np.zeros(self.num_envs, dtype=bool), "_elapsed_steps": self.elapsed_steps}
        return obs.astype(np.float32, copy=False), info

    def step(self, actions: np.ndarray):
        due = self.clock.collect_due()
        if due is not None:
            self.batch.reset(due.astype(np.uint8))
        obs, rewards, dones, _ = self.batch.step(np.asarray(actions, dtype=np.float32))
        terminated = np.asarray(dones, dtype=bool)
        truncated = self.clock.tick(terminated)
        return (obs.astype(np.float32, copy=False), np.asarray(rewards, np.float32), terminated, truncated,
                self._episode_info(obs, terminated, truncated))

    def _episode_info(self, obs: np.ndarray, terminated: np.ndarray, truncated: np.ndarray) -> Dict[str, Any]:
        ended = terminated | truncated
        final_obs = np.full(self.num_envs, None, dtype=object)
        final_info = np.empty(self.num_envs, dtype=object)
        for i in range(self.num_envs):
            final_info[i] = {}
        for i in np.flatnonzero(ended):
            final_obs[i] = np.array(obs[i], dtype=np.float32)
            final_info[i]["episode_step"] = int(self.clock.steps[i])
        return {"TimeLimit.truncated": truncated & ~terminated, "_elapsed_steps": self.elapsed_steps,
                "final_observation": final_obs, "_final_observation": ended.copy(),
                "final_info": final_info, "_final_info": ended.copy()}

    # ---- async form: the request is queued and run by the matching wait ---------------------
    def _take(self, kind: str) -> Tuple[Any, ...]:
        if self._request is None or self._request[0] != kind:
            raise RuntimeError(f"{kind}_wait has no pending {kind}_async request")
        request, self._request = self._request, None
        return request[1:]

    def reset_async(self, seed: Optional[Union[int, List[int]]] = None, options: Optional[Dict[str, Any]] = None) -> None:
        self._request = ("reset", seed, options)

    def reset_wait(self, timeout: Optional[float] = None, seed=None, options=None):
        queued_seed, queued_options = self._take("reset")
        return self.reset(seed=queued_seed if seed is None else seed,
                          options=queued_options if options is None else options)

    def step_async(self, actions: np.ndarray) -> None:
        self._request = ("step", np.array(actions, dtype=np.float32))

    def step_wait(self, timeout: Optional[float] = None):
        (actions,) = self._take("step")
        return self.step(actions)

    # ---- attributes of the batched env ---------------------------------------------------------
    def call(self, name: str, *args, **kwargs) -> Tuple[Any, ...]:
        """Calls ZenoEnv method `name` once for the whole batch (or reads the attribute when it
        is not callable) and returns one entry per env."""
        target = getattr(self.batch, name)
        return _per_env(target(*args, **kwargs) if callable(target) else target, self.num_envs)

    def get_attr(self, name: str) -> Tuple[Any, ...]:
        return _per_env(getattr(self.batch, name), self.num_envs)

    def set_attr(self, name: str, values: Union[Any, Sequence[Any]]) -> None:
        """Sets a ZenoEnv attribute. One batch holds every env, so a per-env sequence must
        hold num_envs equal values."""
        if isinstance(values, (list, tuple)):
            if len(values) != self.num_envs or not all(_same(v, values[0]) for v in values):
                raise ValueError(f"set_attr({name!r}): the envs share one batch; give one value or "
                                 f"{self.num_envs} equal values")
            values = values[0]
        setattr(self.batch, name, values)

    def render(self) -> Optional[np.ndarray]:
        """rgb_array: the SideView frame of env 0."""
        if self.render_mode != "rgb_array":
            return None
        if self._side_view is None:
            self._side_view = SideView(self.batch.world.model_view())
        w = self.batch.world
        return self._side_view.draw(w.get_body_positions(zero_copy=False)[0], w.get_body_quaternions(zero_copy=False)[0])

    def close_extras(self, **kwargs) -> None:
        self.batch.close()

    def close(self, **kwargs) -> None:
        if not self.closed:
            self.close_extras(**kwargs)
            self.closed = True

    # ---- state access beyond the Gymnasium API -----------------------------------------------
    def get_body_positions(self, zero_copy: bool = True) -> np.ndarray:
        return self.batch.world.get_body_positions(zero_copy=zero_copy)

    def get_body_quaternions(self, zero_copy: bool = True) -> np.ndarray:
        return self.batch.world.get_body_quaternions(zero_copy=zero_copy)

    def get_state(self) -> Dict[str, np.ndarray]:
        return self.batch.world.get_state()

    def set_state(self, state: Dict[str, np.ndarray]) -> None:
        self.batch.world.set_state(state)


def register_envs() -> List[str]:
    """Adds every ENV_CONFIGS entry to gymnasium's registry as Zeno/<name>-v0 (ids already
    present are left alone) and returns the ids added; without gymnasium, none."""
    if not HAS_GYMNASIUM:
        return []
    added = []
    for name, cfg in ENV_CONFIGS.items():  # pragma: no cover
        env_id = f"Zeno/{name}-v0"
        if env_id in _gymnasium.envs.registry:
            continue
        _gymnasium.register(id=env_id, entry_point=f"{__name__}:ZenoGymnasiumEnv",
                            kwargs={"mjcf_path": cfg["mjcf_file"]}, max_episode_steps=cfg["max_episode_steps"],
                            reward_threshold=cfg["reward_threshold"])
        added.append(env_id)
    return added


def make_vec(model: str, num_envs: int = 1, **kwargs) -> ZenoVectorEnv:
    """A ZenoVectorEnv for a model name ("ant") or an MJCF path; other keyword arguments go to
    ZenoVectorEnv and on to ZenoEnv."""
    return ZenoVectorEnv(mjcf_path=model, num_envs=num_envs, **kwargs)


def make_sb3_env(model: str, num_envs: int = 1, **kwargs) -> ZenoVectorEnv:
    """The vector environment under the name Stable-Baselines3 users look for."""
    return make_vec(model, num_envs=num_envs, **kwargs)


def check_env(env: Union[ZenoGymnasiumEnv, ZenoVectorEnv]) -> bool:
    """Exercises reset and one step with a sampled action and checks what they return against
    the Gymnasium API: (obs, info) and (obs, reward, terminated, truncated, info), a batch of
    num_envs rows for a vector env, every observation row inside the observation space.
    Returns True when all hold; otherwise warns once per failed check and returns False."""
    vector = isinstance(env, ZenoVectorEnv)
    space = env.single_observation_space if vector else env.observation_space
    failed: List[str] = []

    def rows_ok(obs: Any, when: str) -> None:
        rows = np.asarray(obs)
        rows = rows if vector else rows[None]
        if vector and rows.shape[0] != env.num_envs:
            failed.append(f"{when}: {rows.shape[0]} observation rows for {env.num_envs} envs")
        elif not all(space.contains(r) for r in rows):
            failed.append(f"{when}: observation outside {space}")

    try:
        out = env.reset()
        if not (isinstance(out, tuple) and len(out) == 2 and isinstance(out[1], dict)):
            failed.append("reset() does not return (observation, info dict)")
        else:
            rows_ok(out[0], "reset()")
        out = env.step(env.action_space.sample())
        if not (isinstance(out, tuple) and len(out) == 5 and isinstance(out[4], dict)):
            failed.append("step() does not return (observation, reward, terminated, truncated, info dict)")
        else:
            rows_ok(out[0], "step()")
    except Exception as exc:  # noqa: BLE001 - a raising environment fails the check
        failed.append(f"{type(exc).__name__}: {exc}")
    for what in failed:
        warnings.warn(f"check_env: {what}", stacklevel=2)
    return not failed


register_envs()
