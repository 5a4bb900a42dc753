"""Batched environments over ZenoWorld, with the behaviour of the reference's
python/zeno/env.py (ZenoEnv: env.py:13-213, make: env.py:216-267):

* ``ZenoEnv`` owns one world holding ``num_envs`` copies of an MJCF scene.
* ``step(actions)`` advances every copy once and returns ``(observations, rewards, dones,
  info)``. Observations are a new array on each call; rewards and dones are the world's
  (the reference's step writes neither, so they stay zero). ``info`` holds the number of
  steps since the last reset and a per-env truncation flag, raised for every env once that
  number reaches the episode limit of 1000 steps.
* ``reset(mask)`` restores the selected copies (all without a mask), restarts the step
  count and returns the observations.
* ``make(model)`` accepts an existing MJCF path, or a model name (".xml" optional) looked up
  in this package's assets, then ./assets, then ~/.zeno/assets.
"""
from __future__ import annotations

from pathlib import Path
from typing import Any, Dict, Optional, Tuple

import numpy as np

from .world import ZenoWorld

EPISODE_LIMIT = 1000

# Where model names are looked up, in order: the ten MJCF files shipped with this package,
# the working directory's assets/, the user's ~/.zeno/assets/.
ASSET_DIRS: Tuple[Path, ...] = (
    Path(__file__).resolve().parent / "assets",
    Path.cwd() / "assets",
    Path.home() / ".zeno" / "assets",
)


def find_model(model: str) -> Path:
    """Path of the MJCF file that `model` names: `model` itself when that file exists,
    else the first ASSET_DIRS entry holding it (".xml" is appended to a bare name)."""
    given = Path(model)
    if given.exists():
        return given
    file_name = model if model.endswith(".xml") else model + ".xml"
    for where in ASSET_DIRS:
        candidate = where / file_name
        if candidate.is_file():
            return candidate
    searched = ", ".join(str(d) for d in ASSET_DIRS)
    raise FileNotFoundError(f"no MJCF model {file_name!r} in {searched}")


class ZenoEnv:
    """`num_envs` copies of one scene stepped together on the GPU."""

    def __init__(self, mjcf_path: Optional[str] = None, mjcf_string: Optional[str] = None, num_envs: int = 1,
                 timestep: float = 0, contact_iterations: int = 4, max_contacts_per_env: int = 64,
                 seed: int = 42, substeps: int = 1):
        self.world = ZenoWorld(mjcf_path=mjcf_path, mjcf_string=mjcf_string, num_envs=num_envs,
                               timestep=timestep, contact_iterations=contact_iterations,
                               max_contacts_per_env=max_contacts_per_env, seed=seed, substeps=substeps)
        self.mjcf_path = mjcf_path
        self.max_episode_steps = EPISODE_LIMIT
        self.steps_since_reset = 0

    # The reference's attribute names for the world and the model path
    # (python/zeno/__init__.py:49 documents env._world.get_body_positions(zero_copy=True)).
    @property
    def _world(self) -> ZenoWorld:
        return self.world

    @property
    def _mjcf_path(self) -> Optional[str]:
        return self.mjcf_path

    # ---- sizes ------------------------------------------------------------------------------
    @property
    def num_envs(self) -> int:
        return self.world.num_envs

    @property
    def observation_dim(self) -> int:
        return self.world.obs_dim

    @property
    def action_dim(self) -> int:
        return self.world.action_dim

    @property
    def observation_shape(self) -> Tuple[int, int]:
        return (self.world.num_envs, self.world.obs_dim)

    @property
    def action_shape(self) -> Tuple[int, int]:
        return (self.world.num_envs, self.world.action_dim)

    @property
    def timestep(self) -> float:
        return self.world.timestep

    # ---- episode ------------------------------------------------------------------------------
    def reset(self, mask: Optional[np.ndarray] = None) -> np.ndarray:
        """Restores the envs selected by `mask` (every env when None) to the scene's initial
        state and returns the observations, shape (num_envs, obs_dim)."""
        self.world.reset(mask)
        self.steps_since_reset = 0
        return self.world.get_observations(zero_copy=False)

    def step(self, actions: np.ndarray, substeps: int = 0) -> Tuple[np.ndarray, np.ndarray, np.ndarray, Dict[str, Any]]:
        """One step of every env. `actions` has num_envs * action_dim values, flat or shaped
        (num_envs, action_dim); substeps 0 keeps the configured count."""
        self.world.step(np.asarray(actions, dtype=np.float32).reshape(self.action_shape), substeps)
        self.steps_since_reset += 1
        at_limit = self.steps_since_reset >= self.max_episode_steps
        info = {"step_count": self.steps_since_reset, "truncated": np.full(self.num_envs, at_limit, dtype=bool)}
        observations = self.world.get_observations(zero_copy=False)
        return observations, self.world.get_rewards(), self.world.get_dones().astype(bool), info

    # ---- state for viewers --------------------------------------------------------------------
    def get_body_positions(self) -> np.ndarray:
        """Body positions (num_envs, num_bodies, 4): a view that follows the simulation."""
        return self.world.get_body_positions()

    def get_body_quaternions(self) -> np.ndarray:
        """Body orientations (num_envs, num_bodies, 4), xyzw: a view that follows the simulation."""
        return self.world.get_body_quaternions()

    # ---- lifetime -------------------------------------------------------------------------------
    def close(self) -> None:
        self.world.close()

    def __enter__(self) -> "ZenoEnv":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def make(model: str, num_envs: int = 1, **kwargs) -> ZenoEnv:
    """A ZenoEnv for a model name ("ant", "humanoid.xml") or an MJCF path; other keyword
    arguments go to ZenoEnv."""
    return ZenoEnv(mjcf_path=str(find_model(model)), num_envs=num_envs, **kwargs)
