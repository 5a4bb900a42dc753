"""Batched environment API over ZenoWorld, the counterpart of python/zeno/env.py.

ZenoEnv steps num_envs copies of one MJCF scene together (env.py:13-213) and make() finds a
model by path or by name (env.py:216-267). Names resolve against this package's assets
(the reference's ten MJCF files) before ./assets and ~/.zeno/assets.
"""
from __future__ import annotations

from pathlib import Path
from typing import Any, Dict, Optional, Tuple

import numpy as np

from .world import ZenoWorld

ASSET_DIRS = (
    Path(__file__).resolve().parent / "assets",
    Path.cwd() / "assets",
    Path.home() / ".zeno" / "assets",
)


def find_model(model: str) -> Path:
    """A path that exists, else `model` (".xml" appended when missing) in ASSET_DIRS."""
    path = Path(model)
    if path.exists():
        return path
    name = model if model.endswith(".xml") else f"{model}.xml"
    for d in ASSET_DIRS:
        if (d / name).exists():
            return d / name
    raise FileNotFoundError(f"Could not find model '{name}'. Searched: {[str(d) for d in ASSET_DIRS]}")


class ZenoEnv:
    """num_envs environments of one scene, stepped together on the GPU (env.py:13-213).

    step() returns (observations, rewards, dones, info): observations are a copy of shape
    (num_envs, obs_dim); rewards and dones are the world's buffers (zero: the step writes
    neither); info holds the step count and a truncation flag per env, set once
    max_episode_steps (1000) steps have run since the last reset.
    """

    def __init__(self, mjcf_path: Optional[str] = None, mjcf_string: Optional[str] = None, num_envs: int = 1,
                 timestep: float = 0, contact_iterations: int = 4, max_contacts_per_env: int = 64,
                 seed: int = 42, substeps: int = 1):
        self._world = ZenoWorld(mjcf_path=mjcf_path, mjcf_string=mjcf_string, num_envs=num_envs, timestep=timestep,
                                contact_iterations=contact_iterations, max_contacts_per_env=max_contacts_per_env,
                                seed=seed, substeps=substeps)
        self._num_envs = num_envs
        self._step_count = 0
        self._max_episode_steps = 1000
        self._mjcf_path = mjcf_path
        self._obs_shape = (num_envs, self._world.obs_dim)
        self._action_shape = (num_envs, self._world.action_dim)

    @property
    def num_envs(self) -> int:
        return self._num_envs

    @property
    def observation_dim(self) -> int:
        return self._world.obs_dim

    @property
    def action_dim(self) -> int:
        return self._world.action_dim

    @property
    def timestep(self) -> float:
        return self._world.timestep

    @property
    def observation_shape(self) -> Tuple[int, int]:
        return self._obs_shape

    @property
    def action_shape(self) -> Tuple[int, int]:
        return self._action_shape

    def reset(self, mask: Optional[np.ndarray] = None) -> np.ndarray:
        """Resets the selected envs (all when mask is None); returns a copy of the observations."""
        self._world.reset(mask)
        self._step_count = 0
        return self._world.get_observations().copy()

    def step(self, actions: np.ndarray, substeps: int = 0) -> Tuple[np.ndarray, np.ndarray, np.ndarray, Dict[str, Any]]:
        actions = np.asarray(actions, dtype=np.float32)
        if actions.shape != self._action_shape:
            actions = actions.reshape(self._action_shape)
        self._world.step(actions, substeps)
        self._step_count += 1
        observations = self._world.get_observations().copy()
        rewards = self._world.get_rewards()
        dones = self._world.get_dones()
        truncated = np.zeros(self._num_envs, dtype=bool)
        if self._step_count >= self._max_episode_steps:
            truncated[:] = True
        return observations, rewards, dones.astype(bool), {"step_count": self._step_count, "truncated": truncated}

    def get_body_positions(self) -> np.ndarray:
        return self._world.get_body_positions()

    def get_body_quaternions(self) -> np.ndarray:
        return self._world.get_body_quaternions()

    def close(self) -> None:
        self._world.close()

    def __enter__(self):
        return self

    def __exit__(self, *args):
        self.close()


def make(model: str, num_envs: int = 1, **kwargs) -> ZenoEnv:
    """ZenoEnv for a model name ("ant", "humanoid.xml") or an MJCF path (env.py:216-267)."""
    return ZenoEnv(mjcf_path=str(find_model(model)), num_envs=num_envs, **kwargs)
