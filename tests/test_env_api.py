"""The Python environment layer: CPU-side pieces (model lookup, the Box space) here; the
GPU behaviours of ZenoEnv / ZenoGymnasiumEnv / ZenoVectorEnv are in test_gpu_env.py."""
import numpy as np
import pytest

from zeno_amd.env import ASSET_DIRS, find_model
from zeno_amd.gym import ENV_CONFIGS, Box


def test_find_model_by_name_and_path(tmp_path):
    assert find_model("ant").name == "ant.xml"
    assert find_model("humanoid.xml") == ASSET_DIRS[0] / "humanoid.xml"
    p = tmp_path / "m.xml"
    p.write_text("<mujoco/>")
    assert find_model(str(p)) == p
    with pytest.raises(FileNotFoundError):
        find_model("no_such_model")


def test_env_configs_point_at_shipped_assets():
    for cfg in ENV_CONFIGS.values():
        assert (ASSET_DIRS[0] / cfg["mjcf_file"]).exists()


def test_box_space():
    b = Box(-1.0, 1.0, (3, 2), seed=0)
    for _ in range(20):
        x = b.sample()
        assert x.shape == (3, 2) and x.dtype == np.float32 and b.contains(x)
    assert not b.contains(np.full((3, 2), 2.0, np.float32))
    assert not b.contains(np.zeros(3, np.float32))
    u = Box(-np.inf, np.inf, (4,), seed=1)
    x = u.sample()
    assert x.shape == (4,) and np.all(np.isfinite(x)) and u.contains(x)
