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


def test_episode_clock_marks_and_collects_due_envs():
    from zeno_amd.gym import EpisodeClock
    c = EpisodeClock(4, limit=3)
    assert c.collect_due() is None
    term = np.array([False, True, False, False])
    assert not c.tick(term).any()
    due = c.collect_due()
    np.testing.assert_array_equal(due, term)
    np.testing.assert_array_equal(c.steps, [1, 0, 1, 1])
    none = np.zeros(4, bool)
    c.tick(none)
    trunc = c.tick(none)
    np.testing.assert_array_equal(trunc, [True, False, True, True])   # 3 steps since reset
    np.testing.assert_array_equal(c.collect_due(), [True, False, True, True])
    c.restart()
    assert not c.steps.any() and not c.due.any()


def _one_sphere_model(x, z, r):
    from zeno_amd.model import load_model
    return load_model(mjcf_string=f"""<mujoco><worldbody><geom type="plane" size="5 5 0.1"/>
    <body name="b" pos="{x} 0 {z}"><joint type="free"/><geom type="sphere" size="{r}" mass="1"/></body>
    <body name="c" pos="{x + 1} 0 {z}"><joint type="free"/><geom type="capsule" size="0.05 0.2" mass="1"/></body>
    </worldbody></mujoco>""")


def test_side_view_draws_geoms_where_they_are():
    """The frame fits the sphere (x 0, z 1) and the vertical capsule (x 1, z 1) with a margin;
    each shows its body's palette colour at its centre, the plane fills the rows below z = 0,
    the background is elsewhere."""
    from zeno_amd.gym import SideView
    m = _one_sphere_model(0.0, 1.0, 0.2)
    view = SideView(m, width=320, height=240)
    frame = view.draw(m["init_positions"], m["init_quaternions"])
    assert frame.shape == (240, 320, 3) and frame.dtype == np.uint8
    # bounds: x in [-0.2, 1.05], z in [0.75, 1.25] -> centre (0.425, 1.0), extent 1.25 * 1.3
    px = 240 / (1.25 * 1.3)
    col = lambda x: int(160 + (x - 0.425) * px)
    np.testing.assert_array_equal(frame[120, col(0.0)], SideView.PALETTE[1])
    np.testing.assert_array_equal(frame[120, col(1.0)], SideView.PALETTE[2])
    np.testing.assert_array_equal(frame[120, col(0.5)], SideView.BACKGROUND)
    np.testing.assert_array_equal(frame[0, 0], SideView.BACKGROUND)
    # ground: rows whose z is below 0 (z = 1 - (row + 0.5 - 120) / px)
    assert 1 - (239 + 0.5 - 120) / px > 0          # this frame does not reach z = 0
    low = _one_sphere_model(0.0, 0.3, 0.2)
    f2 = SideView(low, 320, 240).draw(low["init_positions"], low["init_quaternions"])
    np.testing.assert_array_equal(f2[-1, 0], SideView.GROUND)
    np.testing.assert_array_equal(f2[0, 0], SideView.BACKGROUND)


def test_side_view_skips_non_finite_bodies():
    from zeno_amd.gym import SideView
    m = _one_sphere_model(0.0, 1.0, 0.2)
    pos = m["init_positions"].copy()
    pos[1, :3] = np.nan
    frame = SideView(m, 64, 48).draw(pos, m["init_quaternions"])
    assert not np.any(np.all(frame == SideView.PALETTE[1], axis=-1))


def test_reference_attribute_names_on_zeno_env():
    """python/zeno/__init__.py:49 documents env._world.get_body_positions(zero_copy=True)."""
    from zeno_amd.env import ZenoEnv
    env = ZenoEnv.__new__(ZenoEnv)
    sentinel = object()
    env.world = sentinel
    env.mjcf_path = "ant.xml"
    assert env._world is sentinel and env._mjcf_path == "ant.xml"


def test_check_env_reports_a_broken_environment():
    from zeno_amd.gym import Box, check_env

    class Broken:
        observation_space = Box(-1.0, 1.0, (2,))
        action_space = Box(-1.0, 1.0, (1,))

        def reset(self):
            return np.full(2, 5.0, np.float32), {}

        def step(self, action):
            return np.zeros(2, np.float32), 0.0, False, False    # four values

    with pytest.warns(UserWarning) as rec:
        assert check_env(Broken()) is False
    text = " ".join(str(r.message) for r in rec)
    assert "outside" in text and "step()" in text
