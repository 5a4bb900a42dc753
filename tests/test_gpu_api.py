"""World API behaviour on the GPU, through the C ABI: the reference's Python integration
suite (tests/test_python_integration.py) restated for zeno_amd.ZenoWorld, with every state
comparison made against the CPU oracle on the same inputs (bit-exact discrete outputs,
fp32 within 1e-5 rel / 1e-6 abs)."""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import OracleWorld
from tests.parity import compare, gpu_arrays, live_mask, make_pair, oracle_arrays
from zeno_amd.model import load_model
from zeno_amd.scenes import ASSETS
from zeno_amd.world import ZenoWorld

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-6)

# The reference suite's minimal pendulum (test_python_integration.py:26-52).
PENDULUM_MJCF = """<mujoco model="test_pendulum">
    <option timestep="0.02" gravity="0 0 -9.81"/>
    <worldbody>
        <geom type="plane" size="5 5 0.1"/>
        <body name="base" pos="0 0 1.5">
            <geom type="sphere" size="0.05" mass="0"/>
            <body name="pole" pos="0 0 0">
                <joint name="hinge" type="hinge" axis="0 1 0" damping="0.1"/>
                <geom type="capsule" fromto="0 0 0 0 0 -1" size="0.02" mass="1"/>
                <body name="bob" pos="0 0 -1"><geom type="sphere" size="0.1" mass="1"/></body>
            </body>
        </body>
    </worldbody>
    <actuator><motor joint="hinge" ctrlrange="-5 5" gear="1"/></actuator>
    <sensor><jointpos joint="hinge"/><jointvel joint="hinge"/></sensor>
</mujoco>"""


def pair_from_string(xml, num_envs, **kw):
    g = ZenoWorld(mjcf_string=xml, num_envs=num_envs, **kw)
    o = OracleWorld(load_model(mjcf_string=xml), num_envs,
                    max_contacts_per_env=kw.get("max_contacts_per_env", 64),
                    substeps=kw.get("substeps", 1), contact_iterations=kw.get("contact_iterations", 4))
    return g, o


def test_create_and_metadata():
    with ZenoWorld(mjcf_string=PENDULUM_MJCF, num_envs=4) as w:
        info = w.get_info()
        assert info["num_envs"] == 4 and info["num_bodies"] == 4 and info["num_joints"] == 3
        assert info["action_dim"] == 1 and info["obs_dim"] == 2
        assert info["timestep"] == pytest.approx(0.02)
        assert info["metal_available"] is False
        assert info["memory_usage"] > 0 and info["gpu_memory_usage"] >= info["memory_usage"]
        assert w.max_contacts_per_env == 64


def test_create_requires_mjcf():
    with pytest.raises(ValueError):
        ZenoWorld(num_envs=1)


def test_shapes_dtypes_and_zero_outputs():
    E = 8
    with ZenoWorld(mjcf_path=str(ASSETS / "ant.xml"), num_envs=E) as w:
        w.step(np.zeros((E, w.action_dim), np.float32))
        B, J = w.num_bodies, w.num_joints
        assert w.get_observations().shape == (E, w.obs_dim) and w.get_observations().dtype == np.float32
        for fn in (w.get_body_positions, w.get_body_quaternions, w.get_body_velocities,
                   w.get_body_angular_velocities, w.get_body_accelerations):
            a = fn()
            assert a.shape == (E, B, 4) and a.dtype == np.float32
        for fn in (w.get_joint_positions, w.get_joint_velocities, w.get_joint_forces):
            assert fn().shape == (E, J)
        assert w.get_sensor_data().shape == (E, w.obs_dim)
        assert w.get_contacts().shape == (E, 64) and w.get_contacts().itemsize == 64
        assert w.get_contact_counts().shape == (E,) and w.get_contact_counts().dtype == np.uint32
        # Rewards and dones have no writer in the step: they stay 0.
        assert w.get_rewards().shape == (E,) and not w.get_rewards().any()
        assert w.get_dones().shape == (E,) and w.get_dones().dtype == np.uint8 and not w.get_dones().any()


def test_zero_copy_views():
    """test_python_integration.py:165-230: the same host address on every call, a copy
    otherwise, and the view follows the simulation."""
    with ZenoWorld(mjcf_string=PENDULUM_MJCF, num_envs=2) as w:
        p1, p2 = w.get_body_positions(), w.get_body_positions()
        assert p1.ctypes.data == p2.ctypes.data
        pc = w.get_body_positions(zero_copy=False)
        assert pc.ctypes.data != p1.ctypes.data
        np.testing.assert_array_equal(p1, pc)
        o1, o2 = w.get_observations(), w.get_observations()
        assert o1.ctypes.data != o2.ctypes.data  # observations copy by default
        snap = p1.copy()
        for _ in range(5):
            w.step(np.ones((2, 1), np.float32))
        # no getter call in between: the held view shows the stepped state
        assert not np.array_equal(p1, snap)
        raw = w._lib.zeno_world_get_body_positions(w.handle)
        assert C.addressof(raw.contents) == p1.ctypes.data


def test_reused_views_are_separate_arrays_and_copies_do_not_alias():
    """The getters build one ndarray per host mirror and hand out views of it: each zero-copy
    call is its own array object over the mirror, each copy is fresh memory that later steps do
    not change, and closing the world drops the arrays."""
    with ZenoWorld(mjcf_string=PENDULUM_MJCF, num_envs=2) as w:
        v1, v2 = w.get_body_positions(), w.get_body_positions()
        assert v1 is not v2 and v1.ctypes.data == v2.ctypes.data
        v1.shape = (-1,)  # reshaping one handed-out view leaves the next one alone
        assert w.get_body_positions().shape == (2, w.num_bodies, 4)
        o1 = w.get_observations()
        r1, d1 = w.get_rewards(), w.get_dones()
        for _ in range(3):
            w.step(np.ones((2, 1), np.float32))
        o2 = w.get_observations()
        assert not np.shares_memory(o1, o2) and not np.array_equal(o1, o2)
        np.testing.assert_array_equal(o2, w.get_sensor_data())
        assert not np.shares_memory(r1, w.get_rewards()) and not np.shares_memory(d1, w.get_dones())
        assert w._views
    assert not w._views


def test_held_views_follow_every_state_change():
    """Views taken once stay current across step, step_subset, reset, reset_to_state and the
    setters (the reference's shared-memory buffers do), and match the oracle after steps."""
    E = 6
    g, o, acts = make_pair("ant", E, 6, seed=5)
    views = {"positions": g.get_body_positions(), "quaternions": g.get_body_quaternions(),
             "velocities": g.get_body_velocities(), "angular_velocities": g.get_body_angular_velocities(),
             "joint_positions": g.get_joint_positions(), "observations": g.get_sensor_data()}
    con = g.get_contacts()
    for k in range(4):
        g.step(acts[k])
        o.step(acts[k])
    for name, v in views.items():
        np.testing.assert_array_equal(v, getattr(o, name)[:, : v.shape[1]] if v.ndim == 2 else getattr(o, name), name)
    live = live_mask(o.contact_counts, g.max_contacts_per_env)
    np.testing.assert_array_equal(con["indices"][live], o.contacts["indices"][live])
    np.testing.assert_array_equal(con["position_pen"][live], o.contacts["position_pen"][live])
    mask = np.zeros(E, np.uint8)
    mask[::2] = 1
    g.step_subset(acts[4], mask)
    o.step_subset(acts[4], mask)
    np.testing.assert_array_equal(views["positions"], o.positions)
    np.testing.assert_array_equal(views["observations"], o.observations)
    g.reset(mask)
    o.reset(mask)
    np.testing.assert_array_equal(views["positions"], o.positions)
    np.testing.assert_array_equal(views["joint_positions"], o.joint_positions[:, : g.num_joints])
    p = o.positions.copy()
    p[:, 1, 2] += 0.25
    g.set_body_positions(p)
    np.testing.assert_array_equal(views["positions"], p)
    q = o.quaternions.copy()
    g.reset_to_state(p, q, np.zeros_like(p), np.zeros_like(p))
    np.testing.assert_array_equal(views["velocities"], 0.0)


def test_step_subset_matches_reference_semantics():
    """World.stepSubset (world.zig:833-929): masked-out envs keep bodies, joints, obs,
    accelerations, counts and contacts; their lambdas and prev-contact cache advance."""
    g, o, acts = make_pair("ant", 12, 12, seed=21)
    rng = np.random.default_rng(4)
    for k in range(12):
        if k % 3 == 2:
            g.step(acts[k]); o.step(acts[k])
            continue
        mask = (rng.random(12) < 0.5).astype(np.uint8)
        mask[k % 12] = 1
        mask[(k + 5) % 12] = 0
        g.step_subset(acts[k], mask)
        o.step_subset(acts[k], mask)
        compare(gpu_arrays(g), oracle_arrays(o), **TOL)


def test_step_subset_edge_masks():
    g, o, acts = make_pair("cartpole", 6, 3, seed=2)
    before = gpu_arrays(g)
    g.step_subset(acts[0], np.zeros(6, np.uint8))  # no active env: a no-op
    compare(gpu_arrays(g), before, rtol=0, atol=0)
    g.step_subset(acts[1], np.ones(6, np.uint8))  # all active: a plain step
    o.step(acts[1])
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    with pytest.raises(ValueError):
        g.step_subset(acts[2], np.ones(5, np.uint8))


def test_selective_reset_and_counts():
    """World.reset (world.zig:1296-1314): selected envs return to the scene pose with zero
    joint state; every env's contact count is zeroed; prev contacts and lambdas are kept."""
    g, o, acts = make_pair("ant", 8, 6, seed=9)
    for k in range(4):
        g.step(acts[k]); o.step(acts[k])
    mask = np.array([1, 0, 0, 1, 0, 1, 1, 0], np.uint8)
    before = g.get_body_positions(zero_copy=False)
    g.reset(mask); o.reset(mask)
    after = g.get_body_positions(zero_copy=False)
    assert not g.get_contact_counts().any()
    assert g.get_prev_contact_counts().any()
    for i in range(8):
        if mask[i]:
            assert not np.array_equal(before[i], after[i])
        else:
            np.testing.assert_array_equal(before[i], after[i])
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    for k in range(4, 6):
        g.step(acts[k]); o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    g.reset(); o.reset()
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)


def test_reset_to_state_masked_and_optional_velocities():
    g, o, acts = make_pair("humanoid", 6, 4, seed=17)
    for k in range(2):
        g.step(acts[k]); o.step(acts[k])
    rng = np.random.default_rng(1)
    p = g.get_body_positions(zero_copy=False) + rng.normal(0, 0.01, (6, g.num_bodies, 4)).astype(np.float32)
    q = g.get_body_quaternions(zero_copy=False)
    mask = np.array([0, 1, 1, 0, 1, 0], np.uint8)
    g.reset_to_state(p, q, mask=mask)
    o.reset_to_state(p, q, mask=mask)
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    for k in range(2, 4):
        g.step(acts[k]); o.step(acts[k])
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)


def test_setters_gravity_timestep():
    g, o = pair_from_string(PENDULUM_MJCF, 4)
    rng = np.random.default_rng(0)
    v = rng.normal(0, 0.3, (4, 4, 4)).astype(np.float32)
    mask = np.array([1, 0, 1, 1], np.uint8)
    g.set_body_velocities(v, mask); o.set_body_velocities(v, mask)
    p = g.get_body_positions(zero_copy=False) + np.float32(0.01)
    g.set_body_positions(p); o.set_body_positions(p)
    g.set_gravity((0.0, 0.5, -3.0)); o.gravity = [0.0, 0.5, -3.0]
    g.set_timestep(0.005); o.timestep = 0.005
    assert g.timestep == pytest.approx(0.005)
    a = rng.uniform(-1, 1, (6, 4, 1)).astype(np.float32)
    for k in range(6):
        g.step(a[k]); o.step(a[k])
        compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    for bad in (0.0, -1.0):
        with pytest.raises(RuntimeError):
            g.set_timestep(bad)
    assert g.timestep == pytest.approx(0.005)


def test_zero_gravity_pendulum_stays_put():
    """test_python_integration.py:755-775 and the oracle's closed form: no gravity and no
    action -> no vertical motion."""
    with ZenoWorld(mjcf_string=PENDULUM_MJCF, num_envs=1) as w:
        w.set_gravity((0.0, 0.0, 0.0))
        p0 = w.get_body_positions(zero_copy=False)
        for _ in range(50):
            w.step(np.zeros((1, 1), np.float32))
        assert np.all(np.abs(w.get_body_positions(zero_copy=False)[0, :, 2] - p0[0, :, 2]) < 1e-4)


@pytest.mark.parametrize("value", [1e6, -1e6, np.nan, 0.0])
def test_extreme_actions_match_oracle(value):
    g, o = pair_from_string(PENDULUM_MJCF, 2)
    a = np.full((2, 1), value, np.float32)
    for _ in range(3 if value != 0 else 50):
        g.step(a); o.step(a)
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    assert np.all(np.isfinite(g.get_observations()))


def test_action_dtype_coercion():
    g, o = pair_from_string(PENDULUM_MJCF, 3)
    a64 = np.linspace(-1, 1, 3).reshape(3, 1)
    g.step(a64)
    g.step(list(a64.reshape(-1)))
    o.step(a64.astype(np.float32)); o.step(a64.astype(np.float32))
    assert g.get_observations().dtype == np.float32
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    with pytest.raises(ValueError):
        g.step(np.zeros(2, np.float32))


def test_state_roundtrip():
    """test_python_integration.py:711-745"""
    with ZenoWorld(mjcf_string=PENDULUM_MJCF, num_envs=2) as w:
        a = np.full((2, 1), 0.5, np.float32)
        for _ in range(20):
            w.step(a)
        state = w.get_state()
        for _ in range(20):
            w.step(a)
        assert not np.array_equal(w.get_body_positions(zero_copy=False), state["body_positions"])
        w.set_state(state)
        np.testing.assert_array_equal(w.get_body_positions(zero_copy=False), state["body_positions"])
        np.testing.assert_array_equal(w.get_body_velocities(zero_copy=False), state["body_velocities"])


def test_profiling():
    with ZenoWorld(mjcf_string=PENDULUM_MJCF, num_envs=1, enable_profiling=True) as w:
        w.step(np.zeros((1, 1), np.float32))
        d = w.get_profiling_data()
        assert set(d) >= {"integrate_ms", "collision_broad_ms", "collision_narrow_ms",
                          "constraint_solve_ms", "total_step_ms", "num_contacts", "num_active_constraints"}
        assert d["total_step_ms"] > 0
        assert d["num_active_constraints"] == 4
        w.reset_profiling()
        assert w.get_profiling_data()["total_step_ms"] == 0


@pytest.mark.parametrize("asset", ["ant", "cartpole", "cheetah", "hopper", "humanoid", "pendulum",
                                   "pusher", "reacher", "swimmer", "walker"])
def test_every_asset_matches_oracle(asset):
    """test_python_integration.py:666-688 runs each shipped model for 10 steps; here the
    10 steps are also held to the oracle."""
    path = str(ASSETS / f"{asset}.xml")
    g = ZenoWorld(mjcf_path=path, num_envs=3)
    o = OracleWorld(load_model(path), 3)
    rng = np.random.default_rng(len(asset))
    for _ in range(10):
        a = rng.uniform(-1, 1, (3, g.action_dim)).astype(np.float32)
        g.step(a); o.step(a)
    compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    assert np.all(np.isfinite(g.get_observations()))
    g.close()


def test_deterministic_replay():
    """Two worlds fed the same inputs produce bitwise identical state (no atomics or
    unordered reductions on the step path)."""
    outs = []
    for _ in range(2):
        g, _o, acts = make_pair("ant", 256, 20, seed=31)
        for k in range(20):
            g.step(acts[k])
        outs.append(gpu_arrays(g))
        g.close()
    compare(outs[0], outs[1], rtol=0, atol=0)
    np.testing.assert_array_equal(outs[0]["contacts"].view(np.uint8), outs[1]["contacts"].view(np.uint8))


def test_device_resident_loop_matches_host_loop():
    """zeno_amd_world_step_device takes actions already in device memory; the result is the
    same as the host-action step."""
    g1, _o, acts = make_pair("ant", 32, 5, seed=41)
    g2, _o2, _ = make_pair("ant", 32, 5, seed=41)
    hip = C.CDLL("libamdhip64.so")
    flat = np.ascontiguousarray(acts, np.float32)
    dptr = C.c_void_p()
    assert hip.hipMalloc(C.byref(dptr), C.c_size_t(flat.nbytes)) == 0
    try:
        assert hip.hipMemcpy(dptr, C.c_void_p(flat.ctypes.data), C.c_size_t(flat.nbytes), 1) == 0
        stride = acts[0].nbytes
        for k in range(5):
            g1.step(acts[k])
            rc = g2._lib.zeno_amd_world_step_device(g2.handle, C.c_void_p(dptr.value + k * stride), 0)
            assert rc == 0
        g2.synchronize()
        compare(gpu_arrays(g1), gpu_arrays(g2), rtol=0, atol=0)
    finally:
        hip.hipFree(dptr)


def test_worlds_side_by_side_stay_independent():
    """Several worlds in one process (a training and an evaluation batch, say): Ant, the
    pendulum and the pile stepped in turn, with the first world's observation view held (its
    steps are synchronous, the others' are not), each against its own oracle; the pendulum is
    closed halfway and the other two go on."""
    worlds = [make_pair("ant", 48, 12, seed=51), make_pair("pendulum", 20, 12, seed=52), make_pair("pile", 6, 12, seed=53)]
    held = worlds[0][0].get_observations(zero_copy=True)
    for k in range(12):
        for i, (g, o, acts) in enumerate(worlds):
            if g is None:
                continue
            g.step(acts[k])
            o.step(acts[k] if o.A else None)
        np.testing.assert_array_equal(held, worlds[0][1].observations[:, : worlds[0][1].model["obs_dim"]])
        for g, o, _ in worlds:
            if g is not None:
                compare(gpu_arrays(g), oracle_arrays(o), **TOL)
        if k == 5:
            worlds[1][0].close()
            worlds[1] = (None, None, None)
    for g, _, _ in worlds:
        if g is not None:
            g.close()


@pytest.mark.parametrize("xml", [
    '<mujoco><worldbody><geom type="plane" size="5 5 0.1"/></worldbody></mujoco>',
    '<mujoco><worldbody><body name="b" pos="0 0 1"><joint type="free"/><geom type="sphere" size="0.1"/></body>'
    '</worldbody></mujoco>',
    '<mujoco><worldbody><geom type="plane" size="5 5 0.1"/><body name="b" pos="0 0 0.05"><joint type="free"/>'
    '<geom type="sphere" size="0.1"/></body></worldbody></mujoco>'], ids=["world_only", "free_body", "resting_body"])
def test_smallest_scenes_match_oracle(xml):
    """Scenes at the small end: the world body alone (a plane, nothing to move, no pair), one
    free body with no geom to meet, and one free body resting in the plane; 5 envs, each step
    against the oracle."""
    g, o = pair_from_string(xml, 5)
    for _ in range(6):
        g.step(np.zeros((5, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    g.close()
