"""The C-ABI library on the CPU: it loads, exports every function include/*.h declares, and
its host-only entry points (version, error strings, null handles, creation without a
device) behave like the reference's (src/main.zig:139-905). No compute call is made."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from zeno_amd import _lib
from zeno_amd.scenes import ASSETS

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(zeno_[a-z0-9_]+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_function_is_exported(lib):
    declared = declared_functions()
    assert len(declared) >= 60
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = declared - exported
    assert not missing, sorted(missing)
    assert declared == set(_lib.SIGNATURES), sorted(declared ^ set(_lib.SIGNATURES))


def test_library_does_not_link_the_oracle():
    out = subprocess.run(["ldd", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    assert "oracle" not in out
    assert "libamdhip64" in out


def test_struct_sizes():
    """The ABI structs keep the reference's C layouts (main.zig:75-113)."""
    assert C.sizeof(_lib.ZenoConfig) == 48
    assert C.sizeof(_lib.ZenoInfo) == 64
    assert C.sizeof(_lib.ZenoProfilingData) == 28
    assert _lib.ZenoConfig.seed.offset == 16 and _lib.ZenoConfig.enable_profiling.offset == 28
    assert _lib.ZenoInfo.memory_usage.offset == 40 and _lib.ZenoInfo.metal_available.offset == 56


def test_version_and_capabilities(lib):
    assert re.fullmatch(r"\d+\.\d+\.\d+", lib.zeno_version().decode())
    assert lib.zeno_metal_available() is False


def test_error_strings(lib):
    """main.zig:706-719"""
    expect = {0: "success", -1: "invalid handle", -2: "file not found", -3: "parse error",
              -4: "metal error", -5: "out of memory", -6: "invalid argument", -7: "not implemented",
              -99: "unknown error", 5: "unknown error"}
    for code, text in expect.items():
        assert lib.zeno_error_string(code).decode() == text


def test_null_handles(lib):
    """Every entry point taking a world handle rejects NULL: -1 for int results, NULL for
    pointers, 0 for counts (main.zig:228-905)."""
    null = None
    assert lib.zeno_world_step(null, None, 0) == -1
    assert lib.zeno_world_step_subset(null, None, None, 0) == -1
    assert lib.zeno_world_reset(null, None) == -1
    assert lib.zeno_world_reset_to_state(null, None, None, None, None, None) == -1
    assert lib.zeno_world_set_body_positions(null, None, None) == -1
    assert lib.zeno_world_set_body_velocities(null, None, None) == -1
    assert lib.zeno_world_set_gravity(null, 0.0, 0.0, -9.81) == -1
    assert lib.zeno_world_set_timestep(null, 0.01) == -1
    assert lib.zeno_world_get_info(null, None) == -1
    assert lib.zeno_world_get_profiling(null, None) == -1
    lib.zeno_world_reset_profiling(null)
    lib.zeno_world_destroy(null)
    lib.zeno_world_compact_memory(null)
    for getter in ["observations", "rewards", "dones", "body_positions", "body_quaternions",
                   "body_velocities", "body_angular_velocities", "body_accelerations",
                   "joint_positions", "joint_velocities", "joint_forces", "contacts",
                   "contact_counts", "sensor_data"]:
        assert not getattr(lib, f"zeno_world_get_{getter}")(null), getter
    for count in ["num_envs", "num_bodies", "num_joints", "num_sensors", "obs_dim", "action_dim",
                  "memory_usage", "max_contacts_per_env"]:
        assert getattr(lib, f"zeno_world_{count}")(null) == 0, count
    for ext in ["world_get_lambda", "world_get_prev_contact_counts", "world_synchronize",
                "world_set_kernel_timing", "world_model_view", "world_launch_config", "world_modes",
                "world_get_cell_ids", "world_set_extended_contacts", "world_capture_steps",
                "world_graph_launch", "world_release_graph"]:
        fn = getattr(lib, f"zeno_amd_{ext}")
        args = [None] * len(fn.argtypes)
        if ext in ("world_set_kernel_timing", "world_set_extended_contacts"):
            args[1] = 1
        if ext == "world_capture_steps":
            args[2:] = [0, 1, 0]
        assert fn(*args) == -1, ext
    assert lib.zeno_amd_world_step_device(None, None, 0) == -1
    assert lib.zeno_amd_world_get_kernel_timing(None, None, None) == -1


def test_swarm_is_not_part_of_this_build(lib):
    assert not lib.zeno_swarm_create(None, None)
    assert lib.zeno_swarm_step(None, None, None) == -7
    assert lib.zeno_swarm_get_metrics(None, None) == -7
    assert not lib.zeno_swarm_get_agent_states(None)


def test_create_failures_are_reported(lib):
    cfg = _lib.ZenoConfig(num_envs=4)
    assert not lib.zeno_world_create(b"/nonexistent/ant.xml", C.byref(cfg))
    assert "nonexistent" in _lib.last_error() or "not found" in _lib.last_error().lower()
    assert not lib.zeno_world_create(str(ASSETS / "ant.xml").encode(), None)
    assert not lib.zeno_world_create(None, C.byref(cfg))


@pytest.mark.skipif(_lib.load().zeno_amd_device_count() > 0, reason="a HIP device is present")
def test_create_without_device_fails_loudly(lib):
    """No CPU fallback: with no HIP device the world cannot be created."""
    cfg = _lib.ZenoConfig(num_envs=4)
    assert not lib.zeno_world_create(str(ASSETS / "ant.xml").encode(), C.byref(cfg))
    assert "device" in _lib.last_error().lower()


def test_model_create_host_only(lib):
    """The host-side model (parse + decomposition + colouring) needs no device."""
    h = lib.zeno_amd_model_create(str(ASSETS / "ant.xml").encode())
    assert h
    v = _lib.ZenoAmdModelView()
    assert lib.zeno_amd_model_view(h, C.byref(v)) == 0
    assert (v.num_bodies, v.num_joints, v.num_geoms, v.num_actuators, v.obs_dim) == (10, 9, 10, 8, 29)
    lib.zeno_amd_model_destroy(h)
    # The reference parser is lenient (parser.zig:1527-1529): an unparseable number keeps
    # the attribute's default, and an unclosed document still yields a model.
    h = lib.zeno_amd_model_create_from_string(b"<mujoco><worldbody><body><geom type='sphere' size='x'/></body>")
    assert h
    assert lib.zeno_amd_model_view(h, C.byref(v)) == 0
    assert (v.num_bodies, v.num_geoms) == (2, 1)
    lib.zeno_amd_model_destroy(h)
    assert not lib.zeno_amd_model_create(b"/nonexistent/model.xml")


def test_collision_abi_struct_layouts_and_null_arguments(lib):
    """ZenoAmdCollider / ZenoAmdContactResult are 64 B records; the oracle's records share
    the layout; null operands are rejected before any GPU work, and n = 0 is a no-op."""
    from oracle import oracle as O
    from zeno_amd import collision as Z

    assert Z.COLLIDER_DTYPE == O.COLLIDER_DTYPE and Z.CONTACT_RESULT_DTYPE == O.CONTACT_RESULT_DTYPE
    assert Z.COLLIDER_DTYPE.fields["quaternion"][1] == 48 and Z.CONTACT_RESULT_DTYPE.fields["valid"][1] == 28
    assert lib.zeno_amd_detect_collisions(None, None, 4, None, None) == -6
    assert lib.zeno_amd_detect_collisions_host(None, None, 4, None) == -6
    assert lib.zeno_amd_detect_collisions(None, None, 0, None, None) == 0
