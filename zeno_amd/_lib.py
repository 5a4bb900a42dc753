"""ctypes bindings for libzeno.so (the C ABI in include/zeno.h and include/zeno_amd_ext.h).

The reference loads its library with cffi (python/zeno/_ffi.py:41-345); cffi is not part of
this environment, so the same declarations are expressed with ctypes. Loading fails loudly:
there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("ZENO_AMD_LIB", _PKG / "libzeno.so"))


class ZenoConfig(C.Structure):
    """main.zig:75-86"""

    _fields_ = [
        ("num_envs", C.c_uint32),
        ("timestep", C.c_float),
        ("contact_iterations", C.c_uint32),
        ("max_contacts_per_env", C.c_uint32),
        ("seed", C.c_uint64),
        ("substeps", C.c_uint32),
        ("enable_profiling", C.c_bool),
        ("max_bodies_per_env", C.c_uint32),
        ("max_joints_per_env", C.c_uint32),
        ("max_geoms_per_env", C.c_uint32),
    ]


class ZenoInfo(C.Structure):
    """main.zig:89-102"""

    _fields_ = [
        ("num_envs", C.c_uint32),
        ("num_bodies", C.c_uint32),
        ("num_joints", C.c_uint32),
        ("num_actuators", C.c_uint32),
        ("num_sensors", C.c_uint32),
        ("num_geoms", C.c_uint32),
        ("obs_dim", C.c_uint32),
        ("action_dim", C.c_uint32),
        ("timestep", C.c_float),
        ("memory_usage", C.c_uint64),
        ("gpu_memory_usage", C.c_uint64),
        ("metal_available", C.c_bool),
    ]


class ZenoProfilingData(C.Structure):
    """main.zig:105-113"""

    _fields_ = [
        ("integrate_ns", C.c_float),
        ("collision_broad_ns", C.c_float),
        ("collision_narrow_ns", C.c_float),
        ("constraint_solve_ns", C.c_float),
        ("total_step_ns", C.c_float),
        ("num_contacts", C.c_uint32),
        ("num_active_constraints", C.c_uint32),
    ]


class ZenoAmdModelView(C.Structure):
    """include/zeno_amd_ext.h"""

    _fields_ = [
        ("num_bodies", C.c_uint32), ("num_joints", C.c_uint32), ("num_geoms", C.c_uint32),
        ("num_actuators", C.c_uint32), ("num_sensors", C.c_uint32), ("obs_dim", C.c_uint32),
        ("num_constraints", C.c_uint32), ("num_colors", C.c_uint32), ("max_color_size", C.c_uint32),
        ("num_pairs", C.c_uint32),
        ("timestep", C.c_float), ("gravity", C.c_float * 3),
        ("friction", C.c_float), ("restitution", C.c_float), ("baumgarte", C.c_float), ("slop", C.c_float),
        ("bodies", C.c_void_p), ("joints", C.c_void_p), ("geoms", C.c_void_p), ("actuators", C.c_void_p),
        ("sensors", C.c_void_p), ("constraints", C.c_void_p),
        ("color_ranges", C.POINTER(C.c_uint32)), ("pairs", C.POINTER(C.c_uint32)),
        ("joint_limited", C.POINTER(C.c_uint8)),
        ("init_positions", C.POINTER(C.c_float)), ("init_quaternions", C.POINTER(C.c_float)),
        ("init_velocities", C.POINTER(C.c_float)), ("init_angular_velocities", C.POINTER(C.c_float)),
        ("inv_mass_inertia", C.POINTER(C.c_float)),
    ]


_vp = C.c_void_p
_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_u32p = C.POINTER(C.c_uint32)

# name: (restype, argtypes)
SIGNATURES = {
    # zeno.h — the reference ABI
    "zeno_world_create": (_vp, [C.c_char_p, C.POINTER(ZenoConfig)]),
    "zeno_world_create_from_string": (_vp, [C.c_char_p, C.POINTER(ZenoConfig)]),
    "zeno_world_destroy": (None, [_vp]),
    "zeno_world_step": (C.c_int, [_vp, _fp, C.c_uint32]),
    "zeno_world_step_subset": (C.c_int, [_vp, _fp, _u8p, C.c_uint32]),
    "zeno_world_reset": (C.c_int, [_vp, _u8p]),
    "zeno_world_reset_to_state": (C.c_int, [_vp, _fp, _fp, _fp, _fp, _u8p]),
    "zeno_world_get_observations": (_fp, [_vp]),
    "zeno_world_get_rewards": (_fp, [_vp]),
    "zeno_world_get_dones": (_u8p, [_vp]),
    "zeno_world_get_body_positions": (_fp, [_vp]),
    "zeno_world_get_body_quaternions": (_fp, [_vp]),
    "zeno_world_get_body_velocities": (_fp, [_vp]),
    "zeno_world_get_body_angular_velocities": (_fp, [_vp]),
    "zeno_world_get_body_accelerations": (_fp, [_vp]),
    "zeno_world_get_joint_positions": (_fp, [_vp]),
    "zeno_world_get_joint_velocities": (_fp, [_vp]),
    "zeno_world_get_joint_forces": (_fp, [_vp]),
    "zeno_world_get_contacts": (_vp, [_vp]),
    "zeno_world_get_contact_counts": (_u32p, [_vp]),
    "zeno_world_get_sensor_data": (_fp, [_vp]),
    "zeno_world_set_body_positions": (C.c_int, [_vp, _fp, _u8p]),
    "zeno_world_set_body_velocities": (C.c_int, [_vp, _fp, _u8p]),
    "zeno_world_set_gravity": (C.c_int, [_vp, C.c_float, C.c_float, C.c_float]),
    "zeno_world_set_timestep": (C.c_int, [_vp, C.c_float]),
    "zeno_world_num_envs": (C.c_uint32, [_vp]),
    "zeno_world_num_bodies": (C.c_uint32, [_vp]),
    "zeno_world_num_joints": (C.c_uint32, [_vp]),
    "zeno_world_num_sensors": (C.c_uint32, [_vp]),
    "zeno_world_obs_dim": (C.c_uint32, [_vp]),
    "zeno_world_action_dim": (C.c_uint32, [_vp]),
    "zeno_world_get_info": (C.c_int, [_vp, C.POINTER(ZenoInfo)]),
    "zeno_world_get_profiling": (C.c_int, [_vp, C.POINTER(ZenoProfilingData)]),
    "zeno_world_reset_profiling": (None, [_vp]),
    "zeno_version": (C.c_char_p, []),
    "zeno_metal_available": (C.c_bool, []),
    "zeno_error_string": (C.c_char_p, [C.c_int]),
    "zeno_world_memory_usage": (C.c_uint64, [_vp]),
    "zeno_world_compact_memory": (None, [_vp]),
    "zeno_world_max_contacts_per_env": (C.c_uint32, [_vp]),
    "zeno_swarm_create": (_vp, [_vp, _vp]),
    "zeno_swarm_destroy": (None, [_vp]),
    "zeno_swarm_step": (C.c_int, [_vp, _vp, _fp]),
    "zeno_swarm_get_metrics": (C.c_int, [_vp, _vp]),
    "zeno_swarm_get_agent_states": (_vp, [_vp]),
    "zeno_swarm_get_neighbor_counts": (C.c_int, [_vp, _u32p, C.c_uint32]),
    "zeno_swarm_set_body_offset": (None, [_vp, C.c_uint32]),
    "zeno_swarm_evaluate_task": (C.c_int, [_vp, _vp, C.c_uint32, _fp, _vp]),
    "zeno_swarm_apply_attack": (C.c_int, [_vp, _vp]),
    "zeno_swarm_get_neighbor_index_ptr": (_u32p, [_vp]),
    "zeno_swarm_get_neighbor_row_ptr": (_u32p, [_vp]),
    "zeno_swarm_start_recording": (C.c_int, [_vp]),
    "zeno_swarm_stop_recording": (C.c_int, [_vp]),
    "zeno_swarm_get_replay_stats": (C.c_int, [_vp, _vp]),
    # zeno_amd_ext.h — extensions
    "zeno_amd_model_create": (_vp, [C.c_char_p]),
    "zeno_amd_model_create_from_string": (_vp, [C.c_char_p]),
    "zeno_amd_model_destroy": (None, [_vp]),
    "zeno_amd_model_view": (C.c_int, [_vp, C.POINTER(ZenoAmdModelView)]),
    "zeno_amd_world_model_view": (C.c_int, [_vp, C.POINTER(ZenoAmdModelView)]),
    "zeno_amd_last_error": (C.c_char_p, []),
    "zeno_amd_device_count": (C.c_int, []),
    "zeno_amd_world_get_lambda": (C.c_int, [_vp, _fp]),
    "zeno_amd_world_get_prev_contact_counts": (C.c_int, [_vp, _u32p]),
    "zeno_amd_world_set_contact_counts": (C.c_int, [_vp, _u32p]),
    "zeno_amd_world_step_device": (C.c_int, [_vp, C.c_void_p, C.c_uint32]),
    "zeno_amd_world_synchronize": (C.c_int, [_vp]),
    "zeno_amd_world_set_kernel_timing": (C.c_int, [_vp, C.c_int]),
    "zeno_amd_world_get_kernel_timing": (C.c_int, [_vp, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "zeno_amd_world_joint_phases": (C.c_uint32, [C.c_void_p]),
    "zeno_amd_world_launch_config": (C.c_int, [_vp, _u32p, _u32p]),
    "zeno_amd_world_modes": (C.c_int, [_vp, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "zeno_amd_world_get_cell_ids": (C.c_int, [_vp, _u32p]),
    "zeno_amd_world_set_extended_contacts": (C.c_int, [_vp, C.c_int]),
    "zeno_amd_world_capture_steps": (C.c_int, [_vp, _vp, C.c_uint64, C.c_uint32, C.c_uint32]),
    "zeno_amd_world_graph_launch": (C.c_int, [_vp]),
    "zeno_amd_world_release_graph": (C.c_int, [_vp]),
    "zeno_amd_detect_collisions": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p]),
    "zeno_amd_detect_collisions_host": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p]),
    "zeno_amd_detect_collisions_host_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p]),
    "zeno_amd_selfcheck_divide": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]),
    "zeno_amd_selfcheck_sqrt": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32]),
    "zeno_amd_selfcheck_reciprocal_error": (C.c_int, [C.c_void_p]),
    "zeno_amd_world_waves_per_group": (C.c_uint32, [C.c_void_p]),
    "zeno_amd_world_split_groups": (C.c_int, [C.c_void_p]),
}

_lib = None


def load() -> C.CDLL:
    """Loads libzeno.so and declares every entry point. Raises if the library is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"libzeno.so not found at {LIB_PATH}; build it with `python -m zeno_amd.build` "
            "(there is no CPU fallback)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().zeno_amd_last_error().decode()
