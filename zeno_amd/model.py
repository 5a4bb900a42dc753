"""Host-side model inspection: the records a world's kernels read, as numpy arrays.

Backed by the zeno_amd_model_* extension entry points, which parse MJCF and build the
model without touching a GPU (include/zeno_amd_ext.h).
"""
from __future__ import annotations

import ctypes as C
from typing import Any, Dict

import numpy as np

from . import _lib as L

BODY_DTYPE = np.dtype([("position", "4f4"), ("quaternion", "4f4"), ("inv_mass_inertia", "4f4"),
                       ("params", "4f4"), ("com_offset", "4f4")])
JOINT_DTYPE = np.dtype([("anchor_parent", "4f4"), ("anchor_child", "4f4"), ("axis", "4f4"),
                        ("params", "4f4"), ("params2", "4f4")])
GEOM_DTYPE = np.dtype([("type_body", "4u4"), ("pos_size0", "4f4"), ("quat", "4f4"), ("params", "4f4")])
ACTUATOR_DTYPE = np.dtype([("params", "4f4"), ("params2", "4f4")])
SENSOR_DTYPE = np.dtype([("type_object", "4u4"), ("params", "4f4")])
CONSTRAINT_DTYPE = np.dtype([("indices", "4u4"), ("anchor_a", "4f4"), ("anchor_b", "4f4"),
                             ("axis_target", "4f4"), ("limits", "4f4"), ("state", "4f4")])


def _records(ptr, n: int, dtype: np.dtype) -> np.ndarray:
    if n == 0 or not ptr:
        return np.zeros(0, dtype=dtype)
    raw = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint8)), shape=(n * dtype.itemsize,))
    return raw.view(dtype).copy()


def _arr(ptr, n: int, dtype) -> np.ndarray:
    if n == 0 or not ptr:
        return np.zeros(0, dtype=dtype)
    return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)


def view_to_dict(v: L.ZenoAmdModelView) -> Dict[str, Any]:
    B, J = v.num_bodies, v.num_joints
    return {
        "num_bodies": B, "num_joints": J, "num_geoms": v.num_geoms, "num_actuators": v.num_actuators,
        "num_sensors": v.num_sensors, "obs_dim": v.obs_dim, "num_constraints": v.num_constraints,
        "num_colors": v.num_colors, "max_color_size": v.max_color_size, "num_pairs": v.num_pairs,
        "timestep": v.timestep, "gravity": list(v.gravity), "friction": v.friction,
        "restitution": v.restitution, "baumgarte": v.baumgarte, "slop": v.slop,
        "bodies": _records(v.bodies, B, BODY_DTYPE),
        "joints": _records(v.joints, J, JOINT_DTYPE),
        "geoms": _records(v.geoms, v.num_geoms, GEOM_DTYPE),
        "actuators": _records(v.actuators, v.num_actuators, ACTUATOR_DTYPE),
        "sensors": _records(v.sensors, v.num_sensors, SENSOR_DTYPE),
        "constraints": _records(v.constraints, v.num_constraints, CONSTRAINT_DTYPE),
        "color_ranges": _arr(v.color_ranges, 2 * v.num_colors, np.uint32).reshape(-1, 2),
        "pairs": _arr(v.pairs, v.num_pairs, np.uint32),
        "joint_limited": _arr(v.joint_limited, J, np.uint8),
        "init_positions": _arr(v.init_positions, 4 * B, np.float32).reshape(B, 4),
        "init_quaternions": _arr(v.init_quaternions, 4 * B, np.float32).reshape(B, 4),
        "init_velocities": _arr(v.init_velocities, 4 * B, np.float32).reshape(B, 4),
        "init_angular_velocities": _arr(v.init_angular_velocities, 4 * B, np.float32).reshape(B, 4),
        "inv_mass_inertia": _arr(v.inv_mass_inertia, 4 * B, np.float32).reshape(B, 4),
    }


def load_model(mjcf_path: str | None = None, mjcf_string: str | None = None) -> Dict[str, Any]:
    """Parses MJCF on the host and returns the model records (no GPU needed)."""
    lib = L.load()
    if mjcf_path is not None:
        h = lib.zeno_amd_model_create(str(mjcf_path).encode())
    elif mjcf_string is not None:
        h = lib.zeno_amd_model_create_from_string(mjcf_string.encode())
    else:
        raise ValueError("mjcf_path or mjcf_string required")
    if not h:
        raise RuntimeError(f"model creation failed: {L.last_error()}")
    try:
        v = L.ZenoAmdModelView()
        rc = lib.zeno_amd_model_view(h, C.byref(v))
        if rc != 0:
            raise RuntimeError(f"model view failed: {rc}")
        return view_to_dict(v)
    finally:
        lib.zeno_amd_model_destroy(h)
