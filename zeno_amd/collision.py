"""Extended narrow phase: the reference's narrow_phase.detectCollision on the GPU.

`Geom` and `Transform` mirror primitives.Geom (src/collision/primitives.zig:135-200) and
body.Transform (src/physics/body.zig:141-158) for the fields detectCollision reads;
`detect_collision` has its signature and result (narrow_phase.zig:28-123: a ContactResult,
or None where the reference returns null). `detect_collisions` runs a whole batch of pairs in
one launch on COLLIDER_DTYPE records (the C ABI's ZenoAmdCollider).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import numpy as np

from . import _lib as L

GEOM_TYPES = {"sphere": 0, "capsule": 1, "box": 2, "plane": 3, "cylinder": 4, "mesh": 5, "heightfield": 6}

COLLIDER_DTYPE = np.dtype([("type", "u4"), ("size", "3f4"), ("local_pos", "4f4"), ("position", "4f4"),
                           ("quaternion", "4f4")])
CONTACT_RESULT_DTYPE = np.dtype([("point", "3f4"), ("penetration", "f4"), ("normal", "3f4"), ("valid", "u4"),
                                 ("local_a", "4f4"), ("local_b", "4f4")])
assert COLLIDER_DTYPE.itemsize == 64 and CONTACT_RESULT_DTYPE.itemsize == 64


@dataclass
class Geom:
    """primitives.Geom, reduced to what detectCollision reads (its own local rotation is
    not among them: axes come from the body transform)."""
    geom_type: str = "sphere"
    local_pos: Tuple[float, float, float] = (0.0, 0.0, 0.0)
    size: Tuple[float, float, float] = (1.0, 1.0, 1.0)

    @staticmethod
    def sphere(radius: float) -> "Geom":
        return Geom("sphere", size=(radius, 0.0, 0.0))

    @staticmethod
    def capsule(radius: float, half_length: float) -> "Geom":
        return Geom("capsule", size=(radius, half_length, 0.0))

    @staticmethod
    def box(half_x: float, half_y: float, half_z: float) -> "Geom":
        return Geom("box", size=(half_x, half_y, half_z))

    @staticmethod
    def plane(normal: Sequence[float] = (0.0, 0.0, 1.0), offset: float = 0.0) -> "Geom":
        """The reference stores the normal as the geom's local rotation, which
        detectCollision does not read: a plane's normal is its body's +z."""
        return Geom("plane", size=(offset, 0.0, 0.0))

    def get_radius(self) -> float:
        return self.size[0]

    def get_half_length(self) -> float:
        return self.size[1]

    def get_half_extents(self) -> Tuple[float, float, float]:
        return tuple(self.size)

    def get_plane_offset(self) -> float:
        return self.size[0]


@dataclass
class Transform:
    position: Tuple[float, float, float] = (0.0, 0.0, 0.0)
    quaternion: Tuple[float, float, float, float] = (0.0, 0.0, 0.0, 1.0)  # xyzw


@dataclass
class ContactResult:
    point: np.ndarray
    normal: np.ndarray
    penetration: float
    local_a: np.ndarray
    local_b: np.ndarray
    valid: bool = True


def collider(geom: Geom, transform: Transform) -> np.ndarray:
    """One COLLIDER_DTYPE record."""
    r = np.zeros((), COLLIDER_DTYPE)
    r["type"] = GEOM_TYPES[geom.geom_type]
    r["size"] = geom.size
    r["local_pos"][:3] = geom.local_pos
    r["position"][:3] = transform.position
    r["quaternion"] = transform.quaternion
    return r


def detect_collisions(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """detectCollision for every pair (a[i], b[i]) in one GPU launch; returns
    CONTACT_RESULT_DTYPE records (all zero with valid 0 where there is no contact)."""
    a = np.ascontiguousarray(a, COLLIDER_DTYPE).reshape(-1)
    b = np.ascontiguousarray(b, COLLIDER_DTYPE).reshape(-1)
    if a.shape != b.shape:
        raise ValueError(f"operand arrays differ in length: {a.shape[0]} vs {b.shape[0]}")
    out = np.zeros(a.shape[0], CONTACT_RESULT_DTYPE)
    if a.shape[0] == 0:
        return out
    lib = L.load()
    rc = lib.zeno_amd_detect_collisions_host(a.ctypes.data_as(C.c_void_p), b.ctypes.data_as(C.c_void_p),
                                             a.shape[0], out.ctypes.data_as(C.c_void_p))
    if rc != 0:
        raise RuntimeError(f"detect_collisions failed: {rc}: {L.last_error()}")
    return out


def detect_collision(geom_a: Geom, transform_a: Transform, geom_b: Geom,
                     transform_b: Transform) -> Optional[ContactResult]:
    """narrow_phase.detectCollision for one pair (narrow_phase.zig:28-123)."""
    r = detect_collisions(collider(geom_a, transform_a)[None], collider(geom_b, transform_b)[None])[0]
    if not r["valid"]:
        return None
    return ContactResult(point=r["point"].copy(), normal=r["normal"].copy(), penetration=float(r["penetration"]),
                         local_a=r["local_a"][:3].copy(), local_b=r["local_b"][:3].copy())
