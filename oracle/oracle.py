"""Python driver for the CPU oracle (liboracle: zeno_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product. It steps a batch of environments on the CPU with the
scalar restatement of the reference's step, on state arrays in the reference's layouts.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path
from typing import Any, Dict, Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libzeno_oracle.so"

CONTACT_DTYPE = np.dtype([("position_pen", "4f4"), ("normal_friction", "4f4"), ("indices", "4u4"),
                          ("impulses", "4f4")])
CONSTRAINT_DTYPE = np.dtype([("indices", "4u4"), ("anchor_a", "4f4"), ("anchor_b", "4f4"),
                             ("axis_target", "4f4"), ("limits", "4f4"), ("state", "4f4")])


# narrow_phase.detectCollision operands and result (zeno_oracle.h ZoCollider / ZoContactResult)
COLLIDER_DTYPE = np.dtype([("type", "u4"), ("size", "3f4"), ("local_pos", "4f4"), ("position", "4f4"),
                           ("quaternion", "4f4")])
CONTACT_RESULT_DTYPE = np.dtype([("point", "3f4"), ("penetration", "f4"), ("normal", "3f4"), ("valid", "u4"),
                                 ("local_a", "4f4"), ("local_b", "4f4")])


class ZoModel(C.Structure):
    _fields_ = [
        ("num_envs", C.c_uint32), ("num_bodies", C.c_uint32), ("num_joints", C.c_uint32),
        ("num_geoms", C.c_uint32), ("num_actuators", C.c_uint32), ("num_sensors", C.c_uint32),
        ("obs_dim", C.c_uint32), ("num_constraints", C.c_uint32), ("num_colors", C.c_uint32),
        ("max_contacts", C.c_uint32), ("contact_iterations", C.c_uint32), ("config_substeps", C.c_uint32),
        ("timestep", C.c_float), ("gravity", C.c_float * 3),
        ("friction", C.c_float), ("restitution", C.c_float), ("baumgarte", C.c_float), ("slop", C.c_float),
        ("bodies", C.c_void_p), ("joints", C.c_void_p), ("geoms", C.c_void_p), ("actuators", C.c_void_p),
        ("sensors", C.c_void_p), ("color_ranges", C.c_void_p), ("extended_contacts", C.c_uint32),
    ]


class ZoState(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "positions", "quaternions", "velocities", "angular_velocities", "accelerations", "inv_mass_inertia",
        "forces", "torques", "prev_positions", "prev_quaternions", "prev_velocities",
        "joint_positions", "joint_velocities", "joint_torques", "observations",
        "contacts", "contact_counts", "prev_contacts", "prev_contact_counts", "constraints", "cell_ids")]


_lib = None


def load() -> C.CDLL:
    """The oracle library: oracle/libzeno_oracle.so, or the build named by ZENO_ORACLE_LIB
    (the sanitizer test loads an ASan/UBSan build of the same source that way)."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("ZENO_ORACLE_LIB", str(LIB_PATH)))
        if not path.exists():
            raise RuntimeError(f"oracle library missing: {path} (build with python -m zeno_amd.build)")
        lib = C.CDLL(str(path))
        lib.zo_step.restype = C.c_int
        lib.zo_step.argtypes = [C.POINTER(ZoModel), C.POINTER(ZoState), C.c_void_p, C.c_uint32,
                                C.c_uint32, C.c_uint32, C.c_int]
        lib.zo_build_templates.restype = C.c_uint32
        lib.zo_build_templates.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32,
                                           C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32)]
        lib.zo_atan2f.restype = C.c_float
        lib.zo_atan2f.argtypes = [C.c_float, C.c_float]
        lib.zo_asinf.restype = C.c_float
        lib.zo_asinf.argtypes = [C.c_float]
        lib.zo_match_cached.restype = None
        lib.zo_match_cached.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]
        lib.zo_solve_contact_slot.restype = None
        lib.zo_solve_contact_slot.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                              C.c_float, C.c_float, C.c_float]
        lib.zo_sort_contacts.restype = None
        lib.zo_sort_contacts.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32]
        lib.zo_detect_collision.restype = C.c_int
        lib.zo_detect_collision.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        lib.zo_detect_collisions.restype = None
        lib.zo_detect_collisions.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_int]
        lib.zo_broad_phase_hash.restype = None
        lib.zo_broad_phase_hash.argtypes = [C.POINTER(ZoModel), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        lib.zo_collide_env.restype = None
        lib.zo_collide_env.argtypes = [C.POINTER(ZoModel), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        _lib = lib
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def build_templates(model: Dict[str, Any]):
    """Recomputes constraint templates, colours and colour ranges from the joint records."""
    lib = load()
    J = model["num_joints"]
    out = np.zeros(max(3 * J, 1), dtype=CONSTRAINT_DTYPE)
    ranges = np.zeros(512, dtype=np.uint32)
    ncol = C.c_uint32()
    joints = np.ascontiguousarray(model["joints"])
    limited = np.ascontiguousarray(model["joint_limited"], dtype=np.uint8)
    bodies = np.ascontiguousarray(model["bodies"])
    n = lib.zo_build_templates(_p(joints) if J else None, _p(limited) if J else None, J, _p(bodies),
                               model["num_bodies"], _p(out), _p(ranges), C.byref(ncol))
    return out[:n].copy(), ranges[: 2 * ncol.value].reshape(-1, 2).copy(), ncol.value


class OracleWorld:
    """A batch of environments in the reference's buffer layouts, stepped on the CPU."""

    def __init__(self, model: Dict[str, Any], num_envs: int, timestep: float = 0.0,
                 contact_iterations: int = 4, max_contacts_per_env: int = 64, substeps: int = 1):
        self.lib = load()
        self.model = model
        E, B = num_envs, model["num_bodies"]
        # The constraint templates, colours and colour ranges come from the oracle's own builder
        # (zo_build_templates), not from the product's model records.
        tmpl, ranges, self.num_colors = build_templates(model)
        J, A, N = model["num_joints"], model["num_actuators"], len(tmpl)
        Jp, Op, M = max(J, 1), max(model["obs_dim"], 1), max_contacts_per_env
        self.E, self.B, self.J, self.A, self.N, self.M = E, B, J, A, N, M
        self.timestep = float(timestep if timestep > 0 else model["timestep"])
        self.gravity = list(model["gravity"])
        self.contact_iterations = contact_iterations
        self.substeps = substeps
        f4 = lambda: np.zeros((E, B, 4), np.float32)
        self.positions = np.ascontiguousarray(np.broadcast_to(model["init_positions"], (E, B, 4)), np.float32).copy()
        self.quaternions = np.ascontiguousarray(np.broadcast_to(model["init_quaternions"], (E, B, 4)), np.float32).copy()
        self.velocities = np.ascontiguousarray(np.broadcast_to(model["init_velocities"], (E, B, 4)), np.float32).copy()
        self.angular_velocities = np.ascontiguousarray(np.broadcast_to(model["init_angular_velocities"], (E, B, 4)), np.float32).copy()
        self.inv_mass_inertia = np.ascontiguousarray(np.broadcast_to(model["inv_mass_inertia"], (E, B, 4)), np.float32).copy()
        self.accelerations, self.forces, self.torques = f4(), f4(), f4()
        self.prev_positions, self.prev_quaternions, self.prev_velocities = f4(), f4(), f4()
        self.joint_positions = np.zeros((E, Jp), np.float32)
        self.joint_velocities = np.zeros((E, Jp), np.float32)
        self.joint_torques = np.zeros((E, Jp), np.float32)
        self.observations = np.zeros((E, Op), np.float32)
        self.contacts = np.zeros((E, M), CONTACT_DTYPE)
        self.contact_counts = np.zeros(E, np.uint32)
        self.prev_contacts = np.zeros((E, M), CONTACT_DTYPE)
        self.prev_contact_counts = np.zeros(E, np.uint32)
        self.cell_ids = np.zeros((E, max(model["num_geoms"], 1)), np.uint32)
        self.extended_contacts = False
        self.constraints = np.ascontiguousarray(np.broadcast_to(tmpl, (E, N)), CONSTRAINT_DTYPE).copy()
        if N:
            self.constraints["indices"][:, :, 2] = np.arange(E, dtype=np.uint32)[:, None]
        self._keep = {k: np.ascontiguousarray(model[k]) for k in
                      ("bodies", "joints", "geoms", "actuators", "sensors")}
        self._keep["color_ranges"] = np.ascontiguousarray(ranges, dtype=np.uint32).reshape(-1)

    def _model_struct(self) -> ZoModel:
        m = self.model
        zm = ZoModel()
        zm.num_envs, zm.num_bodies, zm.num_joints = self.E, self.B, self.J
        zm.num_geoms, zm.num_actuators, zm.num_sensors = m["num_geoms"], self.A, m["num_sensors"]
        zm.obs_dim, zm.num_constraints, zm.num_colors = m["obs_dim"], self.N, self.num_colors
        zm.max_contacts, zm.contact_iterations, zm.config_substeps = self.M, self.contact_iterations, self.substeps
        zm.timestep = self.timestep
        for i in range(3):
            zm.gravity[i] = self.gravity[i]
        zm.friction, zm.restitution = m["friction"], m["restitution"]
        zm.baumgarte, zm.slop = m["baumgarte"], m["slop"]
        k = self._keep
        zm.bodies = _p(k["bodies"])
        zm.joints = _p(k["joints"]) if self.J else None
        zm.geoms = _p(k["geoms"]) if m["num_geoms"] else None
        zm.actuators = _p(k["actuators"]) if self.A else None
        zm.sensors = _p(k["sensors"]) if m["num_sensors"] else None
        zm.color_ranges = _p(k["color_ranges"]) if k["color_ranges"].size else None
        zm.extended_contacts = 1 if self.extended_contacts else 0
        return zm

    def _state_struct(self) -> ZoState:
        s = ZoState()
        for name, _ in ZoState._fields_:
            setattr(s, name, _p(getattr(self, name)))
        return s

    def step(self, actions: Optional[np.ndarray], substeps: int = 0, env_begin: int = 0,
             env_end: Optional[int] = None, nthreads: int = 0) -> None:
        a = np.zeros((self.E, max(self.A, 1)), np.float32) if actions is None else \
            np.ascontiguousarray(actions, np.float32).reshape(self.E, self.A)
        if self.A == 0:
            a = np.zeros((self.E, 1), np.float32)
        zm, zs = self._model_struct(), self._state_struct()
        end = self.E if env_end is None else env_end
        self.lib.zo_step(C.byref(zm), C.byref(zs), _p(a), substeps, env_begin, end, nthreads)

    _SUBSET_RESTORED = ("positions", "quaternions", "velocities", "accelerations", "angular_velocities",
                        "joint_positions", "joint_velocities", "joint_torques", "observations",
                        "contact_counts", "contacts")

    def step_subset(self, actions: Optional[np.ndarray], env_mask, substeps: int = 0) -> None:
        """World.stepSubset (world.zig:833-929): no active env -> no-op; all active -> step;
        otherwise back up the per-env outputs, step every env, and restore the unmasked envs'
        bodies, accelerations, joints, observations, counts and contacts. Constraint lambdas and
        the prev-contact cache of unmasked envs keep the full step's values."""
        mask = np.asarray(env_mask).astype(bool)
        if not mask.any():
            return
        if mask.all():
            self.step(actions, substeps)
            return
        backup = {k: getattr(self, k).copy() for k in self._SUBSET_RESTORED}
        self.step(actions, substeps)
        keep = ~mask
        for k, v in backup.items():
            getattr(self, k)[keep] = v[keep]

    def set_body_positions(self, positions, mask=None) -> None:
        """World.setBodyPositions: copy the selected envs' positions, nothing else."""
        sel = np.ones(self.E, bool) if mask is None else np.asarray(mask).astype(bool)
        self.positions[sel] = np.asarray(positions, np.float32).reshape(self.E, self.B, 4)[sel]

    def set_body_velocities(self, velocities, mask=None) -> None:
        sel = np.ones(self.E, bool) if mask is None else np.asarray(mask).astype(bool)
        self.velocities[sel] = np.asarray(velocities, np.float32).reshape(self.E, self.B, 4)[sel]

    def reset_to_state(self, positions, quaternions, velocities=None, angular_velocities=None, mask=None):
        """main.zig:290-385: copy the given arrays for the selected envs; zero every count."""
        sel = np.ones(self.E, bool) if mask is None else np.asarray(mask).astype(bool)
        self.positions[sel] = np.asarray(positions, np.float32).reshape(self.E, self.B, 4)[sel]
        self.quaternions[sel] = np.asarray(quaternions, np.float32).reshape(self.E, self.B, 4)[sel]
        if velocities is not None:
            self.velocities[sel] = np.asarray(velocities, np.float32).reshape(self.E, self.B, 4)[sel]
        if angular_velocities is not None:
            self.angular_velocities[sel] = np.asarray(angular_velocities, np.float32).reshape(self.E, self.B, 4)[sel]
        self.contact_counts[:] = 0

    def reset(self, mask=None):
        """world.zig:1296-1314: restore the scene pose, zero joint q/qd, zero every count."""
        sel = np.ones(self.E, bool) if mask is None else np.asarray(mask).astype(bool)
        self.positions[sel] = self.model["init_positions"]
        self.quaternions[sel] = self.model["init_quaternions"]
        self.velocities[sel] = self.model["init_velocities"]
        self.angular_velocities[sel] = self.model["init_angular_velocities"]
        self.joint_positions[sel] = 0
        self.joint_velocities[sel] = 0
        self.contact_counts[:] = 0

    def lambdas(self) -> np.ndarray:
        return self.constraints["state"][:, :, 0].copy()


def sort_contacts(contacts: np.ndarray, count: int) -> None:
    """In-place stable insertion sort of one env's contact list (schedule of the reference)."""
    assert contacts.dtype == CONTACT_DTYPE and contacts.flags["C_CONTIGUOUS"]
    load().zo_sort_contacts(contacts.shape[0], _p(contacts), count)


def match_cached(contacts: np.ndarray, count: int, prev: np.ndarray, prev_count: int) -> None:
    """In-place warm start of one env's contacts from its previous list."""
    assert contacts.shape == prev.shape
    load().zo_match_cached(contacts.shape[0], _p(contacts), count, _p(prev), prev_count)


def solve_contact_slot(inv_mass_inertia: np.ndarray, positions: np.ndarray, velocities: np.ndarray,
                       angular_velocities: np.ndarray, contact: np.ndarray, baumgarte: float = 0.2,
                       slop: float = 0.005, dt: float = 0.01) -> None:
    """solve_contacts on one slot (all_shaders.metal:1644-1793). The [B, 4] float32 state
    arrays and the one-record contact array are updated in place."""
    arrs = [np.ascontiguousarray(x, np.float32) for x in (inv_mass_inertia, positions, velocities, angular_velocities)]
    for x, orig in zip(arrs[1:], (positions, velocities, angular_velocities)):
        assert x is orig, "state arrays must be C-contiguous float32 (updated in place)"
    assert contact.dtype == CONTACT_DTYPE and contact.shape == (1,) and contact.flags["C_CONTIGUOUS"]
    B = arrs[0].shape[0]
    assert all(x.shape == (B, 4) for x in arrs)
    load().zo_solve_contact_slot(B, _p(arrs[0]), _p(positions), _p(velocities), _p(angular_velocities), _p(contact),
                                 baumgarte, slop, dt)


def collide_env(world: "OracleWorld", env: int = 0) -> None:
    """Broad phase + sort + narrow phase of one env on its current positions."""
    zm = world._model_struct()
    cnt = np.array([world.contact_counts[env]], np.uint32)
    con = np.ascontiguousarray(world.contacts[env])
    load().zo_collide_env(C.byref(zm), _p(np.ascontiguousarray(world.positions[env])),
                          _p(np.ascontiguousarray(world.quaternions[env])), _p(con), _p(cnt))
    world.contacts[env] = con
    world.contact_counts[env] = cnt[0]


def broad_phase_hash(world: "OracleWorld", env: int = 0, count: int = 0):
    """The spatial-hash broad phase alone on one env's current positions, at any geom count.

    Returns (cell_ids [G] u32, contacts [M] with indices of the first min(n, M) pairs, n).
    """
    zm = world._model_struct()
    G = world.model["num_geoms"]
    ids = np.zeros(max(G, 1), np.uint32)
    cnt = np.array([count], np.uint32)
    con = np.zeros(world.M, CONTACT_DTYPE)
    load().zo_broad_phase_hash(C.byref(zm), _p(np.ascontiguousarray(world.positions[env])), _p(ids), _p(con), _p(cnt))
    return ids[:G], con, int(cnt[0])


def detect_collisions(a: np.ndarray, b: np.ndarray, nthreads: int = 1) -> np.ndarray:
    """narrow_phase.detectCollision for each pair (a[i], b[i]) of COLLIDER_DTYPE records;
    returns CONTACT_RESULT_DTYPE records (all zero, valid 0, where there is no contact)."""
    a = np.ascontiguousarray(a, COLLIDER_DTYPE)
    b = np.ascontiguousarray(b, COLLIDER_DTYPE)
    assert a.shape == b.shape and a.ndim == 1
    out = np.zeros(a.shape[0], CONTACT_RESULT_DTYPE)
    if a.shape[0]:
        load().zo_detect_collisions(_p(a), _p(b), a.shape[0], _p(out), nthreads)
    return out


def atan2f(y: float, x: float) -> float:
    return load().zo_atan2f(y, x)


def asinf(x: float) -> float:
    return load().zo_asinf(x)
