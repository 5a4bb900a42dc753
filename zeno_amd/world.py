"""ZenoWorld: the Python face of one batched world (python/zeno/_ffi.py:438-1162).

Method names, argument meanings, array shapes and error behaviour follow the reference's
ZenoWorld. Arrays returned with ``zero_copy=True`` are views of the library's pinned host
mirrors. Once a getter has handed a mirror out, the library brings it up to date before
every step, reset or setter returns, so a view held across steps follows the simulation as
the reference's unified-memory views do (at the cost of one device-to-host copy of that
array per call; arrays never handed out are copied only when their getter is called).
"""
from __future__ import annotations

import ctypes as C
from typing import Any, Dict, Optional, Tuple

import numpy as np

from . import _lib as L

CONTACT_DTYPE = np.dtype([
    ("position_pen", "4f4"),
    ("normal_friction", "4f4"),
    ("indices", "4u4"),
    ("impulses", "4f4"),
])


def version() -> str:
    return L.load().zeno_version().decode()


def is_metal_available() -> bool:
    return bool(L.load().zeno_metal_available())


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _u8ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.POINTER(C.c_uint8))


class ZenoWorld:
    """A batch of identical environments stepped together on one GPU."""

    def __init__(
        self,
        mjcf_path: Optional[str] = None,
        mjcf_string: Optional[str] = None,
        num_envs: int = 1,
        timestep: float = 0,
        contact_iterations: int = 4,
        max_contacts_per_env: int = 64,
        seed: int = 42,
        substeps: int = 1,
        enable_profiling: bool = False,
        max_bodies_per_env: int = 64,
        max_joints_per_env: int = 64,
        max_geoms_per_env: int = 128,
    ):
        self._lib = L.load()
        self._handle = None
        self._views: Dict[Any, np.ndarray] = {}
        if mjcf_path is None and mjcf_string is None:
            raise ValueError("Either mjcf_path or mjcf_string must be provided")
        cfg = L.ZenoConfig(num_envs=num_envs, timestep=timestep, contact_iterations=contact_iterations,
                           max_contacts_per_env=max_contacts_per_env, seed=seed, substeps=substeps,
                           enable_profiling=enable_profiling, max_bodies_per_env=max_bodies_per_env,
                           max_joints_per_env=max_joints_per_env, max_geoms_per_env=max_geoms_per_env)
        if mjcf_path is not None:
            h = self._lib.zeno_world_create(str(mjcf_path).encode(), C.byref(cfg))
        else:
            h = self._lib.zeno_world_create_from_string(mjcf_string.encode(), C.byref(cfg))
        if not h:
            raise RuntimeError(f"Failed to create Zeno world: {L.last_error()}")
        self._handle = h
        self._num_envs = int(self._lib.zeno_world_num_envs(h))
        self._obs_dim = int(self._lib.zeno_world_obs_dim(h))
        self._action_dim = int(self._lib.zeno_world_action_dim(h))
        info = L.ZenoInfo()
        self._lib.zeno_world_get_info(h, C.byref(info))
        self._num_bodies = int(info.num_bodies)
        self._num_joints = int(info.num_joints)
        self._num_sensors = int(info.num_sensors)
        self._num_geoms = int(info.num_geoms)
        self._timestep = float(info.timestep)
        self._memory_usage = int(info.memory_usage)
        self._gpu_memory_usage = int(info.gpu_memory_usage)
        self._max_contacts_per_env = int(self._lib.zeno_world_max_contacts_per_env(h))

    def close(self) -> None:
        if self._handle:
            self._views.clear()
            self._lib.zeno_world_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- properties ---------------------------------------------------------------------
    @property
    def handle(self):
        return self._handle

    @property
    def num_envs(self) -> int:
        return self._num_envs

    @property
    def obs_dim(self) -> int:
        return self._obs_dim

    @property
    def action_dim(self) -> int:
        return self._action_dim

    @property
    def num_bodies(self) -> int:
        return self._num_bodies

    @property
    def num_joints(self) -> int:
        return self._num_joints

    @property
    def num_sensors(self) -> int:
        return self._num_sensors

    @property
    def num_geoms(self) -> int:
        return self._num_geoms

    @property
    def timestep(self) -> float:
        return self._timestep

    @property
    def memory_usage(self) -> int:
        return self._memory_usage

    @property
    def gpu_memory_usage(self) -> int:
        return self._gpu_memory_usage

    @property
    def max_contacts_per_env(self) -> int:
        return self._max_contacts_per_env

    # ---- stepping -----------------------------------------------------------------------
    def step(self, actions: np.ndarray, substeps: int = 0) -> None:
        a = np.ascontiguousarray(actions, dtype=np.float32).reshape(-1)
        if a.size < self._num_envs * self._action_dim:
            raise ValueError(f"expected {self._num_envs * self._action_dim} actions, got {a.size}")
        rc = self._lib.zeno_world_step(self._handle, _fptr(a), substeps)
        if rc != 0:
            raise RuntimeError(f"Step failed with error code {rc}: {L.last_error()}")

    def step_subset(self, actions: np.ndarray, env_mask: np.ndarray, substeps: int = 0) -> None:
        a = np.ascontiguousarray(actions, dtype=np.float32).reshape(-1)
        m = np.ascontiguousarray(env_mask, dtype=np.uint8).reshape(-1)
        if m.size != self._num_envs:
            raise ValueError("env_mask must have num_envs entries")
        rc = self._lib.zeno_world_step_subset(self._handle, _fptr(a), _u8ptr(m), substeps)
        if rc != 0:
            raise RuntimeError(f"Step subset failed with error code {rc}: {L.last_error()}")

    def reset(self, mask: Optional[np.ndarray] = None) -> None:
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8).reshape(-1)
        rc = self._lib.zeno_world_reset(self._handle, _u8ptr(m))
        if rc != 0:
            raise RuntimeError(f"Reset failed with error code {rc}")

    def reset_to_state(self, positions: np.ndarray, quaternions: np.ndarray,
                       velocities: Optional[np.ndarray] = None,
                       angular_velocities: Optional[np.ndarray] = None,
                       mask: Optional[np.ndarray] = None) -> None:
        n = self._num_envs * self._num_bodies * 4
        p = np.ascontiguousarray(positions, dtype=np.float32).reshape(-1)
        q = np.ascontiguousarray(quaternions, dtype=np.float32).reshape(-1)
        v = None if velocities is None else np.ascontiguousarray(velocities, dtype=np.float32).reshape(-1)
        w = None if angular_velocities is None else np.ascontiguousarray(angular_velocities, dtype=np.float32).reshape(-1)
        for arr in (p, q, v, w):
            if arr is not None and arr.size != n:
                raise ValueError(f"state arrays must have shape (num_envs, num_bodies, 4) = {n} floats")
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8).reshape(-1)
        rc = self._lib.zeno_world_reset_to_state(self._handle, _fptr(p), _fptr(q),
                                                 None if v is None else _fptr(v),
                                                 None if w is None else _fptr(w), _u8ptr(m))
        if rc != 0:
            raise RuntimeError(f"Reset to state failed with error code {rc}")

    # ---- getters --------------------------------------------------------------------------
    def _view(self, ptr, shape: Tuple[int, ...], ctype, dtype, zero_copy: bool) -> np.ndarray:
        if not ptr:
            return np.zeros(shape, dtype=dtype)
        # Each host mirror keeps one address for the world's lifetime, so its ndarray is built
        # once (a ctypes-to-numpy view costs a few microseconds, a getter call in an RL loop
        # is otherwise ~1 us); the C call above still runs every time and does the refresh.
        key = (C.addressof(ptr.contents), shape, dtype)
        arr = self._views.get(key)
        if arr is None:
            count = int(np.prod(shape))
            arr = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ctype)), shape=(count,)).view(dtype).reshape(shape)
            self._views[key] = arr
        return arr.view() if zero_copy else arr.copy()

    def _body(self, fn, zero_copy: bool) -> np.ndarray:
        return self._view(fn(self._handle), (self._num_envs, self._num_bodies, 4), C.c_float, np.float32, zero_copy)

    def get_observations(self, zero_copy: bool = False) -> np.ndarray:
        return self._view(self._lib.zeno_world_get_observations(self._handle), (self._num_envs, self._obs_dim),
                          C.c_float, np.float32, zero_copy)

    def get_rewards(self) -> np.ndarray:
        return self._view(self._lib.zeno_world_get_rewards(self._handle), (self._num_envs,), C.c_float, np.float32, False)

    def get_dones(self) -> np.ndarray:
        return self._view(self._lib.zeno_world_get_dones(self._handle), (self._num_envs,), C.c_uint8, np.uint8, False)

    def get_body_positions(self, zero_copy: bool = True) -> np.ndarray:
        return self._body(self._lib.zeno_world_get_body_positions, zero_copy)

    def get_body_quaternions(self, zero_copy: bool = True) -> np.ndarray:
        return self._body(self._lib.zeno_world_get_body_quaternions, zero_copy)

    def get_body_velocities(self, zero_copy: bool = True) -> np.ndarray:
        return self._body(self._lib.zeno_world_get_body_velocities, zero_copy)

    def get_body_angular_velocities(self, zero_copy: bool = True) -> np.ndarray:
        return self._body(self._lib.zeno_world_get_body_angular_velocities, zero_copy)

    def get_body_accelerations(self, zero_copy: bool = True) -> np.ndarray:
        return self._body(self._lib.zeno_world_get_body_accelerations, zero_copy)

    def _joint(self, fn, zero_copy: bool) -> np.ndarray:
        jp = max(self._num_joints, 1)
        arr = self._view(fn(self._handle), (self._num_envs, jp), C.c_float, np.float32, zero_copy)
        return arr[:, : self._num_joints]

    def get_joint_positions(self, zero_copy: bool = True) -> np.ndarray:
        return self._joint(self._lib.zeno_world_get_joint_positions, zero_copy)

    def get_joint_velocities(self, zero_copy: bool = True) -> np.ndarray:
        return self._joint(self._lib.zeno_world_get_joint_velocities, zero_copy)

    def get_joint_forces(self, zero_copy: bool = True) -> np.ndarray:
        return self._joint(self._lib.zeno_world_get_joint_forces, zero_copy)

    def get_contacts(self, zero_copy: bool = True) -> np.ndarray:
        shape = (self._num_envs, self._max_contacts_per_env)
        ptr = self._lib.zeno_world_get_contacts(self._handle)
        if not ptr:
            return np.zeros(shape, dtype=CONTACT_DTYPE)
        raw = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint8)), shape=(shape[0] * shape[1] * 64,))
        arr = raw.view(CONTACT_DTYPE).reshape(shape)
        return arr if zero_copy else arr.copy()

    def get_contact_counts(self) -> np.ndarray:
        return self._view(self._lib.zeno_world_get_contact_counts(self._handle), (self._num_envs,),
                          C.c_uint32, np.uint32, False)

    def get_sensor_data(self, zero_copy: bool = True) -> np.ndarray:
        return self._view(self._lib.zeno_world_get_sensor_data(self._handle), (self._num_envs, self._obs_dim),
                          C.c_float, np.float32, zero_copy)

    # ---- setters --------------------------------------------------------------------------
    def set_body_positions(self, positions: np.ndarray, mask: Optional[np.ndarray] = None) -> None:
        p = np.ascontiguousarray(positions, dtype=np.float32).reshape(-1)
        if p.size != self._num_envs * self._num_bodies * 4:
            raise ValueError("positions must have shape (num_envs, num_bodies, 4)")
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8).reshape(-1)
        rc = self._lib.zeno_world_set_body_positions(self._handle, _fptr(p), _u8ptr(m))
        if rc != 0:
            raise RuntimeError(f"Set body positions failed: {rc}")

    def set_body_velocities(self, velocities: np.ndarray, mask: Optional[np.ndarray] = None) -> None:
        v = np.ascontiguousarray(velocities, dtype=np.float32).reshape(-1)
        if v.size != self._num_envs * self._num_bodies * 4:
            raise ValueError("velocities must have shape (num_envs, num_bodies, 4)")
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8).reshape(-1)
        rc = self._lib.zeno_world_set_body_velocities(self._handle, _fptr(v), _u8ptr(m))
        if rc != 0:
            raise RuntimeError(f"Set body velocities failed: {rc}")

    def set_gravity(self, gravity: Tuple[float, float, float]) -> None:
        rc = self._lib.zeno_world_set_gravity(self._handle, float(gravity[0]), float(gravity[1]), float(gravity[2]))
        if rc != 0:
            raise RuntimeError(f"Set gravity failed: {rc}")

    def set_timestep(self, timestep: float) -> None:
        rc = self._lib.zeno_world_set_timestep(self._handle, float(timestep))
        if rc != 0:
            raise RuntimeError(f"Set timestep failed: {rc}")
        self._timestep = float(timestep)

    # ---- profiling / state / info -----------------------------------------------------------
    def get_profiling_data(self) -> Dict[str, Any]:
        d = L.ZenoProfilingData()
        if self._lib.zeno_world_get_profiling(self._handle, C.byref(d)) != 0:
            return {}
        return {
            "integrate_ms": d.integrate_ns / 1e6,
            "collision_broad_ms": d.collision_broad_ns / 1e6,
            "collision_narrow_ms": d.collision_narrow_ns / 1e6,
            "constraint_solve_ms": d.constraint_solve_ns / 1e6,
            "total_step_ms": d.total_step_ns / 1e6,
            "num_contacts": d.num_contacts,
            "num_active_constraints": d.num_active_constraints,
        }

    def reset_profiling(self) -> None:
        self._lib.zeno_world_reset_profiling(self._handle)

    def get_state(self) -> Dict[str, np.ndarray]:
        return {
            "body_positions": self.get_body_positions(zero_copy=False),
            "body_quaternions": self.get_body_quaternions(zero_copy=False),
            "body_velocities": self.get_body_velocities(zero_copy=False),
            "body_angular_velocities": self.get_body_angular_velocities(zero_copy=False),
            "joint_positions": self.get_joint_positions(zero_copy=False),
            "joint_velocities": self.get_joint_velocities(zero_copy=False),
        }

    def set_state(self, state: Dict[str, np.ndarray]) -> None:
        self.reset_to_state(positions=state["body_positions"], quaternions=state["body_quaternions"],
                            velocities=state.get("body_velocities"),
                            angular_velocities=state.get("body_angular_velocities"))

    def get_info(self) -> Dict[str, Any]:
        info = L.ZenoInfo()
        self._lib.zeno_world_get_info(self._handle, C.byref(info))
        return {
            "num_envs": info.num_envs, "num_bodies": info.num_bodies, "num_joints": info.num_joints,
            "num_actuators": info.num_actuators, "num_sensors": info.num_sensors, "num_geoms": info.num_geoms,
            "obs_dim": info.obs_dim, "action_dim": info.action_dim, "timestep": info.timestep,
            "memory_usage": info.memory_usage, "gpu_memory_usage": info.gpu_memory_usage,
            "metal_available": bool(info.metal_available),
        }

    # ---- extensions (include/zeno_amd_ext.h) -------------------------------------------------
    def get_lambda(self) -> np.ndarray:
        view = self.model_view()
        n = view["num_constraints"]
        out = np.zeros((self._num_envs, n), dtype=np.float32)
        if n:
            rc = self._lib.zeno_amd_world_get_lambda(self._handle, _fptr(out))
            if rc != 0:
                raise RuntimeError(f"get_lambda failed: {rc}")
        return out

    def set_contact_counts(self, counts: np.ndarray) -> None:
        c = np.ascontiguousarray(counts, dtype=np.uint32)
        if c.shape != (self._num_envs,):
            raise ValueError(f"counts must have shape ({self._num_envs},), got {c.shape}")
        rc = self._lib.zeno_amd_world_set_contact_counts(self._handle, c.ctypes.data_as(C.POINTER(C.c_uint32)))
        if rc != 0:
            raise RuntimeError(f"set_contact_counts failed: {rc}")

    def get_prev_contact_counts(self) -> np.ndarray:
        out = np.zeros(self._num_envs, dtype=np.uint32)
        rc = self._lib.zeno_amd_world_get_prev_contact_counts(self._handle, out.ctypes.data_as(C.POINTER(C.c_uint32)))
        if rc != 0:
            raise RuntimeError(f"get_prev_contact_counts failed: {rc}")
        return out

    def step_device(self, d_actions: int, substeps: int = 0) -> None:
        """One step with actions already in device memory (address d_actions, E x action_dim
        f32); returns after enqueueing."""
        rc = self._lib.zeno_amd_world_step_device(self._handle, C.c_void_p(d_actions or None), substeps)
        if rc != 0:
            raise RuntimeError(f"step_device failed: {rc}: {L.last_error()}")

    def capture_steps(self, d_actions: int, stride_bytes: int, num_steps: int, substeps: int = 0) -> None:
        """Captures num_steps steps into a HIP graph (step k's actions at d_actions + k *
        stride_bytes in device memory); graph_launch() replays them with one call."""
        rc = self._lib.zeno_amd_world_capture_steps(self._handle, C.c_void_p(d_actions or None), stride_bytes,
                                                    num_steps, substeps)
        if rc != 0:
            raise RuntimeError(f"capture_steps failed: {rc}: {L.last_error()}")

    def graph_launch(self) -> None:
        rc = self._lib.zeno_amd_world_graph_launch(self._handle)
        if rc != 0:
            raise RuntimeError(f"graph_launch failed: {rc}: {L.last_error()}")

    def release_graph(self) -> None:
        self._lib.zeno_amd_world_release_graph(self._handle)

    def synchronize(self) -> None:
        rc = self._lib.zeno_amd_world_synchronize(self._handle)
        if rc != 0:
            raise RuntimeError(f"synchronize failed: {rc}: {L.last_error()}")

    def set_kernel_timing(self, enable, every: int = 1) -> None:
        """Records HIP events around every `every`-th step launch (enable False stops)."""
        self._lib.zeno_amd_world_set_kernel_timing(self._handle, int(every) if enable else 0)

    def get_kernel_timing(self) -> Tuple[float, int]:
        ms = C.c_double()
        n = C.c_uint64()
        rc = self._lib.zeno_amd_world_get_kernel_timing(self._handle, C.byref(ms), C.byref(n))
        if rc != 0:
            raise RuntimeError(f"get_kernel_timing failed: {rc}")
        return ms.value, n.value

    def joint_phases(self) -> int:
        """Joint-solve phases per solver iteration (same-type runs of one colour), after the
        constraints that can never act are left out."""
        return int(self._lib.zeno_amd_world_joint_phases(self._handle))

    def launch_config(self) -> Tuple[int, int]:
        epw = C.c_uint32()
        lds = C.c_uint32()
        self._lib.zeno_amd_world_launch_config(self._handle, C.byref(epw), C.byref(lds))
        return epw.value, lds.value

    def waves_per_group(self) -> int:
        """Environment groups per workgroup of the step launches (the groups of a workgroup
        share one copy of the model records in LDS); one wave each, two when split."""
        return int(self._lib.zeno_amd_world_waves_per_group(self._handle))

    def split_groups(self) -> bool:
        """True when each environment group runs on two waves: one solving the joints and
        contacts, one running the contact pipeline (broad phase to levels) meanwhile."""
        return self._lib.zeno_amd_world_split_groups(self._handle) == 1

    def modes(self) -> Dict[str, Any]:
        """{"placement": 0 model + working sets in LDS, 1 model in HBM and working set in LDS,
        2 both in HBM with the contact pipeline's arrays in LDS, 3 everything in HBM (contact
        lists too long for LDS); "spatial_hash": the spatial-hash broad phase runs (G > 512)}."""
        pl = C.c_int()
        sh = C.c_int()
        self._lib.zeno_amd_world_modes(self._handle, C.byref(pl), C.byref(sh))
        return {"placement": pl.value, "spatial_hash": bool(sh.value)}

    def set_extended_contacts(self, enable: bool) -> None:
        """Extended-contact mode: pairs the reference's narrow phase leaves invalid (box and
        capsule pairs) are tested with narrow_phase.detectCollision. Off by default."""
        rc = self._lib.zeno_amd_world_set_extended_contacts(self._handle, 1 if enable else 0)
        if rc != 0:
            raise RuntimeError(f"set_extended_contacts failed: {rc}")

    def get_cell_ids(self) -> np.ndarray:
        """[num_envs, num_geoms] spatial-hash cell of each geom in the last substep."""
        out = np.zeros((self._num_envs, self.num_geoms), dtype=np.uint32)
        rc = self._lib.zeno_amd_world_get_cell_ids(self._handle, out.ctypes.data_as(C.POINTER(C.c_uint32)))
        if rc != 0:
            raise RuntimeError(f"get_cell_ids failed: {rc} (the scene does not use the spatial hash?)")
        return out

    def model_view(self) -> Dict[str, Any]:
        from .model import view_to_dict
        v = L.ZenoAmdModelView()
        rc = self._lib.zeno_amd_world_model_view(self._handle, C.byref(v))
        if rc != 0:
            raise RuntimeError(f"model view failed: {rc}")
        return view_to_dict(v)
