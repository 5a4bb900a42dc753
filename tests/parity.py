"""GPU-vs-oracle comparison helpers shared by the parity tests and smoke()."""
from __future__ import annotations

import os
from typing import Dict, Optional

import numpy as np

from oracle.oracle import OracleWorld
from zeno_amd.scenes import workload_inputs
from zeno_amd.world import ZenoWorld

FLOAT_FIELDS = ("positions", "quaternions", "velocities", "angular_velocities", "accelerations",
                "joint_positions", "joint_velocities", "joint_torques", "observations")


def gpu_arrays(w: ZenoWorld) -> Dict[str, np.ndarray]:
    J = w.num_joints
    return {
        "positions": w.get_body_positions(zero_copy=False),
        "quaternions": w.get_body_quaternions(zero_copy=False),
        "velocities": w.get_body_velocities(zero_copy=False),
        "angular_velocities": w.get_body_angular_velocities(zero_copy=False),
        "accelerations": w.get_body_accelerations(zero_copy=False),
        "joint_positions": w.get_joint_positions(zero_copy=False),
        "joint_velocities": w.get_joint_velocities(zero_copy=False),
        "joint_torques": w.get_joint_forces(zero_copy=False),
        "observations": w.get_observations(zero_copy=False),
        "contacts": w.get_contacts(zero_copy=False),
        "contact_counts": w.get_contact_counts(),
        "prev_contact_counts": w.get_prev_contact_counts(),
        "lambda": w.get_lambda(),
        "_J": J,
    }


def oracle_arrays(o: OracleWorld) -> Dict[str, np.ndarray]:
    J = o.J
    return {
        "positions": o.positions, "quaternions": o.quaternions, "velocities": o.velocities,
        "angular_velocities": o.angular_velocities, "accelerations": o.accelerations,
        "joint_positions": o.joint_positions[:, :J], "joint_velocities": o.joint_velocities[:, :J],
        "joint_torques": o.joint_torques[:, :J], "observations": o.observations[:, : o.model["obs_dim"]],
        "contacts": o.contacts, "contact_counts": o.contact_counts,
        "prev_contact_counts": o.prev_contact_counts, "lambda": o.lambdas(), "_J": J,
    }


def live_mask(counts: np.ndarray, M: int) -> np.ndarray:
    """[E, M] True for slots < min(count, M)."""
    return np.arange(M)[None, :] < np.minimum(counts, M)[:, None]


def _same_bits(a: np.ndarray, b: np.ndarray, what: str) -> None:
    """fp32 arrays equal bit for bit, signed zeros included. A NaN matches any NaN: IEEE 754
    leaves the payload an operation returns to the implementation (the GPU returns the
    canonical quiet NaN, x86 propagates an operand's)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    differ = (a.view(np.uint32) != b.view(np.uint32)) & ~(np.isnan(a) & np.isnan(b))
    bad = np.argwhere(differ)
    assert bad.size == 0, (f"{what}: {len(bad)} values differ in their bits, first at {tuple(bad[0])}: "
                           f"{a[tuple(bad[0])]!r} vs {b[tuple(bad[0])]!r}")


def compare(g: Dict[str, np.ndarray], o: Dict[str, np.ndarray], rtol: float, atol: float,
            exact: bool = True) -> Dict[str, float]:
    """Discrete outputs must match exactly; float outputs within rtol/atol (the tolerances the
    parity contract states) and, with exact, bit for bit as well (the GPU and the oracle
    evaluate the same fp32 operations in the same order). Returns the max absolute difference
    per field and raises on a violation."""
    out: Dict[str, float] = {}
    np.testing.assert_array_equal(g["contact_counts"], o["contact_counts"], err_msg="contact_counts")
    np.testing.assert_array_equal(g["prev_contact_counts"], o["prev_contact_counts"], err_msg="prev_contact_counts")
    M = g["contacts"].shape[1]
    live = live_mask(o["contact_counts"], M)
    gi, oi = g["contacts"]["indices"], o["contacts"]["indices"]
    np.testing.assert_array_equal(gi[live], oi[live], err_msg="contact indices (pair lists after sort)")
    g_active = (g["contacts"]["position_pen"][..., 3] >= 0) & live
    o_active = (o["contacts"]["position_pen"][..., 3] >= 0) & live
    np.testing.assert_array_equal(g_active, o_active, err_msg="contact active flags")
    for f in ("position_pen", "normal_friction", "impulses"):
        a, b = g["contacts"][f][live], o["contacts"][f][live]
        np.testing.assert_allclose(a, b, rtol=rtol, atol=atol, err_msg=f"contacts.{f}")
        if exact:
            _same_bits(a, b, f"contacts.{f}")
        out[f"contacts.{f}"] = float(np.max(np.abs(a - b))) if a.size else 0.0
    for f in FLOAT_FIELDS + ("lambda",):
        a, b = np.asarray(g[f], np.float32), np.asarray(o[f], np.float32)
        assert a.shape == b.shape, (f, a.shape, b.shape)
        np.testing.assert_allclose(a, b, rtol=rtol, atol=atol, err_msg=f)
        if exact:
            _same_bits(a, b, f)
        out[f] = float(np.max(np.abs(a - b))) if a.size else 0.0
    return out


def make_pair(name: str, num_envs: int, steps: int, seed: int = 0, envs_per_wave: Optional[int] = None,
              substeps: int = 1, max_contacts: int = 64, contact_iterations: int = 4,
              placement: Optional[int] = None, extended_contacts: bool = False, waves: Optional[int] = None,
              split: Optional[bool] = None):
    """GPU world and oracle on the same seeded state. envs_per_wave / waves (environment groups
    per workgroup) / split (two waves per group) / placement (1: model records in HBM, 2:
    working sets in HBM too) override the launch shape the world would choose;
    extended_contacts turns on the extended-contact mode on both."""
    path, xml, model, state, acts = workload_inputs(name, num_envs, steps, seed)
    overrides = {"ZENO_AMD_ENVS_PER_WAVE": None if envs_per_wave is None else str(envs_per_wave),
                 "ZENO_AMD_PLACEMENT": None if placement is None else str(placement),
                 "ZENO_AMD_WAVES": None if waves is None else str(waves),
                 "ZENO_AMD_SPLIT": None if split is None else ("1" if split else "0")}
    saved = {k: os.environ.get(k) for k in overrides}
    try:
        for k, v in overrides.items():
            if v is not None:
                os.environ[k] = v
        g = ZenoWorld(mjcf_path=path, mjcf_string=xml, num_envs=num_envs, substeps=substeps,
                      max_contacts_per_env=max_contacts, contact_iterations=contact_iterations)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    o = OracleWorld(model, num_envs, max_contacts_per_env=max_contacts, substeps=substeps,
                    contact_iterations=contact_iterations)
    if extended_contacts:
        g.set_extended_contacts(True)
        o.extended_contacts = True
    g.reset_to_state(*state)
    o.reset_to_state(*state)
    return g, o, acts
