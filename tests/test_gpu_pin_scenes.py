"""The scenes that pin the oracle (tests/test_oracle_pins.py), run through the HIP step and
compared with the oracle bit for bit. The CPU pins show the oracle reads the reference
right on these cases; this shows the kernel computes the same values on them: offset-COM
gravity torques, motors between two dynamic bodies, tilted capsules, unequal friction and
asymmetric collision masks, the broad-phase margin, a rotation past pi in one substep,
slide and hinge joint states on turned and spinning bodies, accelerations over several
substeps, point constraints on offset-COM bodies, and rotated sliders and welds.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.oracle import OracleWorld
from tests import test_oracle_pins as P
from tests.parity import compare, gpu_arrays, oracle_arrays
from zeno_amd.model import load_model
from zeno_amd.world import ZenoWorld

pytestmark = pytest.mark.gpu

E = 3


def _spheres_xml(pa, ra, pb, rb, ga="", gb=""):
    fmt = lambda v: " ".join(f"{x:.6f}" for x in v)
    return P.SPHERES.format(pa=fmt(pa), pb=fmt(pb), ra=ra, rb=rb, ga=ga, gb=gb)


def _rotated_child(joint):
    qc = P._qaxis([0, 0, 1], np.pi / 2)
    return P.ROTATED_CHILD.format(q=" ".join(f"{v:.7f}" for v in (qc[3], qc[0], qc[1], qc[2])), joint=joint), qc


def _cases():
    qa90x = P._qaxis([1, 0, 0], np.pi / 2)
    _, qc = _rotated_child("")
    d = np.array([2.0, -1.0, 2.0]) / 3.0
    cases = {
        "offset_com_gravity": (P.OFFSET_COM_FREE, None, 4, 1, {1: dict(quat=P._qaxis([0, 0, 1], 1.1))}, None),
        "tilted_capsule_shallow": (P.tilted_capsule_mjcf(0.6, 0.28), None, 4, 1, {}, None),
        "tilted_capsule_flat": (P.tilted_capsule_mjcf(-1.4, 0.1), None, 4, 1, {}, None),
        "sphere_overlap_unequal": (_spheres_xml((0.3, 0.4, 5.0), 0.3, np.array([0.3, 0.4, 5.0]) + 0.8 * d, 0.6),
                                   (0, 0, 0), 4, 1, {}, None),
        "friction_mean": (_spheres_xml((0, 0, 5), 0.5, (0.8, 0, 5), 0.5, ga='friction="0.25 0.005 0.0001"',
                                       gb='friction="1 0.005 0.0001"'), (0, 0, 0), 4, 1, {}, None),
        "contype_asymmetric": (_spheres_xml((0, 0, 5), 0.5, (0.5, 0, 5), 0.5, ga='contype="1" conaffinity="0"',
                                            gb='contype="0" conaffinity="1"'), (0, 0, 0), 4, 1, {}, None),
        "broad_margin_in": (_spheres_xml((0, 0, 5), 0.5, (1.099, 0, 5), 0.5), (0, 0, 0), 4, 1, {}, None),
        "broad_margin_out": (_spheres_xml((0, 0, 5), 0.5, (1.101, 0, 5), 0.5), (0, 0, 0), 4, 1, {}, None),
        "rotation_past_pi": (P.HINGE_LIMIT, (0, 0, 0), 4, 1, {1: dict(quat=P._qaxis([0, 1, 0], 0.8))}, None),
        "slide_state_free": (P.SLIDE_PAIR, (0, 0, 0), 0, 1,
                             {1: dict(quat=P._qaxis([0, 0, 1], 0.3), vel=(0.2, -0.1, 0.05), angvel=(0.5, 0, 0)),
                              2: dict(pos=(0.35, 0.1, 2.25), quat=P._qaxis([1, 2, 3], 0.7), vel=(-0.3, 0.4, 0.1),
                                      angvel=(0.3, -0.2, 2.0))}, None),
        "slide_state_solved": (P.SLIDE_PAIR, (0, 0, 0), 4, 1,
                               {1: dict(quat=P._qaxis([0, 0, 1], 0.3), vel=(0.2, -0.1, 0.05), angvel=(0.5, 0, 0)),
                                2: dict(pos=(0.35, 0.1, 2.25), quat=P._qaxis([1, 2, 3], 0.7), vel=(-0.3, 0.4, 0.1),
                                        angvel=(0.3, -0.2, 2.0))}, None),
        "hinge_local_axis": (P.HINGE_PAIR, (0, 0, 0), 0, 1,
                             {1: dict(quat=qa90x, angvel=(0.1, 0.2, -0.3)),
                              2: dict(pos=(0, 0.5, 2), quat=P._qmul(qa90x, P._qaxis([0, 1, 0], 2.5)),
                                      angvel=(0.4, -0.5, 1.5))}, None),
        "frame_sensors": (P.FRAME_SENSORS, None, 4, 1, {1: dict(vel=(1.0, 0.5, 2.0), angvel=(0.3, -0.4, 1.0))}, None),
        "accel_substeps_2": (P.FREE_BALL, None, 4, 2, {}, None),
        "accel_substeps_4": (P.FREE_BALL, None, 4, 4, {}, None),
        "point_offset_com": (P.BALL_OFFSET_COM, (0, 0, 0), 1, 1, {2: dict(pos=(1.3, 0, 1))}, None),
        "point_offset_com_gravity": (P.BALL_OFFSET_COM, None, 4, 1, {2: dict(pos=(1.3, 0, 1))}, None),
        "slider_rotated": (_rotated_child('<joint type="slide" axis="1 0 0"/>')[0], (0, 0, 0), 1, 1,
                           {1: dict(quat=P._qmul(P._qaxis([1, 0, 0], 0.3), qc))}, None),
        "weld_rotated": (_rotated_child("")[0], (0, 0, 0), 1, 1,
                         {1: dict(quat=P._qmul(P._qaxis([1, 0, 0], 0.3), qc))}, None),
        "spinner_world_frame": (P.SPINNER, (0, 0, 0), 4, 1, {1: dict(quat=qa90x, angvel=(0, 0, 3.0))}, None),
        "raised_plane": (P.RAISED_PLANE, None, 4, 1, {}, None),
        "two_geoms_one_body": (P.TWO_GEOMS_ONE_BODY, (0, 0, 0), 4, 1, {}, None),
        "weld_dynamic_parent": (P.WELD_ON_FREE_PARENT, (0, 0, 0), 1, 1, {2: dict(pos=(0.3, 0.2, 1.0))}, None),
        "angular_limit_lower": (P.HINGE_LIMIT, (0, 0, 0), 3, 1, {1: dict(quat=P._qaxis([0, 1, 0], -0.8))}, None),
        "ball_driven_into_plane": (P.FALLING_BALL, (0, 0, 0), 1, 1, {1: dict(vel=(0.0, 0.0, -2.0))}, None),
    }
    ctrl = np.array([0.5, -0.05, 2e-6, 9e-7, -5e-7, 0.0, 1.0, -1.0], np.float32)
    for kind in ("hinge", "slide"):
        for grav in ((0, 0, 0), None):
            key = f"motor_{kind}_{'nogravity' if grav else 'gravity'}"
            cases[key] = (P.MOTOR_PAIR.format(kind=kind), grav, 4, 1,
                          {1: dict(quat=qa90x), 2: dict(quat=P._qaxis([0, 0, 1], np.pi / 2))}, ctrl)
    return cases


CASES = _cases()


def _state(w_like, B, setup):
    """[E, B, 4] arrays from the model's initial state with `setup` applied to every env; env k
    moves each body by 1e-3 k along x so the envs differ."""
    p = w_like.positions.copy()
    q = w_like.quaternions.copy()
    v = w_like.velocities.copy()
    av = w_like.angular_velocities.copy()
    for b, s in setup.items():
        for arr, key in ((p, "pos"), (v, "vel"), (av, "angvel")):
            if key in s:
                arr[:, b, :3] = s[key]
        if "quat" in s:
            q[:, b] = np.asarray(s["quat"], np.float32)
    p[:, 1:, 0] += (1e-3 * np.arange(E, dtype=np.float32))[:, None]
    return p, q, v, av


@pytest.mark.parametrize("name", list(CASES))
def test_pin_scene_matches_oracle(name):
    xml, gravity, iterations, substeps, setup, ctrl = CASES[name]
    m = load_model(mjcf_string=xml)
    o = OracleWorld(m, E, contact_iterations=iterations, substeps=substeps)
    g = ZenoWorld(mjcf_string=xml, num_envs=E, contact_iterations=iterations, substeps=substeps)
    if gravity is not None:
        o.gravity = list(gravity)
        g.set_gravity(tuple(float(x) for x in gravity))
    state = _state(o, m["num_bodies"], setup)
    o.reset_to_state(*state)
    g.reset_to_state(*state)
    A = max(m["num_actuators"], 1)
    for k in range(12):
        acts = np.zeros((E, A), np.float32)
        if ctrl is not None:
            acts[:, 0] = ctrl[k % len(ctrl)]
        g.step(acts[:, : m["num_actuators"]] if m["num_actuators"] else acts)
        o.step(acts[:, : m["num_actuators"]] if m["num_actuators"] else None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    g.close()
