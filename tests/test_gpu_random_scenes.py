"""Randomised scenes through the whole step, GPU against the oracle, bit for bit.

The shipped assets exercise a handful of fixed trees; these scenes draw the tree shape, the
joint types (hinge, slide, ball, free, implicit fixed), joint axes and ranges, geom types and
sizes (spheres, capsules, boxes, overlapping siblings), motors with gears and control ranges,
and joint/frame sensors from a seed, and run them under every launch-shape family the world
can pick (one or several environments per wave, split groups, several groups per
workgroup, model records in HBM). Every step of every scene must equal the oracle's.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle.oracle import OracleWorld
from tests.parity import compare, gpu_arrays, oracle_arrays
from zeno_amd.model import load_model
from zeno_amd.world import ZenoWorld

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-6)


def _mixed_range(rng: np.random.Generator) -> str:
    """A joint range of one of the kinds the assets carry: none, small in radians, MJCF degrees
    on both sides (bounds beyond +-2 pi: an angular limit that can never act), degrees on one
    side (a hinge limit the angle is always beyond), or bounds at the +-2 pi threshold itself."""
    kind = rng.choice(["none", "radians", "degrees", "one_sided", "threshold"], p=[0.2, 0.2, 0.3, 0.1, 0.2])
    if kind == "none":
        return ""
    if kind == "radians":
        lo, hi = rng.uniform(-1.2, -0.1), rng.uniform(0.1, 1.2)
    elif kind == "degrees":
        lo, hi = -rng.uniform(10, 150), rng.uniform(10, 150)
    elif kind == "one_sided":
        lo, hi = -rng.uniform(60, 150), -rng.uniform(10, 50)
    else:
        b = 6.2832 if rng.random() < 0.5 else 6.2831  # float32: just beyond / just inside 2 fp32(pi)
        lo, hi = -b, b
    return f' range="{lo:.4f} {hi:.4f}"'


def random_scene_mjcf(rng: np.random.Generator, ranges: str = "small") -> str:
    """An articulated scene over a ground plane: 1-3 trees up to depth 3, each body with one
    joint (or none: an implicit fixed joint) and one geom; motors on some hinge and slide
    joints; joint and frame sensors. ranges="mixed" draws the joint ranges from _mixed_range."""
    lines = ["<mujoco><worldbody>", '<geom type="plane" size="5 5 0.1"/>']
    joints, bodies = [], []

    def vec(lo, hi):
        return " ".join(f"{v:.3f}" for v in rng.uniform(lo, hi, 3))

    def body(depth, top):
        name = f"b{len(bodies)}"
        bodies.append(name)
        pos = vec(-0.4, 0.4) if not top else f"{rng.uniform(-1, 1):.3f} {rng.uniform(-1, 1):.3f} {rng.uniform(0.3, 1.2):.3f}"
        out = [f'<body name="{name}" pos="{pos}">']
        kind = rng.choice(["hinge", "slide", "ball", "free", "none"], p=[0.45, 0.15, 0.15, 0.1, 0.15])
        if kind == "free" and not top:
            kind = "hinge"
        if kind != "none":
            jn = f"j{len(joints)}"
            joints.append((jn, kind))
            if ranges == "small":
                rng_attr = f' range="{rng.uniform(-1.2, -0.1):.3f} {rng.uniform(0.1, 1.2):.3f}"' if rng.random() < 0.5 else ""
            else:
                rng_attr = _mixed_range(rng)
            ax = rng.normal(size=3)
            ax /= np.linalg.norm(ax)
            out.append(f'<joint name="{jn}" type="{kind}" axis="{" ".join(f"{v:.4f}" for v in ax)}"'
                       f' pos="{vec(-0.1, 0.1)}"{rng_attr}/>')
        g = rng.choice(["sphere", "capsule", "box", "capsule_fromto"])
        if g == "sphere":
            out.append(f'<geom type="sphere" size="{rng.uniform(0.04, 0.2):.3f}"/>')
        elif g == "capsule":
            out.append(f'<geom type="capsule" size="{rng.uniform(0.03, 0.1):.3f} {rng.uniform(0.05, 0.25):.3f}" pos="{vec(-0.1, 0.1)}"/>')
        elif g == "box":
            out.append(f'<geom type="box" size="{vec(0.03, 0.15)}"/>')
        else:
            out.append(f'<geom type="capsule" size="{rng.uniform(0.03, 0.1):.3f}" fromto="0 0 0 {vec(-0.3, 0.3)}"/>')
        if depth < 3:
            for _ in range(int(rng.integers(0, 3))):
                out += body(depth + 1, False)
        out.append("</body>")
        return out

    for _ in range(int(rng.integers(1, 4))):
        lines += body(0, True)
    lines.append("</worldbody>")
    motors = [(n, k) for n, k in joints if k in ("hinge", "slide") and rng.random() < 0.7]
    if motors:
        lines.append("<actuator>")
        for n, _ in motors:
            lines.append(f'<motor joint="{n}" ctrlrange="-1 1" gear="{rng.uniform(5, 120):.1f}"/>')
        lines.append("</actuator>")
    lines.append("<sensor>")
    for n, k in joints[:4]:
        if k in ("hinge", "slide"):
            lines.append(f'<jointpos joint="{n}"/>')
            lines.append(f'<jointvel joint="{n}"/>')
    lines.append(f'<framepos objtype="body" objname="{bodies[0]}"/>')
    lines.append(f'<framequat objtype="body" objname="{bodies[0]}"/>')
    lines.append("</sensor></mujoco>")
    return "\n".join(lines)


SHAPES = {
    "auto": {},
    "one_env_per_wave": {"ZENO_AMD_ENVS_PER_WAVE": "1", "ZENO_AMD_WAVES": "1", "ZENO_AMD_SPLIT": "0"},
    "split_epw4": {"ZENO_AMD_ENVS_PER_WAVE": "4", "ZENO_AMD_WAVES": "1", "ZENO_AMD_SPLIT": "1"},
    "groups_2x2": {"ZENO_AMD_ENVS_PER_WAVE": "2", "ZENO_AMD_WAVES": "2", "ZENO_AMD_SPLIT": "0"},
    "model_in_hbm": {"ZENO_AMD_PLACEMENT": "1"},
}


def _world(xml: str, envs: int, shape: dict) -> ZenoWorld:
    saved = {k: os.environ.get(k) for k in shape}
    try:
        os.environ.update(shape)
        return ZenoWorld(mjcf_string=xml, num_envs=envs)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


# Seeds whose scenes stay finite over the run. Others blow up within a few steps, on the GPU
# and in the oracle alike: the reference's step does not filter contacts between a parent and
# a child body, so overlapping geoms on jointed neighbours push against the joint every step.
STABLE_SEEDS = [1, 2, 3, 4, 6, 8, 9]


def _run_scene(rng: np.random.Generator, xml: str, shape: str, steps: int = 24, finite: bool = True) -> None:
    E = 13  # an env count that leaves the last group partly empty
    g = _world(xml, E, SHAPES[shape])
    o = OracleWorld(load_model(mjcf_string=xml), E)
    # Perturbed start: every env's bodies moved and spun a little, so contacts and limits
    # differ between envs.
    pos = g.get_body_positions(zero_copy=False)
    vel = g.get_body_velocities(zero_copy=False)
    pos[:, 1:, :3] += rng.uniform(-0.05, 0.05, pos[:, 1:, :3].shape).astype(np.float32)
    vel[:, 1:, :3] += rng.uniform(-0.5, 0.5, vel[:, 1:, :3].shape).astype(np.float32)
    g.set_body_positions(pos)
    o.set_body_positions(pos)
    g.set_body_velocities(vel)
    o.set_body_velocities(vel)
    A = g.action_dim
    for k in range(steps):
        a = rng.uniform(-1, 1, (E, max(A, 1))).astype(np.float32)[:, :A]
        g.step(a)
        o.step(a)
        compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    ok = np.isfinite(g.get_body_positions(zero_copy=False)).all(axis=(1, 2))
    if finite:
        assert ok.all()
    else:
        assert not ok.all() and ok.any()  # some envs went non-finite, others did not
    g.close()


@pytest.mark.parametrize("shape", sorted(SHAPES))
@pytest.mark.parametrize("seed", STABLE_SEEDS)
def test_random_scene_matches_oracle(seed, shape):
    rng = np.random.default_rng(1000 + seed)
    _run_scene(rng, random_scene_mjcf(rng), shape)


# The seeds left out above blow up: positions reach 1e7 and velocities 1e10 within 24 steps,
# and some environments overflow to inf and NaN after 55-58 steps. Run past that point, every
# step compared: NaN poses go through the broad phase (a NaN distance passes the margin test),
# the sort, the narrow phase, the contact levels and the solves, and the discrete outputs
# (counts, pair lists, active flags) must stay exactly the oracle's, the fp32 state bit for
# bit (any NaN matching any NaN).
UNSTABLE_SEEDS = [0, 5, 7]


@pytest.mark.parametrize("shape", ["auto", "one_env_per_wave", "split_epw4", "model_in_hbm"])
@pytest.mark.parametrize("seed", UNSTABLE_SEEDS)
def test_random_scene_through_non_finite_state(seed, shape):
    rng = np.random.default_rng(1000 + seed)
    _run_scene(rng, random_scene_mjcf(rng), shape, steps=64, finite=False)


# Mixed joint ranges: seeds whose scenes stay finite over the run and hold both an angular limit
# that can never act (bounds beyond +-2 pi, left out of the GPU's joint program while the oracle
# evaluates it) and one that can.
MIXED_SEEDS = [2, 5, 8, 9, 12, 14, 15, 16]
TWO_PI_F = np.float32(6.28318548)


@pytest.mark.parametrize("shape", ["auto", "one_env_per_wave", "split_epw4", "model_in_hbm"])
@pytest.mark.parametrize("seed", MIXED_SEEDS)
def test_random_scene_mixed_ranges_match_oracle(seed, shape):
    rng = np.random.default_rng(5000 + seed)
    xml = random_scene_mjcf(rng, ranges="mixed")
    c = load_model(mjcf_string=xml)["constraints"]
    lim = [k for k in range(len(c)) if (int(c[k]["indices"][3]) & 0xFF) == 4]
    never = [k for k in lim if np.float32(c[k]["limits"][0]) <= -TWO_PI_F and np.float32(c[k]["limits"][1]) >= TWO_PI_F]
    assert 0 < len(never) < len(lim)
    _run_scene(rng, xml, shape)


# In the extended-contact mode the same scenes also collide boxes and capsules with each other
# and with the plane (detectCollision inside the step), so slots often write two bodies and
# the contact levels come from relaxation. Seeds that stay finite over the run in that mode:
EXT_SEEDS = [1, 2, 4, 5, 8, 14]


@pytest.mark.parametrize("shape", ["auto", "one_env_per_wave", "model_in_hbm"])
@pytest.mark.parametrize("seed", EXT_SEEDS)
def test_random_scene_extended_contacts_match_oracle(seed, shape):
    _run_extended(seed, shape, steps=24, finite=True)


# Extended-mode seeds that overflow to inf / NaN in some environments after 43-57 steps.
EXT_UNSTABLE_SEEDS = [0, 6, 10]


@pytest.mark.parametrize("shape", ["auto", "model_in_hbm"])
@pytest.mark.parametrize("seed", EXT_UNSTABLE_SEEDS)
def test_random_scene_extended_contacts_through_non_finite_state(seed, shape):
    _run_extended(seed, shape, steps=64, finite=False)


def _run_extended(seed: int, shape: str, steps: int, finite: bool) -> None:
    rng = np.random.default_rng(1000 + seed)
    xml = random_scene_mjcf(rng)
    E, M = 13, 128
    saved = {k: os.environ.get(k) for k in SHAPES[shape]}
    try:
        os.environ.update(SHAPES[shape])
        g = ZenoWorld(mjcf_string=xml, num_envs=E, max_contacts_per_env=M)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    o = OracleWorld(load_model(mjcf_string=xml), E, max_contacts_per_env=M)
    g.set_extended_contacts(True)
    o.extended_contacts = True
    pos = g.get_body_positions(zero_copy=False)
    vel = g.get_body_velocities(zero_copy=False)
    pos[:, 1:, :3] += rng.uniform(-0.05, 0.05, pos[:, 1:, :3].shape).astype(np.float32)
    vel[:, 1:, :3] += rng.uniform(-0.5, 0.5, vel[:, 1:, :3].shape).astype(np.float32)
    g.set_body_positions(pos)
    o.set_body_positions(pos)
    g.set_body_velocities(vel)
    o.set_body_velocities(vel)
    A = g.action_dim
    active = 0
    for k in range(steps):
        a = rng.uniform(-1, 1, (E, max(A, 1))).astype(np.float32)[:, :A]
        g.step(a)
        o.step(a)
        compare(gpu_arrays(g), oracle_arrays(o), **TOL)
        live = np.arange(M)[None, :] < np.minimum(o.contact_counts, M)[:, None]
        active += int(((o.contacts["position_pen"][..., 3] >= 0) & live).sum())
    assert active > 0
    ok = np.isfinite(g.get_body_positions(zero_copy=False)).all(axis=(1, 2))
    assert ok.all() if finite else (not ok.all() and ok.any())
    g.close()
