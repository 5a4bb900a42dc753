"""The count-only broad phases of a full contact list, against the oracle bit for bit.

Once a list is full (count >= M; no step clears the count, all_shaders.metal:765-766) and a
substep cannot wrap the count past 2^32, the one-environment-per-wave kernel only counts the
listed pairs that pass (:468-533): the pairs with a plane as a model constant, the others by a
sweep of the non-plane geoms (at most 64) across the wave's lanes. These scenes force one
environment per wave and a short list, so the sweep runs from the first substep on, with
bodies of one and two geoms, random contype/conaffinity masks (zero masks included), NaN
positions, and counts on both sides of the wrap guard (count <= 2^32 - 1 - P). The spatial
hash has a count-only form as well (its last test).
"""
import os

import numpy as np
import pytest

from oracle.oracle import OracleWorld
from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays
from zeno_amd.model import load_model
from zeno_amd.world import ZenoWorld

pytestmark = pytest.mark.gpu

M = 8


def masked_scene(nbodies: int, two_geoms_every: int, seed: int) -> str:
    rng = np.random.default_rng(seed)
    lines = ["<mujoco><worldbody>", '<geom type="plane" size="5 5 0.1"/>']
    for i in range(nbodies):
        x, y = rng.uniform(-0.6, 0.6, 2)
        z = rng.uniform(0.05, 1.0)
        lines.append(f'<body name="b{i}" pos="{x:.3f} {y:.3f} {z:.3f}"><joint type="free"/>')
        for k in range(2 if (i + 1) % two_geoms_every == 0 else 1):
            kind = ["sphere", "capsule", "box"][int(rng.integers(0, 3))]
            size = {"sphere": 1, "capsule": 2, "box": 3}[kind]
            sz = " ".join(f"{v:.3f}" for v in rng.uniform(0.04, 0.14, size))
            off = " ".join(f"{v:.3f}" for v in (rng.uniform(-0.1, 0.1, 3) if k else np.zeros(3)))
            ct, ca = (int(v) for v in rng.integers(0, 4, 2))
            lines.append(f'<geom type="{kind}" size="{sz}" pos="{off}" contype="{ct}" conaffinity="{ca}"/>')
        lines.append("</body>")
    lines.append("</worldbody></mujoco>")
    return "\n".join(lines)


def pair_one_env_per_wave(xml: str, envs: int, max_contacts: int = M, epw: int = 1, split: bool = None):
    overrides = {"ZENO_AMD_ENVS_PER_WAVE": str(epw), "ZENO_AMD_SPLIT": None if split is None else str(int(split))}
    saved = {k: os.environ.get(k) for k in overrides}
    try:
        for k, v in overrides.items():
            if v is not None:
                os.environ[k] = v
        g = ZenoWorld(mjcf_string=xml, num_envs=envs, max_contacts_per_env=max_contacts)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    m = load_model(mjcf_string=xml)
    o = OracleWorld(m, envs, max_contacts_per_env=max_contacts)
    assert g.launch_config()[0] == epw
    if split is not None:
        assert g.split_groups() == split
    return m, g, o


def hinged_row(n: int) -> str:
    """n capsules hinged to the world body over a plane, swinging under gravity."""
    lines = ["<mujoco><worldbody>", '<geom type="plane" size="5 5 0.1"/>']
    for i in range(n):
        lines.append(f'<body name="p{i}" pos="{0.3 * i:.2f} 0 1"><joint type="hinge" axis="0 1 0"/>'
                     f'<geom type="capsule" size="0.05 0.3" pos="0.2 0 0" quat="0.7071 0 0.7071 0"/></body>')
    lines.append("</worldbody></mujoco>")
    return "\n".join(lines)


@pytest.mark.parametrize("scene,epw", [("free32", 2), ("free16", 4), ("hinged16", 4), ("hinged64", 1)])
def test_static_world_body_set_aside(scene, epw):
    """Scenes whose bodies after the world body fill whole passes of an environment's lanes
    (B - 1 = 64 / EPW or 64), without split groups: the per-body stages take bodies 1.. across
    the lanes and set the static world body aside. Free bodies, and bodies hinged to the world (whose joints read
    the world body's pose), every step against the oracle."""
    xml = {"free32": masked_scene(32, 1000, 7), "free16": masked_scene(16, 1000, 8),
           "hinged16": hinged_row(16), "hinged64": hinged_row(64)}[scene]
    m, g, o = pair_one_env_per_wave(xml, 8, max_contacts=16, epw=epw, split=False)
    assert (m["num_bodies"] - 1) % (64 // epw) == 0
    for _ in range(12):
        g.step(np.zeros((8, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    g.close()


@pytest.mark.parametrize("nbodies,every,seed", [(40, 3, 0), (30, 1, 1), (64, 1000, 2), (45, 2, 3)])
def test_sweep_counts_match_oracle(nbodies, every, seed):
    """40 bodies with every third holding two geoms (53 non-plane geoms), 30 with two each
    (60), 64 with one (64: the widest sweep), and 45 with every second holding two (67: over
    64, so the pair loop runs instead); env 2 starts with a NaN position."""
    xml = masked_scene(nbodies, every, seed)
    m, g, o = pair_one_env_per_wave(xml, 4)
    B = m["num_bodies"]
    state = [np.ascontiguousarray(np.broadcast_to(m[k], (4, B, 4)), np.float32).copy()
             for k in ("init_positions", "init_quaternions", "init_velocities", "init_angular_velocities")]
    rng = np.random.default_rng(seed + 10)
    state[0][:, 1:, :2] += rng.uniform(-0.05, 0.05, (4, B - 1, 2)).astype(np.float32)
    state[0][2, 3, 0] = np.nan
    g.reset_to_state(*state)
    o.reset_to_state(*state)
    for _ in range(10):
        g.step(np.zeros((4, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    assert np.all(o.contact_counts >= M)
    g.close()


def test_sweep_wrap_guard_boundary():
    """The pile (P = 2080 listed pairs): counts at 2^32 - 1 - P (the last count the sweep
    takes), one above it (the pair loop), 10 below 2^32 (the pair loop, wrapping) and one far
    from the wrap."""
    g, o, acts = make_pair("pile", 4, 6, seed=5, envs_per_wave=1)
    P = int(o.model["num_pairs"])
    for k in range(2):
        g.step(acts[k])
        o.step(acts[k])
    top = np.uint64((1 << 32) - 1 - P)
    counts = np.array([top, top + 1, (1 << 32) - 10, 1000], np.uint64).astype(np.uint32)
    g.set_contact_counts(counts)
    o.contact_counts[:] = counts
    for k in range(2, 6):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    g.close()


def test_hash_count_only_matches_oracle():
    """The spatial hash's count-only queries (a full list, no wrap possible this substep:
    count <= 2^32 - 1 - G (G - 1) / 2): the 600-body hash pile with a 16-slot list, env 1's
    bodies crowded into the clamped corner cells (long runs, dealt out across the wave), env 2
    with NaN positions, and counts on both sides of the wrap guard, every step against the
    oracle."""
    g, o, acts = make_pair("pile_hash", 4, 8, seed=11, max_contacts=16)
    B = o.B
    state = [o.positions.copy(), o.quaternions.copy(), o.velocities.copy(), o.angular_velocities.copy()]
    rng = np.random.default_rng(12)
    state[0][1, 1:201, :2] = rng.uniform(-4.0, 0.9, (200, 2)).astype(np.float32)
    state[0][2, 5:9, 0] = np.nan
    g.reset_to_state(*state)
    o.reset_to_state(*state)
    g.step(acts[0])
    o.step(acts[0])
    compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    G = int(o.model["num_geoms"])
    top = np.uint64((1 << 32) - 1 - G * (G - 1) // 2)
    counts = o.contact_counts.astype(np.uint64)
    counts[0], counts[3] = top, top + 1
    counts = counts.astype(np.uint32)
    g.set_contact_counts(counts)
    o.contact_counts[:] = counts
    for k in range(1, 8):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    assert np.all(o.contact_counts[1:3] >= 16)
    g.close()


@pytest.mark.parametrize("substeps", [1, 2])
def test_bodies_finished_at_integration_match_oracle(substeps):
    """Working sets in HBM with a full list: the bodies no slot or constraint names are finished
    by the fused integration (velocity update and accelerations in registers, no previous pose
    stored); the others take the velocity update. The hash pile forced into placement 2 with a
    16-slot list: without views, with the body views held (the write-back then writes every
    acceleration), and through step_subset, every step against the oracle."""
    g, o, acts = make_pair("pile_hash", 3, 9, seed=17, max_contacts=16, placement=2, substeps=substeps)
    assert g.modes()["placement"] == 2
    for k in range(3):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    held = (g.get_body_positions(zero_copy=True), g.get_body_velocities(zero_copy=True))
    for k in range(3, 6):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
        np.testing.assert_array_equal(held[0], g.get_body_positions(zero_copy=False))
    mask = np.array([1, 0, 1], np.uint8)
    for k in range(6, 9):
        g.step_subset(acts[k], mask)
        o.step_subset(acts[k], mask)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    assert np.all(o.contact_counts >= 16)
    g.close()


@pytest.mark.parametrize("region", ["upper", "mixed"])
def test_hash_count_only_at_the_grid_edges(region):
    """Count-only hash queries where the runs meet the grid's edges: bodies around cells 62-63
    on every axis (coordinates up to 66 clamp into cell 63, so x + 1, y + 1 and z + 1 leave
    the grid), and a mixed layout of the far corner, the origin's clamped cells and open
    space, every step against the oracle with a 16-slot list."""
    g, o, acts = make_pair("pile_hash", 3, 6, seed=23, max_contacts=16)
    state = [o.positions.copy(), o.quaternions.copy(), o.velocities.copy(), o.angular_velocities.copy()]
    rng = np.random.default_rng(29)
    n = o.B - 1
    if region == "upper":
        state[0][:, 1:, :3] = rng.uniform(61.5, 66.0, (3, n, 3)).astype(np.float32)
    else:
        pick = rng.integers(0, 3, n)
        far = rng.uniform(61.5, 66.0, (3, n, 3))
        low = rng.uniform(-3.0, 1.5, (3, n, 3))
        mid = rng.uniform(10.0, 14.0, (3, n, 3))
        state[0][:, 1:, :3] = np.where(pick[None, :, None] == 0, far, np.where(pick[None, :, None] == 1, low, mid)).astype(np.float32)
    state[2][:] = 0.0
    state[3][:] = 0.0
    g.reset_to_state(*state)
    o.reset_to_state(*state)
    for k in range(6):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
        np.testing.assert_array_equal(g.get_cell_ids(), o.cell_ids[:, : g.num_geoms])
    assert np.all(o.contact_counts >= 16)
    g.close()
