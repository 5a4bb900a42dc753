"""Contact levels wider than a wave's lane pairs, against the oracle bit for bit.

With one environment per wave the contact solve takes a level's slots on the wave's 32 lane
pairs, so a wider level takes two or more passes (lane pair k solves slots k, k + 32, ...).
These scenes rest many bodies on the plane at once, so the first level holds one slot per
resting body (33-64 wide, then over 64) and the duplicate slots of the next substeps make
narrower levels after it; a long pile run ends with its bodies settled on the plane. Every
launch placement that runs one environment per wave is covered (working sets in LDS, model
records in HBM, working sets in HBM).
"""
import os

import numpy as np
import pytest

from oracle.oracle import OracleWorld
from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays
from zeno_amd.model import load_model
from zeno_amd.world import ZenoWorld

pytestmark = pytest.mark.gpu


def resting_scene(n: int, seed: int, stacked: int = 0) -> str:
    """n bodies on a grid 0.35 apart (no pair but the plane's within the broad phase's reach),
    each sunk 2-8 mm into the plane: spheres, and capsules lying along x. The first `stacked`
    spheres carry a second sphere resting on top of them (a sphere-sphere slot beside the
    plane's)."""
    rng = np.random.default_rng(seed)
    side = int(np.ceil(np.sqrt(n)))
    lines = ["<mujoco><worldbody>", '<geom type="plane" size="20 20 0.1"/>']
    for i in range(n):
        x, y = 0.35 * (i % side), 0.35 * (i // side)
        r = float(rng.uniform(0.05, 0.1))
        sink = float(rng.uniform(0.002, 0.008))
        if i % 5 == 4:
            lines.append(f'<body name="c{i}" pos="{x:.3f} {y:.3f} {r - sink:.4f}"><joint type="free"/>'
                         f'<geom type="capsule" size="{r:.4f} 0.06" quat="0.7071068 0 0.7071068 0"/></body>')
        else:
            lines.append(f'<body name="s{i}" pos="{x:.3f} {y:.3f} {r - sink:.4f}"><joint type="free"/>'
                         f'<geom type="sphere" size="{r:.4f}"/></body>')
            if i < stacked:
                lines.append(f'<body name="t{i}" pos="{x:.3f} {y:.3f} {2 * r + 0.045:.4f}"><joint type="free"/>'
                             f'<geom type="sphere" size="0.05"/></body>')
    lines.append("</worldbody></mujoco>")
    return "\n".join(lines)


def level_widths(contacts: np.ndarray, counts: np.ndarray, inv_mass: np.ndarray) -> list:
    """Widths of the contact levels of each env (schedule S4: a valid slot's level is one more
    than the highest level of an earlier valid slot sharing a dynamic body)."""
    out = []
    for e in range(contacts.shape[0]):
        lev, width = {}, {}
        for k in range(min(int(counts[e]), contacts.shape[1])):
            if contacts["position_pen"][e, k, 3] < 0:
                continue
            dyn = [int(b) for b in contacts["indices"][e, k, :2] if inv_mass[int(b)] > 1e-8]
            lv = 1 + max([lev.get(b, 0) for b in dyn] + [0])
            for b in dyn:
                lev[b] = lv
            width[lv] = width.get(lv, 0) + 1
        out.append(width)
    return out


def pair(xml: str, envs: int, max_contacts: int, placement: int):
    overrides = {"ZENO_AMD_ENVS_PER_WAVE": "1", "ZENO_AMD_PLACEMENT": str(placement), "ZENO_AMD_SPLIT": "0"}
    saved = {k: os.environ.get(k) for k in overrides}
    try:
        os.environ.update(overrides)
        g = ZenoWorld(mjcf_string=xml, num_envs=envs, max_contacts_per_env=max_contacts)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    m = load_model(mjcf_string=xml)
    o = OracleWorld(m, envs, max_contacts_per_env=max_contacts)
    assert g.launch_config()[0] == 1 and g.modes()["placement"] == placement
    return m, g, o


@pytest.mark.parametrize("placement", [0, 1, 2])
@pytest.mark.parametrize("n,M,stacked", [(48, 64, 0), (100, 128, 0), (60, 96, 12)])
def test_wide_levels_match_oracle(n, M, stacked, placement):
    """48 resting bodies with a 64-slot list (a 48-wide first level, then the 16 duplicates of
    the second step), 100 with 128 slots (a 100-wide level: lanes take a second slot), and 60
    with 12 of them carrying a second sphere (96 slots); env 1 starts with its bodies moving."""
    xml = resting_scene(n, seed=n + stacked, stacked=stacked)
    m, g, o = pair(xml, 3, M, placement)
    B = m["num_bodies"]
    state = [np.ascontiguousarray(np.broadcast_to(m[k], (3, B, 4)), np.float32).copy()
             for k in ("init_positions", "init_quaternions", "init_velocities", "init_angular_velocities")]
    rng = np.random.default_rng(n)
    state[2][1, 1:, :3] = rng.uniform(-0.3, 0.3, (B - 1, 3)).astype(np.float32)
    state[3][1, 1:, :3] = rng.uniform(-2.0, 2.0, (B - 1, 3)).astype(np.float32)
    g.reset_to_state(*state)
    o.reset_to_state(*state)
    widest = 0
    for _ in range(8):
        g.step(np.zeros((3, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
        w = level_widths(o.contacts, o.contact_counts, m["inv_mass_inertia"][:, 0])
        widest = max([widest] + [max(x.values()) for x in w if x])
    assert widest > (64 if n == 100 else 32)
    g.close()


def test_settled_pile_matches_oracle():
    """The rigid pile (64 bodies per env) over 600 steps at one environment per wave with the
    model records in HBM (the shape the world picks for it at 8192 envs), compared every 100
    steps: by the end its bodies rest on the plane and their slots make levels over 32 wide."""
    g, o, acts = make_pair("pile", 4, 600, seed=3, envs_per_wave=1, placement=1, split=False)
    z = np.zeros((4, 0), np.float32)
    for k in range(600):
        g.step(z)
        o.step(None)
        if k % 100 == 99:
            compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    w = level_widths(o.contacts, o.contact_counts, o.model["inv_mass_inertia"][:, 0])
    assert max(max(x.values()) for x in w if x) > 32
    g.close()
