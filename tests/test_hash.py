"""Pins the oracle's spatial-hash broad phase (all_shaders.metal:556-703; world.zig:534 turns
it on above 512 geoms) with checks that do not restate its loops:

  cell ids        closed forms at chosen coordinates: floor, clamping to [0, 63], NaN and
                  negative coordinates in cell 0, x + 64 y + 4096 z
  pair set        the set definition: g < o, cells at most one apart on every axis, the
                  broad phase's body / contype / distance filters (planes skip distance)
  pair order      the sequential order written as a sort key: (g, dz, dy, dx, o)
  vs O(G^2)       with every geom inside the grid and radius sums + 0.1 below one cell, the
                  non-plane pairs equal those of the O(G^2) broad phase
  plane reach     a plane pairs only with geoms in the 27 cells around its own cell
  filters         geoms sharing a body, contype/conaffinity masks and geom offsets, against
                  the same set definition
  threshold       the step takes the hash above 512 geoms only
  overflow        the count runs past the list's capacity; the first entries are kept
"""
import numpy as np
import pytest

from oracle import oracle as O
from zeno_amd.model import load_model
from zeno_amd.scenes import PILES, pile_initial_state, pile_mjcf


def _pile(name="pile_hash", num_envs=1, max_contacts=64, seed=0, edit=None):
    nb, xy = PILES[name]
    m = load_model(mjcf_string=pile_mjcf(nb, seed=seed, xy=xy))
    if edit is not None:
        edit(m)
    o = O.OracleWorld(m, num_envs, max_contacts_per_env=max_contacts)
    o.reset_to_state(*pile_initial_state(m, num_envs, seed + 1, xy=xy))
    return m, o


def _cells(world_pos: np.ndarray) -> np.ndarray:
    """[G, 3] cell coordinates: floor, then clamp; NaN floors to NaN and lands in cell 0."""
    f = np.floor(world_pos.astype(np.float32))
    c = np.where(np.isnan(f), 0.0, np.clip(f, 0.0, 63.0))
    return c.astype(np.int64)


def _geom_world(m: dict, pos: np.ndarray) -> np.ndarray:
    tb, ps = m["geoms"]["type_body"], m["geoms"]["pos_size0"]
    return (pos[tb[:, 1], :3] + ps[:, :3]).astype(np.float32)


def _expected_pairs(m: dict, pos: np.ndarray, use_cells: bool = True):
    """Ordered (body_a, body_b, g, o) from the set definition and the (g, dz, dy, dx, o) key."""
    tb, ps = m["geoms"]["type_body"].astype(np.int64), m["geoms"]["pos_size0"]
    wp = _geom_world(m, pos)
    c = _cells(wp)
    G = len(tb)
    out = []
    for g in range(G):
        o = np.arange(g + 1, G)
        d = c[o] - c[g]
        ok = tb[o, 1] != tb[g, 1]
        ok &= ((tb[g, 3] & tb[o, 2]) != 0) | ((tb[o, 3] & tb[g, 2]) != 0)
        if use_cells:
            ok &= np.all(np.abs(d) <= 1, axis=1)
        plane = (tb[o, 0] == 3) | (tb[g, 0] == 3)
        diff = (wp[o] - wp[g]).astype(np.float32)
        dsq = (diff[:, 0] * diff[:, 0] + diff[:, 1] * diff[:, 1]) + diff[:, 2] * diff[:, 2]
        md = (ps[g, 3] + ps[o, 3]) + np.float32(0.1)
        ok &= plane | ~(dsq >= md * md)
        sel = np.nonzero(ok)[0]
        keys = sorted(sel, key=lambda i: (d[i, 2], d[i, 1], d[i, 0], o[i]))
        out += [(int(tb[g, 1]), int(tb[o[i], 1]), g, int(o[i])) for i in keys]
    return out


def test_cell_ids_closed_form():
    m, o = _pile()
    pts = [
        ((0.5, 0.5, 0.5), 0),
        ((-0.5, 2.0, 63.5), 0 + 2 * 64 + 63 * 4096),
        ((float("nan"), 5.0, 4.9999995), 0 + 5 * 64 + 4 * 4096),
        ((1e30, -1e30, 62.999996), 63 + 0 + 62 * 4096),
        ((63.0, 64.0, -0.0), 63 + 63 * 64 + 0),
        ((7.25, 1.0 - 2.0 ** -24, 1.0), 7 + 0 * 64 + 1 * 4096),
    ]
    for b, (p, _) in enumerate(pts, start=1):
        o.positions[0, b, :3] = p
    ids, _, _ = O.broad_phase_hash(o, 0)
    for b, (_, want) in enumerate(pts, start=1):
        assert ids[b] == want, (b, ids[b], want)
    assert ids[0] == 0  # the plane at the origin


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_pairs_match_set_definition_and_order(seed):
    m, o = _pile(max_contacts=60000, seed=seed)
    ids, con, n = O.broad_phase_hash(o, 0)
    want = _expected_pairs(m, o.positions[0])
    assert n == len(want) and n < 60000
    got = [tuple(int(v) for v in r) for r in con["indices"][:n]]
    assert got == want
    c = _cells(_geom_world(m, o.positions[0]))
    np.testing.assert_array_equal(ids, c[:, 0] + 64 * c[:, 1] + 4096 * c[:, 2])


def test_non_plane_pairs_equal_quadratic_broad_phase():
    """Inside the grid, two geoms closer than radius_a + radius_b + 0.1 < 1 share a cell
    neighbourhood, so the hash finds exactly the O(G^2) broad phase's non-plane pairs."""
    m, o = _pile(max_contacts=60000, seed=3)
    rng = np.random.default_rng(7)
    o.positions[0, 1:, :2] = rng.uniform(0.0, 9.0, size=(o.B - 1, 2))
    o.positions[0, 1:, 2] = rng.uniform(0.0, 3.0, size=o.B - 1)
    assert float(m["geoms"]["pos_size0"][:, 3][1:].max()) * 2 + 0.1 < 1.0
    _, con, n = O.broad_phase_hash(o, 0)
    tb = m["geoms"]["type_body"]
    hashed = {tuple(int(v) for v in r) for r in con["indices"][:n] if tb[r[2], 0] != 3 and tb[r[3], 0] != 3}
    quad = {p for p in _expected_pairs(m, o.positions[0], use_cells=False) if tb[p[2], 0] != 3 and tb[p[3], 0] != 3}
    assert len(quad) > 20 and hashed == quad


def test_plane_reaches_only_neighbouring_cells():
    m, o = _pile(max_contacts=60000)
    o.positions[0, 1:, :] = 0.0
    o.positions[0, 1:, 0] = np.linspace(30.0, 50.0, o.B - 1)  # far from the plane's cell
    o.positions[0, 1:, 2] = 40.0
    o.positions[0, 1, :3] = (1.5, 1.9, 1.2)   # cell (1, 1, 1): next to the plane's cell 0
    o.positions[0, 2, :3] = (2.0, 0.5, 0.5)   # cell (2, 0, 0): two cells away
    _, con, n = O.broad_phase_hash(o, 0)
    planes = [tuple(int(v) for v in r) for r in con["indices"][:n] if r[2] == 0]
    assert planes == [(0, 1, 0, 1)]


@pytest.mark.parametrize("nb,hashed", [(511, False), (512, True)])
def test_hash_only_above_512_geoms(nb, hashed):
    """World.stepOnce takes the spatial hash only when num_geoms > 512 (world.zig:534). With
    every body far from the plane's cell and from each other, the list broad phase still pairs
    the plane with each of them (planes skip the distance test), the hash with none."""
    m = load_model(mjcf_string=pile_mjcf(nb, seed=0))
    assert m["num_geoms"] == nb + 1
    o = O.OracleWorld(m, 1, max_contacts_per_env=1024)
    o.gravity = [0.0, 0.0, 0.0]
    k = np.arange(nb)
    o.positions[0, 1:, 0] = 30.0 + 1.5 * (k % 8)
    o.positions[0, 1:, 1] = 30.0 + 1.5 * ((k // 8) % 8)
    o.positions[0, 1:, 2] = 40.0 + 1.5 * (k // 64)
    o.velocities[:] = 0.0
    o.angular_velocities[:] = 0.0
    o.step(None)
    assert int(o.contact_counts[0]) == (0 if hashed else nb)


def test_geom_offset_moves_the_cell():
    """A geom's cell is that of its body position plus its offset (all_shaders.metal:574-580)."""
    def edit(m):
        m["geoms"]["pos_size0"][1, :3] = (0.7, -0.2, 1.6)
    m, o = _pile(edit=edit)
    o.positions[0, 1, :3] = (0.5, 0.5, 0.5)
    ids, _, _ = O.broad_phase_hash(o, 0)
    assert ids[1] == 1 + 0 * 64 + 2 * 4096


@pytest.mark.parametrize("seed", [0, 1])
def test_pairs_with_shared_bodies_masks_and_offsets(seed):
    """Geoms moved onto a neighbour's body, given offsets and random contype/conaffinity
    masks: the pairs still follow the set definition (same-body pairs dropped, a pair kept
    when either geom's contype meets the other's conaffinity, positions with offsets)."""
    rng = np.random.default_rng(100 + seed)

    def edit(m):
        tb, ps = m["geoms"]["type_body"], m["geoms"]["pos_size0"]
        G = len(tb)
        share = np.arange(2, G, 3)
        tb[share, 1] = tb[share - 1, 1]
        ps[1:, :3] = rng.uniform(-0.3, 0.3, (G - 1, 3))
        tb[1:, 2] = rng.integers(0, 4, G - 1)
        tb[1:, 3] = rng.integers(0, 4, G - 1)
    m, o = _pile(max_contacts=60000, seed=seed, edit=edit)
    _, con, n = O.broad_phase_hash(o, 0)
    want = _expected_pairs(m, o.positions[0])
    got = [tuple(int(v) for v in r) for r in con["indices"][:n]]
    assert got == want
    tb = m["geoms"]["type_body"]
    same = [(g, x) for g in range(len(tb)) for x in range(g + 1, min(g + 3, len(tb))) if tb[g, 1] == tb[x, 1]]
    assert len(same) > 100 and not any((p[2], p[3]) in set(same) for p in got)
    masked = sum(1 for p in _expected_pairs(m, o.positions[0]) if (tb[p[2], 3] & tb[p[3], 2]) == 0)
    assert masked > 0  # pairs kept through the other direction of the mask rule


def test_count_runs_past_the_list_capacity():
    """The counter takes every pair (atomic add before the capacity check, all_shaders.metal:
    692-698); only the first M are written."""
    _, big = _pile(max_contacts=60000)
    _, full, n_full = O.broad_phase_hash(big, 0)
    _, small = _pile(max_contacts=16)
    _, con, n = O.broad_phase_hash(small, 0)
    assert n == n_full > 16
    np.testing.assert_array_equal(con["indices"][:16], full["indices"][:16])
