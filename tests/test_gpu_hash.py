"""Spatial-hash broad phase (scenes above 512 geoms, world.zig:534) and working sets in HBM,
on the GPU against the CPU oracle through the C ABI.

hash_terrain (521 geoms, 9 bodies) runs the hash with the model records and its working
set in LDS; pile_hash (601 geoms and bodies) reads its model records from HBM with the
working set in LDS, and is also forced to keep the working set in HBM. Ant, Humanoid and
the 64-body pile forced into each larger-scene placement check those paths. Discrete outputs, including each geom's hash cell, are bit-exact; fp32 state
within the contact-rich tolerance of the other multi-step tests.
"""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,envs,steps,force,placement", [("hash_terrain", 16, 40, None, 0),
                                                              ("pile_hash", 8, 12, None, 1),
                                                              ("pile_hash", 4, 6, 2, 2)])
def test_spatial_hash_parity(name, envs, steps, force, placement):
    g, o, acts = make_pair(name, envs, steps, seed=3, placement=force)
    assert g.modes() == {"placement": placement, "spatial_hash": True}
    G = g.num_geoms
    worst = {}
    for k in range(steps):
        g.step(acts[k])
        o.step(acts[k])
        d = compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
        np.testing.assert_array_equal(g.get_cell_ids(), o.cell_ids[:, :G], err_msg=f"cell ids, step {k}")
        for f, v in d.items():
            worst[f] = max(worst.get(f, 0.0), v)
    assert (o.contact_counts > 0).mean() > 0.5  # most envs have pairs (plane or neighbours)
    print(name, "worst |diff| over", steps, "steps:", worst)


@pytest.mark.parametrize("placement", [1, 2])
@pytest.mark.parametrize("name,envs,steps", [("ant", 16, 20), ("humanoid", 8, 20), ("pile", 4, 10)])
def test_placement_parity(name, envs, steps, placement):
    g, o, acts = make_pair(name, envs, steps, seed=9, placement=placement)
    assert g.modes() == {"placement": placement, "spatial_hash": False}
    epw, lds = g.launch_config()
    assert epw == 1 and lds > 0
    for k in range(steps):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)


def test_cell_ids_need_the_hash():
    g, _, _ = make_pair("ant", 2, 1)
    assert g.modes()["spatial_hash"] is False
    with pytest.raises(RuntimeError):
        g.get_cell_ids()


@pytest.mark.parametrize("num_bodies", [512, 1023, 1024, 1500])
def test_hash_key_sort_sizes(num_bodies):
    """The sort of the hash keys at the sizes that change its form: 513 geoms (the smallest
    scene hashed, padded to 1024 keys), 1024 (every one of the 1024 places a real key), 1025
    (padded to 2048: the network runs in LDS instead of registers) and 1501. Piles of that
    many bodies at the 601-body pile's density, every step against the oracle, cell ids
    included."""
    from oracle.oracle import OracleWorld
    from zeno_amd.model import load_model
    from zeno_amd.scenes import pile_initial_state, pile_mjcf
    from zeno_amd.world import ZenoWorld
    side = 16.0 * np.sqrt(num_bodies / 600.0)
    xy = (-3.0, -3.0 + side)
    xml = pile_mjcf(num_bodies, seed=num_bodies, xy=xy)
    m = load_model(mjcf_string=xml)
    assert m["num_geoms"] == num_bodies + 1
    g = ZenoWorld(mjcf_string=xml, num_envs=3)
    o = OracleWorld(m, 3)
    assert g.modes()["spatial_hash"]
    state = pile_initial_state(m, 3, num_bodies + 1, xy=xy)
    g.reset_to_state(*state)
    o.reset_to_state(*state)
    G = m["num_geoms"]
    for k in range(5):
        g.step(np.zeros((3, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
        np.testing.assert_array_equal(g.get_cell_ids(), o.cell_ids[:, :G], err_msg=f"cell ids, step {k}")
    assert (o.contact_counts > 0).all()
    g.close()


def _filtered_pile(num_bodies: int, classes: str) -> str:
    """The hash pile with a contype / conaffinity pair on every body's geom: "few" draws them
    from three contypes and two conaffinities (six classes, with pairs the filter rejects, the
    plane's too), "many" from nine and five (45 classes, more than the model's class rows
    hold, so the queries read both geoms' masks from the records)."""
    from zeno_amd.scenes import pile_mjcf
    lines = pile_mjcf(num_bodies, seed=7, xy=(-3.0, 13.0)).split("\n")
    out, i = [], 0
    for ln in lines:
        if "<geom" in ln and "plane" not in ln:
            ct, ca = (1 << (i % 3), 1 << ((i // 3) % 2)) if classes == "few" else (1 + i % 9, 1 + (i // 9) % 5)
            ln = ln.replace("<geom ", f'<geom contype="{ct}" conaffinity="{ca}" ')
            i += 1
        out.append(ln)
    assert i == num_bodies
    return "\n".join(out)


@pytest.mark.parametrize("classes", ["few", "many"])
@pytest.mark.parametrize("placement", [None, 2, 3])
def test_hash_filter_classes(classes, placement):
    """The hash queries' contype / conaffinity filter (:493-522) through the model's class rows
    (six classes) and through the records (45 classes), with the working set in LDS, in HBM
    with the compact LDS arrays, and all in HBM: every step against the oracle, cell ids
    included."""
    import os
    from oracle.oracle import OracleWorld
    from zeno_amd.model import load_model
    from zeno_amd.scenes import pile_initial_state
    from zeno_amd.world import ZenoWorld
    xml = _filtered_pile(600, classes)
    m = load_model(mjcf_string=xml)
    E = 3
    saved = os.environ.get("ZENO_AMD_PLACEMENT")
    if placement is not None:
        os.environ["ZENO_AMD_PLACEMENT"] = str(placement)
    try:
        g = ZenoWorld(mjcf_string=xml, num_envs=E)
    finally:
        os.environ.pop("ZENO_AMD_PLACEMENT", None)
        if saved is not None:
            os.environ["ZENO_AMD_PLACEMENT"] = saved
    assert g.modes()["spatial_hash"]
    if placement is not None:
        assert g.modes()["placement"] == placement
    o = OracleWorld(m, E)
    state = pile_initial_state(m, E, 11, xy=(-3.0, 13.0))
    g.reset_to_state(*state)
    o.reset_to_state(*state)
    G = m["num_geoms"]
    for k in range(6):
        g.step(np.zeros((E, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
        np.testing.assert_array_equal(g.get_cell_ids(), o.cell_ids[:, :G], err_msg=f"cell ids, step {k}")
    assert (o.contact_counts > 0).all()
    g.close()


@pytest.mark.parametrize("placement", [None, 2])
def test_hash_snapshot_after_count_changes(placement):
    """The previous-contact snapshot when the counts drop between calls: after a reset (every
    count to 0, the previous list kept, world.zig:1296-1314) and after the host lowers some
    counts, the first substep's appends land on slots of the previous list. With the working
    set in HBM the snapshot is taken after the broad phase, from the call's list as loaded;
    the cache matching must still see the previous list. Every step against the oracle."""
    g, o, acts = make_pair("pile_hash", 4, 16, seed=13, placement=placement)
    if placement is not None:
        assert g.modes()["placement"] == placement
    for k in range(5):
        g.step(acts[k])
        o.step(acts[k])
    assert np.all(o.contact_counts >= 64)
    g.reset()
    o.reset()
    for k in range(5, 9):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    counts = o.contact_counts.copy()
    counts[0] = 0
    counts[1] = 10
    counts[2] = counts[2] // 2
    g.set_contact_counts(counts)
    o.contact_counts[:] = counts
    for k in range(9, 13):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    g.close()


@pytest.mark.parametrize("placement", [None, 2, 3])
def test_hash_count_wrap(placement):
    """Counts just below 2^32 on the hash pile: a substep's appends wrap the count and land on
    the list's first slots (slots compare against the raw count, :765-766), which still hold
    the previous list when the snapshot for the cache matching is taken. Every step against
    the oracle, with the working set in LDS, in HBM with the compact LDS arrays, and all in
    HBM."""
    g, o, acts = make_pair("pile_hash", 4, 8, seed=17, placement=placement)
    if placement is not None:
        assert g.modes()["placement"] == placement
    for k in range(2):
        g.step(acts[k])
        o.step(acts[k])
    near = np.array([(1 << 32) - 5, (1 << 32) - 60, (1 << 32) - 150, (1 << 32) - 250], np.uint64).astype(np.uint32)
    g.set_contact_counts(near)
    o.contact_counts[:] = near
    for k in range(2, 8):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    assert np.all(o.contact_counts < (1 << 20))  # every count wrapped
    g.close()
