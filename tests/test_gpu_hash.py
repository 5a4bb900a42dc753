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
