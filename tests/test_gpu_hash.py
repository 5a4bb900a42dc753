"""Spatial-hash broad phase (scenes above 512 geoms, world.zig:534) and working sets in HBM,
on the GPU against the CPU oracle through the C ABI.

hash_terrain (521 geoms, 9 bodies) runs the hash with its working set in LDS; pile_hash
(601 geoms and bodies) is too large for LDS and runs the hash with its working set in HBM.
Ant and Humanoid forced into HBM working sets check that path against the LDS one's
oracle. Discrete outputs, including each geom's hash cell, are bit-exact; fp32 state
within the contact-rich tolerance of the other multi-step tests.
"""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,envs,steps,hbm", [("hash_terrain", 16, 40, False), ("pile_hash", 8, 12, True)])
def test_spatial_hash_parity(name, envs, steps, hbm):
    g, o, acts = make_pair(name, envs, steps, seed=3)
    assert g.modes() == {"hbm": hbm, "spatial_hash": True}
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


@pytest.mark.parametrize("name,envs,steps", [("ant", 16, 20), ("humanoid", 8, 20), ("pile", 4, 10)])
def test_hbm_working_set_parity(name, envs, steps):
    g, o, acts = make_pair(name, envs, steps, seed=9, working_set="hbm")
    assert g.modes() == {"hbm": True, "spatial_hash": False}
    assert g.launch_config() == (1, 0)
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
