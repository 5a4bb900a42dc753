"""Extended-contact mode of the step on the GPU against the CPU oracle, through the C ABI
(zeno_amd_world_set_extended_contacts). The pile's box and capsule pairs go through
narrow_phase.detectCollision in both; discrete outputs are bit-exact and fp32 state within
the contact-rich tolerance of the other multi-step tests.
"""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu


# One environment per workgroup with M >= 64 runs the narrow phase grouped by geom-type pair
# (every placement, with and without the hash, is covered below); Ant at four environments
# per wave runs it ungrouped.
@pytest.mark.parametrize("name,envs,steps,M,placement,epw", [("pile", 8, 12, 512, None, None),
                                                             ("pile", 4, 8, 512, 2, None),
                                                             ("pile", 4, 8, 512, 0, 1),
                                                             ("pile_hash", 4, 6, 512, None, None),
                                                             ("pile_hash", 2, 4, 512, 2, None),
                                                             ("ant", 16, 20, 128, None, 1),
                                                             ("ant", 16, 20, 64, None, None)])
def test_extended_contacts_parity(name, envs, steps, M, placement, epw):
    g, o, acts = make_pair(name, envs, steps, seed=5, max_contacts=M, placement=placement,
                           envs_per_wave=epw, extended_contacts=True)
    active = 0
    for k in range(steps):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
        live = np.arange(M)[None, :] < np.minimum(o.contact_counts, M)[:, None]
        active += int(((o.contacts["position_pen"][..., 3] >= 0) & live).sum())
    if name != "ant":
        assert active > 0


def test_mode_is_off_by_default_and_switchable():
    g, o, acts = make_pair("pile", 2, 2, seed=6, max_contacts=512)
    g.step(acts[0])
    o.step(acts[0])
    compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    g.set_extended_contacts(True)
    o.extended_contacts = True
    g.step(acts[1])
    o.step(acts[1])
    compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)


def test_extended_mode_switches_to_the_grouped_shape_and_back():
    """A placement-0 world with a long contact list runs the extended mode in the
    one-environment-per-wave shape without split groups (the type-grouped narrow phase) and
    returns to its creation-time shape when the mode is turned off; both stay on the oracle."""
    g, o, acts = make_pair("pile", 24, 6, seed=8, max_contacts=512)
    if g.modes()["placement"] != 0:
        pytest.skip("the world placed this scene outside LDS")
    base = (g.launch_config()[0], g.waves_per_group(), g.split_groups())
    g.set_extended_contacts(True)
    o.extended_contacts = True
    assert g.launch_config()[0] == 1 and not g.split_groups()
    for k in range(3):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    g.set_extended_contacts(False)
    o.extended_contacts = False
    assert (g.launch_config()[0], g.waves_per_group(), g.split_groups()) == base
    for k in range(3, 6):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
