"""Contact lists of any length that fits a workgroup's LDS (src/physics/state.zig:64-97
allocates num_envs x max_contacts_per_env for whatever the caller asks), on the GPU against
the CPU oracle through the C ABI:

* the 601-body spatial-hash pile at max_contacts_per_env = 1024: the working set and the
  per-body slot masks (601 x 1024 bits) live in HBM, the contact records in LDS, and lists
  above 512 slots (8 per lane) are sorted by the bitonic network;
* Ant at 512 contacts per environment, with one environment per wave (the shape the world
  picks) and with two (32 lanes, so lists above 256 slots take the bitonic sort); Ant's list
  grows by 13 candidate pairs per substep and fills after 40 steps.

Discrete outputs (counts, pair lists after the sort, active flags) are compared exactly and
fp32 state within 1e-5 rel / 1e-6 abs (reference mode) or the contact-rich tolerance of the
extended mode.
"""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, live_mask, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("extended", [False, True])
def test_hash_pile_1024_contacts(extended):
    g, o, acts = make_pair("pile_hash", 2, 8, seed=11, max_contacts=1024, extended_contacts=extended)
    assert g.modes()["placement"] == 2
    tol = dict(rtol=1e-4, atol=1e-4) if extended else dict(rtol=1e-5, atol=1e-6)
    for k in range(8):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), **tol)
    assert o.contact_counts.min() > 512  # the bitonic path ran
    live = live_mask(o.contact_counts, 1024)
    assert ((o.contacts["position_pen"][..., 3] >= 0) & live).sum() > 0


@pytest.mark.parametrize("epw", [None, 2])
def test_ant_512_contacts(epw):
    g, o, acts = make_pair("ant", 4, 44, seed=12, max_contacts=512, envs_per_wave=epw)
    if epw is not None:
        assert g.launch_config()[0] == epw
    for k in range(44):
        g.step(acts[k])
        o.step(acts[k])
        if k % 4 == 3 or k > 38:
            compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    assert o.contact_counts.min() >= 512
    np.testing.assert_array_equal(g.get_contact_counts(), o.contact_counts)
