"""Contact lists of any length (src/physics/state.zig:64-97 allocates num_envs x
max_contacts_per_env for whatever the caller asks; main.zig:79,160), on the GPU against the
CPU oracle through the C ABI:

* the 601-body spatial-hash pile at max_contacts_per_env = 1024: the working set and the
  per-body slot masks (601 x 1024 bits) live in HBM, the contact records in LDS, and lists
  above 512 slots (8 per lane) are sorted by the bitonic network;
* Ant at 512 contacts per environment, with one environment per wave (the shape the world
  picks) and with two (32 lanes, so lists above 256 slots take the bitonic sort); Ant's list
  grows by 13 candidate pairs per substep and fills after 40 steps;
* lists too long for any LDS layout (2,048 slots: 128 KB of records alone, ~104 B per slot
  with the snapshot and sort keys): the world falls back to placement 3, the whole working set
  in HBM, for the hash pile and for Ant (filled after 158 steps);
* placement 3 forced on scenes that fit LDS, with and without the spatial hash and the
  extended-contact mode.

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


@pytest.mark.parametrize("extended", [False, True])
def test_hash_pile_2048_contacts_in_hbm(extended):
    g, o, acts = make_pair("pile_hash", 2, 24, seed=13, max_contacts=2048, extended_contacts=extended)
    assert g.modes()["placement"] == 3 and g.launch_config()[1] == 0
    tol = dict(rtol=1e-4, atol=1e-4) if extended else dict(rtol=1e-5, atol=1e-6)
    for k in range(24):
        g.step(acts[k])
        o.step(acts[k])
        if k % 4 == 3:
            compare(gpu_arrays(g), oracle_arrays(o), **tol)
    assert o.contact_counts.min() > 1024  # 80-95 pairs per step
    if extended:  # box and capsule pairs make contacts only in the extended mode
        live = live_mask(o.contact_counts, 2048)
        assert ((o.contacts["position_pen"][..., 3] >= 0) & live).sum() > 0
    # the shapes that did not fit left no error behind for the next world
    g2, o2, acts2 = make_pair("pile", 2, 1, seed=7)
    g2.step(acts2[0])
    o2.step(acts2[0])
    compare(gpu_arrays(g2), oracle_arrays(o2), rtol=1e-5, atol=1e-6)


def test_ant_2048_contacts_in_hbm():
    g, o, acts = make_pair("ant", 3, 162, seed=14, max_contacts=2048)
    assert g.modes()["placement"] == 3
    for k in range(162):
        g.step(acts[k])
        o.step(acts[k])
        if k % 20 == 19 or k > 155:
            compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    assert o.contact_counts.min() >= 2048
    np.testing.assert_array_equal(g.get_contact_counts(), o.contact_counts)


@pytest.mark.parametrize("name,envs,steps,M,extended", [("ant", 5, 12, 64, False), ("pile", 3, 6, 128, False),
                                                        ("pile", 3, 6, 512, True), ("pile_hash", 2, 4, 256, False),
                                                        ("humanoid", 3, 8, 64, False)])
def test_forced_placement_3(name, envs, steps, M, extended):
    g, o, acts = make_pair(name, envs, steps, seed=15, max_contacts=M, placement=3, extended_contacts=extended)
    assert g.modes()["placement"] == 3
    tol = dict(rtol=1e-4, atol=1e-4) if extended else dict(rtol=1e-5, atol=1e-6)
    for k in range(steps):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), **tol)
