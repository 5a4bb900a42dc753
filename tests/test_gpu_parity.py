"""HIP step vs CPU oracle on identical seeded inputs, through the C ABI.

Discrete outputs (contact counts, sorted pair lists, active flags, previous counts) must be
bit-exact. fp32 state must agree within 1e-5 relative / 1e-6 absolute after one step; the
kernels and the oracle evaluate the same expressions in the same order without FMA
contraction, so in practice they agree bitwise and the tests also record that.
Long runs: Pendulum and Cartpole 1000 steps within 1e-3; Ant and Humanoid are chaotic, so
they are held to one-step parity plus invariants over long runs.
"""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu

ONE_STEP = dict(rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name,envs", [("pendulum", 64), ("cartpole", 64), ("ant", 64), ("humanoid", 32), ("pile", 8)])
def test_one_step_parity(name, envs):
    g, o, acts = make_pair(name, envs, 1, seed=3)
    g.step(acts[0])
    o.step(acts[0])
    diffs = compare(gpu_arrays(g), oracle_arrays(o), **ONE_STEP)
    print(name, "max |diff| per field:", diffs)


@pytest.mark.parametrize("name,envs,steps", [("pendulum", 32, 1000), ("cartpole", 32, 1000)])
def test_long_run_smooth(name, envs, steps):
    g, o, acts = make_pair(name, envs, steps, seed=5)
    for k in range(steps):
        g.step(acts[k])
        o.step(acts[k])
    diffs = compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-3, atol=1e-3)
    print(name, steps, "steps, max |diff|:", diffs)


@pytest.mark.parametrize("name,envs,steps", [("ant", 16, 50), ("humanoid", 8, 50), ("pile", 4, 30)])
def test_multi_step_contacts(name, envs, steps):
    """Contact-rich stretch (ground contact, saturated lists, warm starts): every step checked."""
    g, o, acts = make_pair(name, envs, steps, seed=7)
    worst = {}
    for k in range(steps):
        g.step(acts[k])
        o.step(acts[k])
        d = compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
        for f, v in d.items():
            worst[f] = max(worst.get(f, 0.0), v)
    print(name, "worst |diff| over", steps, "steps:", worst)


@pytest.mark.parametrize("epw", [1, 2, 4, 8])
def test_launch_shapes_agree(epw):
    """Every environments-per-wave instantiation gives the oracle's result."""
    g, o, acts = make_pair("ant", 24, 8, seed=11, envs_per_wave=epw)
    assert g.launch_config()[0] == epw
    for k in range(8):
        g.step(acts[k])
        o.step(acts[k])
    compare(gpu_arrays(g), oracle_arrays(o), **ONE_STEP)


@pytest.mark.parametrize("name,envs,epw,waves", [("ant", 37, 4, 4), ("ant", 20, 2, 2), ("humanoid", 21, 4, 4),
                                                ("pendulum", 9, 1, 4)])
def test_multi_wave_workgroups_agree(name, envs, epw, waves):
    """Workgroups of several waves sharing one copy of the model records: each wave steps its
    own environments; env counts that leave the last workgroup partly empty included."""
    g, o, acts = make_pair(name, envs, 6, seed=17, envs_per_wave=epw, waves=waves)
    assert g.launch_config()[0] == epw and g.waves_per_group() == waves
    for k in range(6):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), **ONE_STEP)


@pytest.mark.parametrize("name,envs,epw,waves,substeps", [("ant", 37, 4, 4, 1), ("ant", 20, 2, 2, 1),
                                                          ("humanoid", 21, 4, 4, 1), ("pendulum", 9, 1, 4, 1),
                                                          ("cartpole", 13, 2, 4, 3), ("pile", 5, 1, 2, 2)])
def test_split_groups_agree(name, envs, epw, waves, substeps):
    """Two waves per environment group: the helper runs the snapshot, broad phase, sort,
    narrow phase, matching and levels on the poses after integration while the solver runs the
    joints, and writes the contact list back; several substeps (three barriers each) and env
    counts that leave the last workgroup partly empty included."""
    g, o, acts = make_pair(name, envs, 6, seed=23, envs_per_wave=epw, waves=waves, split=True, substeps=substeps)
    assert g.launch_config()[0] == epw and g.waves_per_group() == waves and g.split_groups()
    for k in range(6):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), **ONE_STEP)


def test_split_groups_subset_and_extended_contacts():
    """Split groups with a step subset (the helper records the advanced contact list of the
    environments not stepped) and with the extended-contact narrow phase."""
    g, o, acts = make_pair("ant", 12, 4, seed=29, envs_per_wave=4, waves=2, split=True, extended_contacts=True)
    assert g.split_groups()
    mask = (np.arange(12) % 3 != 0).astype(np.uint8)
    for k in range(4):
        g.step_subset(acts[k], mask) if k % 2 else g.step(acts[k])
        o.step_subset(acts[k], mask) if k % 2 else o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("waves", [2, 4])
def test_grouped_narrow_phase_multi_wave(waves):
    """Extended-contact mode at one environment per wave launches the narrow-phase instance
    that visits slots grouped by geom-type pair; with several waves per workgroup every wave
    steps its own environment (11 envs: the last workgroup partly empty)."""
    g, o, acts = make_pair("ant", 11, 6, seed=19, envs_per_wave=1, waves=waves, extended_contacts=True)
    assert g.launch_config()[0] == 1 and g.waves_per_group() == waves
    for k in range(6):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    assert np.all(g.get_contact_counts() > 0)


def test_substeps_parity():
    g, o, acts = make_pair("cartpole", 16, 5, seed=13, substeps=3)
    for k in range(5):
        g.step(acts[k])
        o.step(acts[k])
    compare(gpu_arrays(g), oracle_arrays(o), **ONE_STEP)
