"""The contact count is a u32 that no step clears (all_shaders.metal:765-766 compare the raw
count against slot ids). After 2^32 appends it wraps, the broad phase's appends restart at slot
0, and the sort (:711-745, over min(count, M) entries every step) must order them again. The
counts are set just below 2^32 on the GPU (zeno_amd_world_set_contact_counts) and in the CPU
oracle, and every following step is compared with the oracle; one environment stays short of
the wrap as a control.
"""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu

BELOW_WRAP = [1, 3, 7, 12, 20, 40, 64, 5000]


@pytest.mark.parametrize("name,envs", [("ant", 8), ("pile", 4), ("humanoid", 8)])
def test_count_wrap_matches_oracle(name, envs):
    g, o, acts = make_pair(name, envs, 12, seed=21)
    for k in range(6):
        g.step(acts[k])
        o.step(acts[k])
    compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    near = (np.uint64(1 << 32) - np.array(BELOW_WRAP[-envs:], np.uint64)).astype(np.uint32)
    g.set_contact_counts(near)
    o.contact_counts[:] = near
    np.testing.assert_array_equal(g.get_contact_counts(), near)
    for k in range(6, 12):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    wrapped = o.contact_counts < near
    assert wrapped.any() and not wrapped.all()


def _pair_from_mjcf(xml, envs):
    from oracle.oracle import OracleWorld
    from zeno_amd.model import load_model
    from zeno_amd.world import ZenoWorld
    m = load_model(mjcf_string=xml)
    return m, ZenoWorld(mjcf_string=xml, num_envs=envs), OracleWorld(m, envs)


def test_wrap_with_appends_out_of_key_order():
    """A body with two geoms makes the broad phase append pairs out of key order
    (tests/test_count_wrap.py shows the oracle's list after the wrap then differs from the
    append order): with the count 1-6 appends below 2^32, the wrapped appends must be sorted."""
    from tests.test_count_wrap import WITH_PLANE
    m, g, o = _pair_from_mjcf(WITH_PLANE, 6)
    near = (np.uint64(1 << 32) - np.arange(1, 7, dtype=np.uint64)).astype(np.uint32)
    g.set_contact_counts(near)
    o.contact_counts[:] = near
    for _ in range(3):
        g.step(np.zeros((6, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)
    assert np.all(o.contact_counts < near)
    g.close()


def test_host_count_exposes_stale_slots():
    """Slots a reset left behind, exposed again by a count the host sets on a step with no
    appends: the step sorts them as the reference does (tests/test_count_wrap.py builds the
    same sequence on the oracle and shows the exposed list is out of order)."""
    from tests.test_count_wrap import NO_PLANE, stale_slot_sequence
    m, g, o = _pair_from_mjcf(NO_PLANE, 2)

    def step():
        g.step(np.zeros((2, 0), np.float32))
        o.step(None)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-5, atol=1e-6)

    def reset_to_state(p, q):
        g.reset_to_state(p, q)
        o.reset_to_state(p, q)

    def set_counts(c):
        g.set_contact_counts(c)
        o.contact_counts[:] = c

    stale_slot_sequence(2, m, reset_to_state, set_counts, step)
    np.testing.assert_array_equal(g.get_contact_counts(), [5, 5])
    g.close()
