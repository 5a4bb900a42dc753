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
