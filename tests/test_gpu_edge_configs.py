"""World configurations at the edges of ZenoConfig, GPU against the oracle bit for bit:
an empty or one-slot contact list (the count still grows, main.zig:79 takes any
max_contacts_per_env), list lengths that are no multiple of a wave's lanes, zero, one and
many solver iterations (contact_iterations drives both the joint and the contact loops,
world.zig:1163-1213), and several substeps per call."""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,envs,M,iters,substeps", [
    ("ant", 6, 0, 4, 1),
    ("ant", 6, 1, 4, 1),
    ("ant", 9, 13, 1, 1),
    ("ant", 6, 64, 0, 1),
    ("humanoid", 5, 37, 7, 3),
    ("pendulum", 7, 3, 2, 2),
    ("pile", 3, 5, 4, 1),
])
def test_edge_config_matches_oracle(name, envs, M, iters, substeps):
    g, o, acts = make_pair(name, envs, 10, seed=2, max_contacts=M, contact_iterations=iters,
                           substeps=substeps)
    assert g.max_contacts_per_env == M
    for k in range(10):
        g.step(acts[k])
        o.step(acts[k])
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    assert np.isfinite(g.get_body_positions(zero_copy=False)).all()
