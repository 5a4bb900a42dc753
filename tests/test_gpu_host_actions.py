"""Host-action steps (zeno_world_step) when the host runs ahead of the GPU.

Actions from the host are read by the step kernel in place from a ring of pinned, coherent
buffers; the host refills a buffer only after the steps that read it have finished. Here the
host enqueues many steps with different actions and reads nothing in between, so it runs
ahead and reuses every buffer several times; the result must still match the CPU oracle fed
the same action sequence.
"""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,envs,steps", [("ant", 32, 40), ("pendulum", 256, 60)])
def test_host_actions_running_ahead_match_oracle(name, envs, steps):
    g, o, acts = make_pair(name, envs, steps, seed=21)
    assert len({a.tobytes() for a in acts}) == steps  # every step has its own actions
    for k in range(steps):
        g.step(acts[k])
    for k in range(steps):
        o.step(acts[k])
    compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)


def test_host_steps_and_subset_steps_interleave():
    """zeno_world_step and zeno_world_step_subset both stage host actions through the ring;
    interleaved, they keep its bookkeeping consistent."""
    g, o, acts = make_pair("ant", 16, 24, seed=22)
    mask = (np.arange(16) % 3 != 0).astype(np.uint8)
    for k in range(24):
        if k % 5 == 4:
            g.step_subset(acts[k], mask)
            o.step_subset(acts[k], mask)
        else:
            g.step(acts[k])
            o.step(acts[k])
    compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
