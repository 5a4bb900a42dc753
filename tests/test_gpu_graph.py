"""Multi-step HIP-graph replay (zeno_amd_world_capture_steps / zeno_amd_world_graph_launch)
against eager step launches of the same kernel, through the C ABI.

A replay runs the same kernels with the same arguments as eager zeno_amd_world_step_device
calls, so the state after each replay must equal an eager world's state bit for bit. The
graph is replayed several times, with eager work and synchronisations between the replays
(the other world's steps, host reads of the state, an eager step on the captured world), and
every replay is checked. The eager
path itself is pinned against the oracle by the parity tests; one oracle comparison here
ties the multi-substep replay to it directly.
"""
import ctypes as C

import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu

STATE = ("positions", "quaternions", "velocities", "angular_velocities", "accelerations", "joint_positions",
         "joint_velocities", "joint_torques", "observations", "contact_counts", "prev_contact_counts", "lambda")


class DeviceBuffer:
    def __init__(self, host: np.ndarray):
        self.hip = C.CDLL("libamdhip64.so")
        self.ptr = C.c_void_p()
        assert self.hip.hipMalloc(C.byref(self.ptr), C.c_size_t(max(host.nbytes, 4))) == 0
        if host.nbytes:
            assert self.hip.hipMemcpy(self.ptr, C.c_void_p(host.ctypes.data), C.c_size_t(host.nbytes), 1) == 0

    def free(self):
        self.hip.hipFree(self.ptr)


def assert_same_state(a, b, what):
    ga, gb = gpu_arrays(a), gpu_arrays(b)
    for f in STATE:
        np.testing.assert_array_equal(np.asarray(ga[f]), np.asarray(gb[f]), err_msg=f"{what}: {f}")
    M = ga["contacts"].shape[1]
    live = np.arange(M)[None, :] < np.minimum(ga["contact_counts"], M)[:, None]
    assert ga["contacts"][live].tobytes() == gb["contacts"][live].tobytes(), f"{what}: contacts"


@pytest.mark.parametrize("name,envs,steps,substeps", [("ant", 64, 12, 1), ("humanoid", 32, 8, 2),
                                                      ("pile", 16, 10, 1)])
def test_graph_replays_match_eager_steps(name, envs, steps, substeps):
    eager, _, acts = make_pair(name, envs, 3 * steps, seed=11)
    graph, _, _ = make_pair(name, envs, 3 * steps, seed=11)
    A = eager.action_dim
    flat = np.ascontiguousarray(acts[:steps], np.float32).reshape(-1)
    buf = DeviceBuffer(flat)
    stride = envs * A * 4
    try:
        graph.capture_steps(buf.ptr.value, stride, steps, substeps)
        for replay in range(3):
            graph.graph_launch()
            for k in range(steps):
                eager.step_device(buf.ptr.value + k * stride if A else 0, substeps)
            graph.synchronize()
            eager.synchronize()
            assert_same_state(graph, eager, f"replay {replay}")
            if replay == 1:  # eager work on the captured world between replays
                eager.step(acts[steps + 1], substeps)
                graph.step(acts[steps + 1], substeps)
                assert_same_state(graph, eager, "eager step between replays")
    finally:
        graph.release_graph()
        buf.free()


def test_multi_substep_replay_matches_oracle():
    g, o, acts = make_pair("ant", 16, 6, seed=12)
    flat = np.ascontiguousarray(acts, np.float32).reshape(-1)
    buf = DeviceBuffer(flat)
    try:
        g.capture_steps(buf.ptr.value, 16 * g.action_dim * 4, 6, 3)
        g.graph_launch()
        g.synchronize()
        for k in range(6):
            o.step(acts[k], substeps=3)
        compare(gpu_arrays(g), oracle_arrays(o), rtol=1e-4, atol=1e-4)
    finally:
        g.release_graph()
        buf.free()


def test_setters_release_the_graph():
    g, _, acts = make_pair("pendulum", 8, 2, seed=13)
    buf = DeviceBuffer(np.ascontiguousarray(acts, np.float32).reshape(-1))
    try:
        for setter in (lambda: g.set_gravity((0.0, 0.0, -9.0)), lambda: g.set_timestep(0.01),
                       lambda: g.set_extended_contacts(True)):
            g.capture_steps(buf.ptr.value, 8 * g.action_dim * 4, 2)
            g.graph_launch()
            setter()
            with pytest.raises(RuntimeError):
                g.graph_launch()
        g.synchronize()
        assert np.isfinite(g.get_body_positions(zero_copy=False)).all()
    finally:
        buf.free()
