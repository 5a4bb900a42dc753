"""The benchmark configurations at their full sizes (Pendulum and Cartpole 1024 envs, Ant 4096,
Humanoid 16384, the 64-body pile 8192), HIP step against the multithreaded CPU oracle on the
same inputs, also at their benchmark lengths (1000 steps, the pile's 500), plus the
size-independent invariants of the step over longer runs:
unit quaternions, finite state, an untouched world body, the world-body observation
constants, and never-decreasing contact counts (the step appends and never clears them)."""
import numpy as np
import pytest

from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name,envs,steps", [
    ("pendulum", 1024, 1000), ("cartpole", 1024, 1000), ("ant", 4096, 200),
    ("humanoid", 16384, 50), ("pile", 8192, 30)])
def test_full_size_parity(name, envs, steps):
    g, o, acts = make_pair(name, envs, steps, seed=101)
    for k in range(steps):
        g.step(acts[k])
        o.step(acts[k])
    diffs = compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    print(name, envs, steps, "max |diff|:", {k: v for k, v in diffs.items() if v})
    g.close()


@pytest.mark.parametrize("name,envs,steps", [("ant", 4096, 300), ("humanoid", 16384, 100)])
def test_full_size_invariants(name, envs, steps):
    g, _o, acts = make_pair(name, envs, steps, seed=202)
    p0 = g.get_body_positions(zero_copy=False)
    counts_prev = g.get_contact_counts().copy()
    for k in range(steps):
        g.step(acts[k])
        if k % 25 == 24 or k == steps - 1:
            q = g.get_body_quaternions(zero_copy=False)
            p = g.get_body_positions(zero_copy=False)
            assert np.all(np.isfinite(p)) and np.all(np.isfinite(q))
            assert np.max(np.abs(np.linalg.norm(q[:, 1:], axis=-1) - 1)) < 1e-5
            np.testing.assert_array_equal(p[:, 0], p0[:, 0])
            obs = g.get_observations(zero_copy=False)
            # Frame sensors read body 0: position 0, identity quaternion, zero velocities.
            np.testing.assert_array_equal(obs[:, :13], np.tile([0, 0, 0, 0, 0, 0, 1] + [0] * 6, (envs, 1)))
            c = g.get_contact_counts()
            assert np.all(c >= counts_prev)
            counts_prev = c.copy()
    g.close()


@pytest.mark.parametrize("name,envs,steps", [("ant", 4096, 1000), ("humanoid", 16384, 1000), ("pile", 8192, 500)])
def test_benchmark_length_parity(name, envs, steps):
    """The configurations at their benchmark lengths (Ant 4096 x 1000 steps, Humanoid 16384 x
    1000, the pile 8192 x 500), bit for bit against the oracle at four points along the run.
    The first 100 steps' action rows are used over and over (the same rows on both sides)."""
    g, o, acts = make_pair(name, envs, 100, seed=303)
    for k in range(steps):
        g.step(acts[k % 100])
        o.step(acts[k % 100])
        if (k + 1) % (steps // 4) == 0:
            compare(gpu_arrays(g), oracle_arrays(o), **TOL)
    assert np.all(np.isfinite(g.get_body_positions(zero_copy=False)))
    g.close()
