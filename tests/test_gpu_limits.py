"""Angular limits whose bounds lie beyond +-2 pi can never act: the limit angle is 2 atan2(...)
(all_shaders.metal:1206), within +-2 fp32(pi) for every input, so the violation stays 0 and the
solve writes nothing (:1216). The reference's parser keeps MJCF ranges in degrees as given, so
most hinge limits of the assets are of that kind (ant.xml's hips: -30..30). The joint program
leaves them out; the CPU oracle still evaluates every limit, and the GPU parity tests (all ten
assets in tests/test_gpu_api.py, the benchmark configurations at full size in
tests/test_gpu_full_size.py) compare the two bit for bit. Here: the phase counts the program is
left with, and parity on the assets that lose phases."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.parity import compare, gpu_arrays, make_pair, oracle_arrays
from zeno_amd.model import load_model
from zeno_amd.scenes import ASSETS
from zeno_amd.world import ZenoWorld

TWO_PI_F = np.float32(6.28318548)
ORDER = [2, 7, 3, 4, 5, 10]  # positional, weld, angular, angular limit, linear limit, slider


def expected_phases(m):
    """Same-type runs of each colour, without the constraints that can never act."""
    c, invmi = m["constraints"], m["inv_mass_inertia"]
    n = 0
    for off, cnt in m["color_ranges"]:
        for ty in ORDER:
            k_live = 0
            for k in range(off, off + cnt):
                ia, ib, _, t = (int(x) for x in c[k]["indices"])
                if (t & 0xFF) != ty:
                    continue
                if invmi[ia][0] + invmi[ib][0] < np.float32(1e-8):
                    continue
                lo, hi = np.float32(c[k]["limits"][0]), np.float32(c[k]["limits"][1])
                if ty == 4 and lo <= -TWO_PI_F and hi >= TWO_PI_F:
                    continue
                k_live += 1
            n += k_live > 0
    return n


def test_atan2_range_premise():
    """The oracle's atan2 (the reference's, restated) never exceeds fp32(pi) in magnitude."""
    rng = np.random.default_rng(5)
    vals = [0.0, -0.0, 1e-45, -1e-45, 1e-30, -1e-30, 1.0, -1.0, 3.4e38, -3.4e38, np.inf, -np.inf]
    ys = list(vals) + list(rng.standard_normal(300) * 10.0 ** rng.integers(-8, 8, 300))
    xs = list(vals) + list(rng.standard_normal(300) * 10.0 ** rng.integers(-8, 8, 300))
    worst = 0.0
    for y in ys[:60]:
        for x in xs[:60]:
            worst = max(worst, abs(np.float32(O.atan2f(float(np.float32(y)), float(np.float32(x))))))
    for y, x in zip(ys, xs):
        worst = max(worst, abs(np.float32(O.atan2f(float(np.float32(y)), float(np.float32(x))))))
    assert worst <= np.float32(np.pi)
    assert np.float32(2.0) * np.float32(np.pi) == TWO_PI_F


@pytest.mark.gpu
@pytest.mark.parametrize("asset,dropped", [("ant", 4), ("humanoid", 11), ("cheetah", 4), ("hopper", 2),
                                           ("walker", 4), ("swimmer", 4), ("reacher", 0), ("pusher", 0)])
def test_joint_phases_leave_out_unreachable_limits(asset, dropped):
    m = load_model(str(ASSETS / f"{asset}.xml"))
    c = m["constraints"]
    lim = [k for k in range(len(c)) if (int(c[k]["indices"][3]) & 0xFF) == 4]
    unreachable = [k for k in lim if np.float32(c[k]["limits"][0]) <= -TWO_PI_F and np.float32(c[k]["limits"][1]) >= TWO_PI_F]
    assert len(unreachable) == dropped
    w = ZenoWorld(mjcf_path=str(ASSETS / f"{asset}.xml"), num_envs=4)
    try:
        assert w.joint_phases() == expected_phases(m)
    finally:
        w.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["ant", "humanoid"])
def test_parity_without_unreachable_limits(name):
    """The benchmark workloads (seeded perturbed starts, random actions) for 40 steps: the GPU
    program without the unreachable limits against the oracle that evaluates them."""
    g, o, acts = make_pair(name, 9, 40, seed=23)
    for k in range(40):
        g.step(acts[k])
        o.step(acts[k])
    compare(gpu_arrays(g), oracle_arrays(o), rtol=0, atol=0)
    g.close()
