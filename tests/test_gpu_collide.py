"""Extended narrow phase on the GPU (zeno_amd_detect_collisions) against the CPU oracle.

Every (type_a, type_b) combination of sphere, capsule, box, plane, cylinder and mesh, with
random sizes, poses and local offsets, plus degenerate cases (coincident centres, a sphere
centre inside a box, zero-length and parallel capsules, parallel box edges). Results are
compared bit for bit: the kernel and the oracle evaluate the same fp32 operations in the
same order.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from zeno_amd import _lib as L
from zeno_amd import collision as Z

pytestmark = pytest.mark.gpu


def random_colliders(rng, n, types):
    r = np.zeros(n, Z.COLLIDER_DTYPE)
    r["type"] = types
    r["size"] = rng.uniform(0.05, 0.6, (n, 3))
    r["local_pos"][:, :3] = rng.uniform(-0.2, 0.2, (n, 3)) * (rng.random((n, 1)) < 0.5)
    r["position"][:, :3] = rng.uniform(-0.7, 0.7, (n, 3))
    q = rng.normal(size=(n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    ident = rng.random(n) < 0.2  # some axis-aligned operands (parallel edges, face contacts)
    q[ident] = (0, 0, 0, 1)
    r["quaternion"] = q
    return r


def assert_bitwise(gpu, ref):
    g, o = gpu.view(np.uint32).reshape(len(gpu), -1), ref.view(np.uint32).reshape(len(ref), -1)
    bad = np.nonzero((g != o).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} pairs differ, first {bad[:5]}: gpu {gpu[bad[0]]} oracle {ref[bad[0]]}"


def test_all_type_pairs_bitwise():
    rng = np.random.default_rng(0)
    per = 600
    ta, tb = np.meshgrid(np.arange(6), np.arange(6), indexing="ij")
    ta, tb = np.repeat(ta.ravel(), per), np.repeat(tb.ravel(), per)
    a, b = random_colliders(rng, ta.size, ta), random_colliders(rng, tb.size, tb)
    gpu = Z.detect_collisions(a, b)
    ref = O.detect_collisions(a, b)
    assert_bitwise(gpu, ref)
    hits = {(i, j): int(gpu["valid"][(ta == i) & (tb == j)].sum()) for i in range(4) for j in range(4)}
    handled = [(0, 0), (0, 1), (0, 2), (0, 3), (1, 0), (1, 1), (1, 3), (2, 0), (2, 2), (2, 3), (3, 0), (3, 1), (3, 2)]
    assert all(hits[p] > 20 for p in handled), hits
    assert hits[(1, 2)] == hits[(2, 1)] == hits[(3, 3)] == 0
    assert gpu["valid"][(ta >= 4) | (tb >= 4)].sum() == 0


def test_shuffled_mixed_batch_bitwise():
    """Every type pair (heightfield included) in random order, so that each 256-pair block
    holds most classes and the kernel's in-block grouping by type pair reorders nearly every
    pair; 20,001 pairs end in a partial block."""
    rng = np.random.default_rng(7)
    n = 20001
    ta, tb = rng.integers(0, 7, n), rng.integers(0, 7, n)
    a, b = random_colliders(rng, n, ta), random_colliders(rng, n, tb)
    gpu = Z.detect_collisions(a, b)
    assert_bitwise(gpu, O.detect_collisions(a, b))
    assert gpu["valid"].sum() > 1000
    assert gpu["valid"][(ta >= 4) | (tb >= 4)].sum() == 0


def test_degenerate_cases_bitwise():
    cases = []

    def pair(ka, sa, pa, kb, sb, pb, qa=(0, 0, 0, 1), qb=(0, 0, 0, 1)):
        a = Z.collider(Z.Geom(ka, size=sa), Z.Transform(pa, qa))
        b = Z.collider(Z.Geom(kb, size=sb), Z.Transform(pb, qb))
        cases.append((a, b))

    pair("sphere", (0.5, 0, 0), (0, 0, 0), "sphere", (0.5, 0, 0), (0, 0, 0))          # coincident
    pair("sphere", (0.2, 0, 0), (0.1, 0, 0), "box", (1, 1, 1), (0, 0, 0))             # centre inside box
    pair("sphere", (0.2, 0, 0), (0, 0, 0), "box", (1, 1, 1), (0, 0, 0))               # centre at box centre
    pair("capsule", (0.2, 0, 0), (0, 0, 0), "capsule", (0.2, 0, 0), (0.1, 0, 0))      # zero-length segments
    pair("capsule", (0.2, 1, 0), (0, 0, 0), "capsule", (0.2, 1, 0), (0.3, 0, 0.5))    # parallel (denom 0)
    pair("capsule", (0.2, 0, 0), (0, 0, 0), "capsule", (0.2, 1, 0), (0.3, 0, 0.5))    # one degenerate
    pair("box", (0.5, 0.5, 0.5), (0, 0, 0), "box", (0.5, 0.5, 0.5), (0.9, 0.1, 0))    # parallel edges
    pair("box", (0.5, 0.5, 0.5), (0, 0, 0), "plane", (0.0, 0, 0), (0, 0, 0.2))         # plane above centre
    pair("sphere", (0.3, 0, 0), (0, 0, 0.25), "capsule", (0.1, 0.5, 0), (0, 0, 0))    # on the axis
    a = np.stack([c[0] for c in cases]).astype(Z.COLLIDER_DTYPE)
    b = np.stack([c[1] for c in cases]).astype(Z.COLLIDER_DTYPE)
    gpu, ref = Z.detect_collisions(a, b), O.detect_collisions(a, b)
    assert_bitwise(gpu, ref)
    assert gpu["valid"].all()


def test_reference_kats_through_the_single_pair_api():
    """tests/test_collision.zig:54-80 and 173-199 through detect_collision."""
    t0 = Z.Transform((0, 0, 0), (0, 0, 0, 1))
    r = Z.detect_collision(Z.Geom.sphere(0.5), t0, Z.Geom.sphere(0.5), Z.Transform((0.8, 0, 0)))
    assert r is not None and abs(r.penetration - 0.2) < 0.01 and abs(r.normal[0] - 1.0) < 0.01
    assert Z.detect_collision(Z.Geom.sphere(0.5), t0, Z.Geom.sphere(0.5), Z.Transform((2.0, 0, 0))) is None
    r = Z.detect_collision(Z.Geom.sphere(0.5), Z.Transform((0, 0, 0.3)), Z.Geom.plane((0, 0, 1), 0.0), t0)
    assert r is not None and abs(r.penetration - 0.2) < 0.01
    assert Z.detect_collision(Z.Geom.sphere(0.5), Z.Transform((0, 0, 1.0)), Z.Geom.plane((0, 0, 1), 0.0), t0) is None


def test_device_pointer_entry_point():
    """zeno_amd_detect_collisions on device buffers (hipMalloc through libamdhip64)."""
    rng = np.random.default_rng(1)
    n = 5000
    types = rng.integers(0, 4, n)
    a, b = random_colliders(rng, n, types), random_colliders(rng, n, rng.integers(0, 4, n))
    hip = C.CDLL("libamdhip64.so")
    ptrs = []
    try:
        for arr in (a, b, np.zeros(n, Z.CONTACT_RESULT_DTYPE)):
            p = C.c_void_p()
            assert hip.hipMalloc(C.byref(p), C.c_size_t(arr.nbytes)) == 0
            assert hip.hipMemcpy(p, arr.ctypes.data_as(C.c_void_p), C.c_size_t(arr.nbytes), 1) == 0
            ptrs.append(p)
        lib = L.load()
        assert lib.zeno_amd_detect_collisions(ptrs[0], ptrs[1], n, ptrs[2], None) == 0
        out = np.zeros(n, Z.CONTACT_RESULT_DTYPE)
        assert hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), ptrs[2], C.c_size_t(out.nbytes), 2) == 0
    finally:
        for p in ptrs:
            hip.hipFree(p)
    assert_bitwise(out, O.detect_collisions(a, b))
