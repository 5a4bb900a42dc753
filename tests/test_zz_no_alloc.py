"""zeno_amd_detect_collisions_host_noalloc (static device staging, no allocation) against
zeno_amd_detect_collisions_host (per-call device buffers), through the C ABI: bit-identical
results on two calls in a row, the second with fewer pairs, and a clear error above the
array's limit."""
import ctypes as C

import numpy as np
import pytest

from zeno_amd import _lib as L
from zeno_amd.collision import COLLIDER_DTYPE, CONTACT_RESULT_DTYPE

pytestmark = pytest.mark.gpu

MAX_PAIRS = 16384
ZENO_INVALID_ARGUMENT = -6


def _pairs(n: int, seed: int):
    """Sphere / capsule / box / plane on both sides, sizes U[0.05, 0.6], positions
    U[-0.7, 0.7]^3 (about a third of the pairs touch), random rotations."""
    rng = np.random.default_rng(seed)
    sides = []
    for _ in range(2):
        r = np.zeros(n, COLLIDER_DTYPE)
        r["type"] = rng.integers(0, 4, n)
        r["size"] = rng.uniform(0.05, 0.6, (n, 3))
        r["position"][:, :3] = rng.uniform(-0.7, 0.7, (n, 3))
        q = rng.normal(size=(n, 4))
        r["quaternion"] = q / np.linalg.norm(q, axis=1, keepdims=True)
        sides.append(r)
    return sides


def _call(fn, a, b, n, out):
    return fn(a.ctypes.data_as(C.c_void_p), b.ctypes.data_as(C.c_void_p), n, out.ctypes.data_as(C.c_void_p))


def test_no_alloc_matches_allocating_entry_point():
    lib = L.load()
    for n, seed in ((MAX_PAIRS, 1), (2999, 2)):
        print(f"no-alloc collide: n={n} seed={seed}", flush=True)
        a, b = _pairs(n, seed)
        want = np.zeros(n, CONTACT_RESULT_DTYPE)
        assert _call(lib.zeno_amd_detect_collisions_host, a, b, n, want) == 0
        # one spare record past n: the entry point must write exactly n results
        got = np.zeros(n + 1, CONTACT_RESULT_DTYPE)
        got.view(np.uint8)[:] = 0xAB
        sentinel = got[n:].copy()
        assert _call(lib.zeno_amd_detect_collisions_host_noalloc, a, b, n, got) == 0
        assert got[:n].tobytes() == want.tobytes()
        assert got[n:].tobytes() == sentinel.tobytes()
        assert want["valid"].sum() > n // 10  # the batch exercises contacts, not only misses


def test_no_alloc_rejects_batches_above_its_limit():
    lib = L.load()
    n = MAX_PAIRS + 1
    a, b = _pairs(n, 3)
    out = np.zeros(n, CONTACT_RESULT_DTYPE)
    assert _call(lib.zeno_amd_detect_collisions_host_noalloc, a, b, n, out) == ZENO_INVALID_ARGUMENT
    assert "16384" in L.last_error()
    assert not out.view(np.uint8).any()
    assert _call(lib.zeno_amd_detect_collisions_host_noalloc, a, b, 0, out) == 0


def test_concurrent_calls_take_turns():
    """Two host threads call the entry point at once on the one GPU with different batches;
    the per-device lock makes each call's copy in, launch and copy back one unit, so every
    result equals the allocating entry point's (ctypes drops the GIL during the calls)."""
    import threading
    lib = L.load()
    batches = [_pairs(n, seed) for n, seed in ((9000, 4), (12000, 5))]
    wants = []
    for a, b in batches:
        w = np.zeros(len(a), CONTACT_RESULT_DTYPE)
        assert _call(lib.zeno_amd_detect_collisions_host, a, b, len(a), w) == 0
        wants.append(w)
    errors = []

    def worker(i):
        a, b = batches[i]
        for rep in range(20):
            got = np.zeros(len(a), CONTACT_RESULT_DTYPE)
            rc = _call(lib.zeno_amd_detect_collisions_host_noalloc, a, b, len(a), got)
            if rc != 0 or got.tobytes() != wants[i].tobytes():
                errors.append((i, rep, rc))
                return

    print("no-alloc collide: two threads x 20 calls", flush=True)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
