"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer (host code only).

The oracle's C source is rebuilt with -fsanitize=address,undefined into a temporary
directory and driven, in a child Python process with the ASan runtime preloaded, through
every entry point the tests use: steps of Ant, Humanoid and the pile (reference and
extended-contact modes), a spatial-hash scene, step_subset, the candidate-pair and hash
broad phases alone and the batched narrow phase. Any sanitizer report fails the test.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

DRIVER = r"""
import numpy as np
from oracle import oracle as O
from oracle.oracle import OracleWorld
from zeno_amd.scenes import workload_inputs

for name, envs, steps, kw in [("ant", 8, 6, {}), ("humanoid", 4, 4, {}), ("pile", 2, 4, {}),
                              ("pile", 2, 4, {"max_contacts_per_env": 512, "extended": True}),
                              ("hash_terrain", 2, 3, {})]:
    path, xml, model, state, acts = workload_inputs(name, envs, steps, 0)
    ext = kw.pop("extended", False)
    o = OracleWorld(model, envs, **kw)
    o.extended_contacts = ext
    o.reset_to_state(*state)
    for k in range(steps):
        o.step(acts[k], nthreads=1)
    mask = np.zeros(envs, np.uint8)
    mask[0] = 1
    o.step_subset(acts[0], mask)
    O.collide_env(o, 0)
    O.broad_phase_hash(o, 0)
    assert np.isfinite(o.positions).all(), name

rng = np.random.default_rng(0)
n = 2000
a = np.zeros(n, O.COLLIDER_DTYPE)
b = np.zeros(n, O.COLLIDER_DTYPE)
for r in (a, b):
    r["type"] = rng.integers(0, 6, n)
    r["size"] = rng.uniform(0.05, 0.6, (n, 3))
    r["position"][:, :3] = rng.uniform(-0.7, 0.7, (n, 3))
    q = rng.normal(size=(n, 4))
    r["quaternion"] = q / np.linalg.norm(q, axis=1, keepdims=True)
O.detect_collisions(a, b)
print("sanitized oracle ok")
"""


def _sanitizer_runtime():
    gcc = shutil.which("gcc")
    if gcc is None:
        return None, None
    asan = subprocess.run([gcc, "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return gcc, asan if asan and Path(asan).exists() else None


def test_oracle_is_clean_under_asan_and_ubsan(tmp_path):
    gcc, asan = _sanitizer_runtime()
    if gcc is None or asan is None:
        pytest.skip("gcc with the ASan runtime is required")
    lib = tmp_path / "libzeno_oracle_asan.so"
    build = subprocess.run(
        [gcc, "-O1", "-g", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
         "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
         str(ROOT / "oracle" / "zeno_oracle.c"), "-o", str(lib), "-lm"],
        capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    env = dict(os.environ, ZENO_ORACLE_LIB=str(lib), LD_PRELOAD=asan,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1",
               PYTHONPATH=str(ROOT))
    run = subprocess.run([sys.executable, "-c", DRIVER], cwd=str(ROOT), env=env, capture_output=True, text=True,
                         timeout=600)
    report = run.stdout + run.stderr
    assert run.returncode == 0 and "sanitized oracle ok" in run.stdout, report[-4000:]
    assert "runtime error" not in report and "AddressSanitizer" not in report, report[-4000:]
