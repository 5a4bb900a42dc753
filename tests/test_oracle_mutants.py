"""Mutation check of the oracle pins: each plausible misreading of the contact solve, the
lambda warm start and the accelerometer / gyro sensors, planted in a copy of the oracle's C
source, must make tests/test_contact_solve.py fail.

Each mutant is compiled into a temporary directory and the pin tests run in a child pytest
with ZENO_ORACLE_LIB pointing at it. The unmutated copy must pass the same run, so a failure
is the mutation's doing.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "oracle" / "zeno_oracle.c"
PINS = "tests/test_contact_solve.py"

# (name, original text, mutated text); the original must occur exactly once in the source.
MUTANTS = [
    ("friction sign of body a",
     "st3(Va, vsub(ld3(Va), vscale(impulse_t, inv_mass_a)));",
     "st3(Va, vadd(ld3(Va), vscale(impulse_t, inv_mass_a)));"),
    ("friction sign of body b",
     "st3(Vb, vadd(ld3(Vb), vscale(impulse_t, inv_mass_b)));",
     "st3(Vb, vsub(ld3(Vb), vscale(impulse_t, inv_mass_b)));"),
    ("friction cone clamp min -> max",
     "float j_t = fminf(j_t_desired, j_t_max);",
     "float j_t = fmaxf(j_t_desired, j_t_max);"),
    ("friction cone without the stored impulse",
     "float j_n_acc = e->con[s].impulses[0] + j_n;",
     "float j_n_acc = j_n;"),
    ("stored impulse is the running sum",
     "    e->con[s].impulses[0] = j_n;\n}",
     "    e->con[s].impulses[0] = j_n_acc;\n}"),
    ("restitution threshold sign",
     "float vel_restitution = vel_normal < -0.5f ? restitution * vel_normal : 0.0f;",
     "float vel_restitution = vel_normal > -0.5f ? restitution * vel_normal : 0.0f;"),
    ("restitution dropped",
     "float j_n = (-(vel_normal + vel_restitution) + bias) / w_normal;",
     "float j_n = (-(vel_normal) + bias) / w_normal;"),
    ("warm start factor 0.8 -> 0.5",
     "e->cs[i].state[0] = 0.8f * e->cs[i].state[1];",
     "e->cs[i].state[0] = 0.5f * e->cs[i].state[1];"),
    ("accelerometer rotates by q instead of its conjugate",
     "v3 lg = qrot(V(m->gravity[0], m->gravity[1], m->gravity[2]), qconj(q));",
     "v3 lg = qrot(V(m->gravity[0], m->gravity[1], m->gravity[2]), q);"),
    ("gyro reads the linear velocity",
     "case 3: case 10: { const float* w = P4(e->angvel, obj);",
     "case 3: case 10: { const float* w = P4(e->vel, obj);"),
]


def _build(src_text: str, out: Path) -> None:
    gcc = shutil.which("gcc")
    c = out.with_suffix(".c")
    c.write_text(src_text)
    shutil.copy(ROOT / "oracle" / "zeno_oracle.h", out.parent / "zeno_oracle.h")
    r = subprocess.run([gcc, "-O1", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
                        str(c), "-o", str(out), "-lm"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def _run_pins(lib: Path) -> subprocess.CompletedProcess:
    env = dict(os.environ, ZENO_ORACLE_LIB=str(lib), PYTHONPATH=str(ROOT))
    return subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", PINS],
                          cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=300)


@pytest.fixture(scope="module")
def source():
    if shutil.which("gcc") is None:
        pytest.skip("gcc is required")
    return SRC.read_text()


def test_unmutated_copy_passes(source, tmp_path):
    lib = tmp_path / "oracle_ref.so"
    _build(source, lib)
    r = _run_pins(lib)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]


@pytest.mark.parametrize("name,orig,mut", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_mutant_is_caught(source, tmp_path, name, orig, mut):
    assert source.count(orig) == 1, f"mutation site for '{name}' not found exactly once"
    lib = tmp_path / "oracle_mut.so"
    _build(source.replace(orig, mut), lib)
    r = _run_pins(lib)
    assert r.returncode != 0, f"mutant '{name}' passed every pin test"
    assert "failed" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
