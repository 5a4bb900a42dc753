"""The host-side scene code (MJCF parser, model builder: zeno_amd/csrc/mjcf.cpp, model.cpp)
under AddressSanitizer and UndefinedBehaviorSanitizer.

A small driver, compiled here with g++ -fsanitize=address,undefined together with those two
files, parses and builds every asset the library ships, generated piles (with and without
the spatial hash) and a set of malformed documents. The reference's parser is lenient (its
InvalidXml error is declared but never returned, mjcf/parser.zig:12-19), so those may parse or
be rejected; they must not crash. Any sanitizer report or crash fails the test. Host code
only: nothing here touches a GPU.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

from zeno_amd.scenes import pile_mjcf, terrain_mjcf

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "zeno_amd" / "csrc"

DRIVER = r"""
#include <cstdio>
#include <string>
#include "model.h"
#include "scene.h"

int main(int argc, char** argv) {
    int built = 0, rejected = 0;
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        const bool malformed = arg.rfind("bad:", 0) == 0;
        const std::string path = malformed ? arg.substr(4) : arg;
        za::Scene scene;
        const za::ParseResult r = za::parse_mjcf_file(path, scene);
        if (r.error != 0) {
            if (!malformed) { std::fprintf(stderr, "unexpected parse error in %s: %s\n", path.c_str(), r.message.c_str()); return 2; }
            ++rejected;
            continue;
        }
        za::Model m;
        za::build_model(scene, m);
        if (!malformed && m.num_bodies < 2) { std::fprintf(stderr, "empty model from %s\n", path.c_str()); return 3; }
        ++built;
    }
    std::printf("built %d rejected %d\n", built, rejected);
    return 0;
}
"""

MALFORMED = [
    "<mujoco><worldbody><body name='a'><geom type='sphere' size='0.1'/></worldbody></mujoco>",  # unclosed body
    "<mujoco><worldbody><geom type='sphere' size='abc'/></worldbody></mujoco>",
    "<mujoco><worldbody>",
    "",
    "<mujoco><worldbody><body><joint type='hinge' axis='0 0'/><geom size='0.1'/></body></worldbody></mujoco>",
]


def test_parser_and_model_builder_are_clean_under_asan_and_ubsan(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is required")
    (tmp_path / "driver.cpp").write_text(DRIVER)
    exe = tmp_path / "scene_driver"
    build = subprocess.run(
        [gxx, "-O1", "-g", "-std=c++17", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=all", "-I", str(CSRC), str(CSRC / "mjcf.cpp"), str(CSRC / "model.cpp"),
         str(tmp_path / "driver.cpp"), "-o", str(exe)],
        capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-4000:]
    inputs = sorted(str(p) for p in (ROOT / "zeno_amd" / "assets").glob("*.xml"))
    for name, xml in [("pile64.xml", pile_mjcf(64, seed=1)), ("pile600.xml", pile_mjcf(600, seed=2, xy=(-3.0, 13.0))),
                      ("terrain.xml", terrain_mjcf(8, seed=3))]:
        (tmp_path / name).write_text(xml)
        inputs.append(str(tmp_path / name))
    for i, xml in enumerate(MALFORMED):
        (tmp_path / f"bad{i}.xml").write_text(xml)
        inputs.append("bad:" + str(tmp_path / f"bad{i}.xml"))
    run = subprocess.run([str(exe), *inputs], capture_output=True, text=True, timeout=600,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    report = run.stdout + run.stderr
    assert run.returncode == 0, report[-4000:]
    assert "runtime error" not in report and "AddressSanitizer" not in report, report[-4000:]
    built, rejected = (int(w) for w in run.stdout.split()[1::2])
    assert built + rejected == len(inputs) and built >= len(inputs) - len(MALFORMED), report[-2000:]
