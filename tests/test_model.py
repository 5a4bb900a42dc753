"""Host engine (MJCF parser, joint decomposition, colouring, records) of libzeno, on the CPU.

Pinned by the closed-form fixtures in tests/golden/model_fixtures.json (C1-C4), the
reference's own parser and decomposition tests (test_mjcf.zig, test_physics_integration.zig)
restated as MJCF inputs, and the parser quirks the step depends on (parser.zig:425-432,
851, 910-975, 1229-1243, 1340-1342; world.zig:323, 397-429).
"""
import json
from pathlib import Path

import numpy as np
import pytest

from zeno_amd.model import load_model
from zeno_amd.scenes import ASSETS

GOLD = json.loads((Path(__file__).parent / "golden" / "model_fixtures.json").read_text())


def colour(t):
    return (t["indices"][:, 3] >> 8) & 0xFF


def ctype(t):
    return t["indices"][:, 3] & 0xFF


@pytest.mark.parametrize("name", ["pendulum", "cartpole", "ant", "humanoid"])
def test_counts(name):
    m = load_model(str(ASSETS / f"{name}.xml"))
    for k, v in GOLD[name]["counts"].items():
        assert m[k] == v, (k, m[k], v)


@pytest.mark.parametrize("name", ["pendulum", "cartpole"])
def test_small_scenes_templates(name):
    m = load_model(str(ASSETS / f"{name}.xml"))
    g = GOLD[name]
    jt = m["joints"]
    got_joints = [[int(jt["params"][j, 0]), int(jt["params"][j, 1]), int(jt["params"][j, 2])] for j in range(m["num_joints"])]
    assert got_joints == g["joints"]
    expect = sorted(g["templates_joint_order"], key=lambda r: r[3])  # stable by colour
    t = m["constraints"]
    got = [[int(ctype(t)[i]), int(t["indices"][i, 0]), int(t["indices"][i, 1]), int(colour(t)[i])] for i in range(len(t))]
    assert got == expect
    np.testing.assert_array_equal(m["color_ranges"], g["color_ranges"])


@pytest.mark.parametrize("name", ["ant", "humanoid"])
def test_hinge_triple_colours(name):
    """Fixtures C3/C4: each hinge decomposes to (point, hinge, angular limit) with colours
    base, base+1, base+2; the list is stably sorted by colour."""
    m = load_model(str(ASSETS / f"{name}.xml"))
    g = GOLD[name]
    pre = []
    for a, b, base in g["hinge_triples"]:
        pre += [[2, a, b, base], [3, a, b, base + 1], [4, a, b, base + 2]]
    expect = sorted(pre, key=lambda r: r[3])
    t = m["constraints"]
    got = [[int(ctype(t)[i]), int(t["indices"][i, 0]), int(t["indices"][i, 1]), int(colour(t)[i])] for i in range(len(t))]
    assert got == expect
    np.testing.assert_array_equal(m["color_ranges"][:, 1], g["color_sizes"])
    np.testing.assert_array_equal(m["color_ranges"][:, 0], np.cumsum([0] + g["color_sizes"][:-1]))


def test_pendulum_bodies():
    m = load_model(str(ASSETS / "pendulum.xml"))
    g = GOLD["pendulum"]
    inv = m["inv_mass_inertia"]
    masses = [0.0 if x == 0 else 1.0 / x for x in inv[:, 0]]
    np.testing.assert_allclose(masses, g["masses"], rtol=1e-6)
    np.testing.assert_allclose(1.0 / inv[3, 1:], g["inertia"]["3"], rtol=1e-6)
    assert np.all(inv[1, 1:] == 0)  # base: mass attribute 0 -> mass 1, inertia 0
    np.testing.assert_allclose(m["init_positions"][:, :3], g["init_positions"])


def test_cartpole_bodies():
    m = load_model(str(ASSETS / "cartpole.xml"))
    g = GOLD["cartpole"]
    np.testing.assert_allclose(1.0 / m["inv_mass_inertia"][2, 0], g["masses"][2], rtol=1e-6)
    np.testing.assert_allclose(m["bodies"]["com_offset"][2, :3], g["com"]["2"], rtol=1e-6)
    t = m["constraints"]
    lim = t[ctype(t) == 5]
    np.testing.assert_array_equal(lim["limits"][0, :2], g["linear_limit"])
    assert m["geoms"]["type_body"][1, 2] == 0 and m["geoms"]["type_body"][1, 3] == 0  # rail: no collision


def test_ant_masses_closed_form():
    """Density 5 (the Ant default class): torso sphere r 0.25, legs capsules r 0.08 whose half
    length comes from fromto (0.2*sqrt2/2, 0.4*sqrt2/2)."""
    m = load_model(str(ASSETS / "ant.xml"))
    sphere = 5 * 4 / 3 * np.pi * 0.25 ** 3

    def capsule(length):
        r = 0.08
        return 5 * (np.pi * r * r * length + 4 / 3 * np.pi * r ** 3)

    masses = 1.0 / m["inv_mass_inertia"][1:, 0].astype(np.float64)
    expect = [sphere] + [capsule(0.2 * np.sqrt(2)), capsule(0.4 * np.sqrt(2))] * 4
    np.testing.assert_allclose(masses, expect, rtol=1e-5)
    assert np.all(m["bodies"]["com_offset"][:, :3] == 0)  # COM uses the geom pos attribute (0)


def test_ant_quirks():
    m = load_model(str(ASSETS / "ant.xml"))
    g = GOLD["ant"]
    t = m["constraints"]
    lims = t[ctype(t) == 4]["limits"][:, :2]
    assert any(np.allclose(l, g["ankle_limits_radians"]) for l in lims)  # range used as radians
    np.testing.assert_array_equal(m["actuators"]["params"][:, 0], g["actuator_joints"])
    assert np.all(m["actuators"]["params"][:, 3] == g["actuator_gear"])
    assert np.all(np.isinf(m["actuators"]["params2"][:, :2]))  # force range default +-inf
    caps = m["geoms"][m["geoms"]["type_body"][:, 0] == 1]
    np.testing.assert_array_equal(caps["quat"], np.tile([0, 0, 0, 1], (len(caps), 1)))  # fromto keeps default quat
    s = m["sensors"]
    assert list(s["type_object"][:4, 0]) == [7, 8, 9, 10] and np.all(s["type_object"][:4, 1] == 0)
    assert list(s["params"][:, 3].astype(int)) == [0, 3, 7, 10] + list(range(13, 29))


def test_free_joint_has_no_constraints_and_implicit_fixed_joint():
    xml = """<mujoco><worldbody><body name="a" pos="0 0 1"><joint type="free"/>
    <geom type="sphere" size="0.1"/><body name="b" pos="0.3 0 0"><geom type="sphere" size="0.1"/></body>
    </body></worldbody></mujoco>"""
    m = load_model(mjcf_string=xml)
    jt = m["joints"]
    assert [int(x) for x in jt["params"][:, 0]] == [4, 0]  # free, then the implicit fixed joint
    assert int(jt["params"][1, 1]) == 1 and int(jt["params"][1, 2]) == 2
    np.testing.assert_array_equal(jt["anchor_parent"][1, :3], np.float32([0.3, 0, 0]))
    t = m["constraints"]
    assert list(ctype(t)) == [7]  # only the weld


@pytest.mark.parametrize("jtype,rng,expect", [
    ("hinge", "", [2, 3]), ("hinge", ' range="-1 1"', [2, 3, 4]), ("hinge", ' range="1 -1"', [2, 3]),
    ("hinge", ' range="0.3 0.3"', [2, 3]), ("slide", ' range="0.3 0.3"', [10]), ("ball", ' range="0.5 0.5"', [2]),
    ("slide", "", [10]), ("slide", ' range="-1 1"', [10, 5]),
    ("ball", "", [2]), ("ball", ' range="0 0.5"', [2, 4]), ("free", "", []),
])
def test_decomposition(jtype, rng, expect):
    """test_physics_integration.zig:16-198: revolute -> point + hinge (+ angular limit when
    limited with lower < upper); prismatic -> slider (+ linear limit); ball -> point
    (+ cone limit as a symmetric angular limit); free -> nothing."""
    xml = f"""<mujoco><worldbody><body name="a" pos="0 0 1"><joint type="{jtype}" axis="0 1 0"{rng}/>
    <geom type="sphere" size="0.1"/></body></worldbody></mujoco>"""
    m = load_model(mjcf_string=xml)
    t = m["constraints"]
    assert sorted(ctype(t).tolist()) == sorted(expect)
    if jtype == "ball" and 4 in expect:
        lim = t[ctype(t) == 4]
        np.testing.assert_allclose(lim["limits"][0, :2], [-0.5, 0.5])


def test_mjcf_mass_kats():
    """test_mjcf.zig:395-496"""
    def body_of(xml):
        m = load_model(mjcf_string=xml)
        inv = m["inv_mass_inertia"][1]
        return 1.0 / inv[0], 1.0 / inv[1:]

    mass, inertia = body_of("""<mujoco><worldbody><body name="ball" pos="0 0 1"><joint type="free"/>
        <geom type="sphere" size="0.1" mass="2.5"/></body></worldbody></mujoco>""")
    assert abs(mass - 2.5) < 1e-3 and np.allclose(inertia, 0.01, atol=1e-3)
    mass, _ = body_of("""<mujoco><worldbody><body name="ball" pos="0 0 1"><joint type="free"/>
        <geom type="sphere" size="0.1" density="500"/></body></worldbody></mujoco>""")
    assert abs(mass - 2.094) < 0.05
    mass, inertia = body_of("""<mujoco><worldbody><body name="c" pos="0 0 1"><joint type="free"/>
        <geom type="sphere" size="0.1" mass="1.0" pos="0 0 0"/><geom type="sphere" size="0.1" mass="1.0" pos="0.5 0 0"/>
        </body></worldbody></mujoco>""")
    assert abs(mass - 2.0) < 1e-3 and inertia[1] > inertia[0] and inertia[2] > inertia[0]
    mass, inertia = body_of("""<mujoco><worldbody><body name="b" pos="0 0 1"><joint type="free"/>
        <geom type="box" size="0.5 0.3 0.1" mass="6.0"/></body></worldbody></mujoco>""")
    assert abs(mass - 6.0) < 1e-3
    np.testing.assert_allclose(inertia, [0.2, 0.52, 0.68], atol=0.01)


def test_parser_layout_quirks():
    """Parser quirks (parser.zig:425-427, 910-975, 1340-1342): body positions add without rotating; joint anchor_parent = body.pos +
    joint.pos; quaternions are stored xyzw; the joint axis is not normalised; worldbody
    geoms belong to body 0; geom defaults contype = conaffinity = 1, friction[0] used."""
    xml = """<mujoco><worldbody><geom type="plane" size="1 1 0.1" friction="0.7 0.1 0.1"/>
    <body name="a" pos="1 2 3" quat="0.5 0.5 0.5 0.5"><joint type="hinge" pos="0.1 0 0" axis="0 0 2"/>
    <geom type="sphere" size="0.1"/>
    <body name="b" pos="1 0 0"><joint type="hinge"/><geom type="sphere" size="0.1"/></body></body>
    </worldbody></mujoco>"""
    m = load_model(mjcf_string=xml)
    np.testing.assert_allclose(m["init_positions"][1:, :3], [[1, 2, 3], [2, 2, 3]])
    np.testing.assert_allclose(m["init_quaternions"][1], [0.5, 0.5, 0.5, 0.5])
    jt = m["joints"]
    np.testing.assert_allclose(jt["anchor_parent"][0, :3], [1.1, 2, 3], rtol=1e-6)
    np.testing.assert_allclose(jt["axis"][0, :3], [0, 0, 2])
    g = m["geoms"]
    assert g["type_body"][0, 1] == 0 and g["type_body"][0, 2] == 1 and g["type_body"][0, 3] == 1
    np.testing.assert_allclose(g["params"][0, 2], 0.7)


def test_self_closing_body_swallows_following_content():
    """The reference tokenizer emits only a start token for `<body .../>`, so the body's
    content runs to the next `</body>` (parser.zig:1390-1396)."""
    xml = """<mujoco><worldbody><body name="a" pos="0 0 1"/>
    <body name="b" pos="0 0 2"><geom type="sphere" size="0.1"/></body></body>
    </worldbody></mujoco>"""
    m = load_model(mjcf_string=xml)
    assert m["num_bodies"] == 3
    assert int(m["bodies"]["params"][2, 0]) == 1  # b nests inside a


def test_defaults_class_and_nested_close():
    xml = """<mujoco><default><geom density="7" contype="2" conaffinity="2"/><joint damping="3"/></default>
    <worldbody><body name="a" pos="0 0 1"><joint type="hinge"/><geom type="sphere" size="0.1"/></body>
    </worldbody></mujoco>"""
    m = load_model(mjcf_string=xml)
    assert m["geoms"]["type_body"][0, 2] == 2 and m["geoms"]["type_body"][0, 3] == 2
    np.testing.assert_allclose(1.0 / m["inv_mass_inertia"][1, 0], 7 * 4 / 3 * np.pi * 0.001, rtol=1e-5)
    assert m["joints"]["params2"][0, 1] == 3


def test_auto_sensors_read_body_zero():
    """No <sensor> block: four frame sensors on body 0 plus (pos, vel) per joint."""
    xml = """<mujoco><worldbody>""" + "".join(
        f'<body name="b{i}" pos="{i} 0 1"><joint type="free"/><geom type="box" size="0.1 0.1 0.1"/></body>'
        for i in range(5)) + "</worldbody></mujoco>"
    m = load_model(mjcf_string=xml)
    assert m["obs_dim"] == 13 + 2 * 5
    s = m["sensors"]["type_object"]
    assert list(s[:4, 0]) == [7, 8, 9, 10] and np.all(s[:4, 1] == 0)
    assert list(s[4:, 0]) == [0, 1] * 5


def test_candidate_pairs_filtered():
    """Static broad-phase filters: same-body pairs and contype/conaffinity mismatches are
    dropped; the list stays in (g, g') order."""
    m = load_model(str(ASSETS / "cartpole.xml"))
    pairs = [(int(p) & 0xFFFF, int(p) >> 16) for p in m["pairs"]]
    assert pairs == [(0, 2), (0, 3), (0, 4), (2, 3), (2, 4)]
    m = load_model(str(ASSETS / "ant.xml"))
    assert m["num_pairs"] == 45


def test_unknown_file_and_bad_xml():
    with pytest.raises(RuntimeError):
        load_model("/nonexistent/model.xml")
    m = load_model(mjcf_string="<notmujoco/>")
    assert m["num_bodies"] == 1  # only the world body; no geoms
