"""Pins the oracle's contact solve (solve_contact, all_shaders.metal:1644-1793), its lambda
warm start (:1408-1444) and its accelerometer / gyro sensors (:1838-1858) with physical
laws and closed forms, not by restating the code.

One slot is solved through the oracle's single-slot hook (zo_solve_contact_slot). The cases
put each contact point on the line through the body centres along the normal (r parallel
to n) and give every dynamic body an isotropic inverse inertia s. Then the normal impulse
turns no body, and a tangential impulse j along t (t perpendicular to r) changes the relative
tangential velocity of the contact points by exactly -j (w_a + w_b) t with
w = inv_m + s |r|^2. The laws checked:

  normal impulse     the relative normal velocity after the slot is the Baumgarte bias
                     velocity beta * max(pen - slop, 0) / dt (or stays put when separating)
  restitution        approaching faster than 0.5 m/s: v_n' = -e v_n (+ bias)
  stick (large mu)   the relative tangential velocity of the contact points goes to zero
  slip (small mu)    the tangential impulse is mu * (stored impulse + this slot's normal
                     impulse) and opposes the tangential velocity
  both bodies        linear momentum is conserved; the stored impulse is this slot's own
                     normal impulse m * dv_n, not a running sum
  warm start         a point constraint that is already satisfied keeps lambda = 0.8 of the
                     previous step's value (0.8, 0.64, ... of the closed form -C m)
  accelerometer      gravity expressed in the body frame (R^T g) of a body turned 90 degrees
  gyro               the body's angular velocity
"""
import numpy as np
import pytest

from oracle import oracle as O
from zeno_amd.model import load_model

BETA, SLOP, DT = 0.2, 0.005, 0.01
C_POSITIONAL = 2


def _bodies(specs):
    """specs: list of (inv_mass, s, pos, vel, angvel) per body -> the four [B, 4] arrays."""
    B = len(specs)
    imi = np.zeros((B, 4), np.float32)
    pos, vel, ang = (np.zeros((B, 4), np.float32) for _ in range(3))
    for i, (im, s, p, v, w) in enumerate(specs):
        imi[i] = [im, s, s, s]
        pos[i, :3], vel[i, :3], ang[i, :3] = p, v, w
    return imi, pos, vel, ang


def _contact(a, b, point, normal, pen, mu, jn_prev=0.0, restitution=0.0):
    c = np.zeros(1, O.CONTACT_DTYPE)
    c["position_pen"][0] = [*point, pen]
    c["normal_friction"][0] = [*normal, mu]
    c["indices"][0] = [a, b, 0, 0]
    c["impulses"][0] = [jn_prev, 0.0, 0.0, restitution]
    return c


def _point_velocity(pos, vel, ang, b, point):
    r = np.asarray(point, np.float64) - pos[b, :3].astype(np.float64)
    return vel[b, :3].astype(np.float64) + np.cross(ang[b, :3].astype(np.float64), r)


def _ground_case(v, w=(0.0, 0.0, 0.0), mu=1.0, pen=0.0, jn_prev=0.0, restitution=0.0):
    """Sphere (body 1: m 2, s 125, radius 0.1) on the static body 0; the contact point is
    straight below its centre and the normal +z pushes the sphere (body a) up."""
    imi, pos, vel, ang = _bodies([(0.0, 0.0, (0, 0, 0), (0, 0, 0), (0, 0, 0)),
                                  (0.5, 125.0, (0, 0, 0.1 - pen), v, w)])
    point = (0.0, 0.0, -pen / 2)
    c = _contact(1, 0, point, (0, 0, 1), pen, mu, jn_prev, restitution)
    before = (pos.copy(), vel.copy(), ang.copy())
    O.solve_contact_slot(imi, pos, vel, ang, c, BETA, SLOP, DT)
    return before, (pos, vel, ang), c, point


def _rel(state, point, a=1, b=0, levers=None):
    """Relative velocity of the contact points of bodies a and b. The solve forms its levers
    r = point - centre from the positions it starts from (the position correction moves the
    centres afterwards), so `levers` passes those positions."""
    pos, vel, ang = state
    if levers is not None:
        pos = levers
    return _point_velocity(pos, vel, ang, a, point) - _point_velocity(pos, vel, ang, b, point)


@pytest.mark.parametrize("pen", [0.0, 0.003, 0.02])
def test_normal_impulse_reaches_bias_velocity(pen):
    before, after, c, point = _ground_case(v=(0.0, 0.0, -0.3), pen=pen)
    bias = BETA * max(pen - SLOP, 0.0) / DT
    vn = _rel(after, point)[2]
    np.testing.assert_allclose(vn, bias, atol=1e-5)
    # the stored impulse is the momentum the slot gave the sphere (m = 2)
    np.testing.assert_allclose(c["impulses"][0, 0], 2.0 * (after[1][1, 2] - before[1][1, 2]), rtol=1e-5)


def test_separating_contact_gets_no_impulse():
    before, after, c, _ = _ground_case(v=(0.2, 0.0, 1.0), mu=1.0)
    assert c["impulses"][0, 0] == 0.0
    np.testing.assert_array_equal(after[1], before[1])
    np.testing.assert_array_equal(after[2], before[2])


@pytest.mark.parametrize("e", [0.0, 0.5, 1.0])
@pytest.mark.parametrize("vn", [-2.0, -0.3])
def test_restitution_law(e, vn):
    """Below -0.5 m/s the sphere bounces with v_n' = -e v_n; slower approaches stop (v_n' = 0)."""
    _, after, _, point = _ground_case(v=(0.0, 0.0, vn), restitution=e)
    want = -e * vn if vn < -0.5 else 0.0
    np.testing.assert_allclose(_rel(after, point)[2], want, atol=1e-5)


def test_friction_sticks_with_large_mu():
    before, after, c, point = _ground_case(v=(1.0, -0.5, -0.2), w=(0.3, 0.2, 0.1), mu=10.0)
    vt0 = _rel(before, point)[:2]
    assert np.linalg.norm(vt0) > 0.5
    np.testing.assert_allclose(_rel(after, point)[:2], [0.0, 0.0], atol=1e-5)


def test_friction_slips_with_small_mu():
    mu, jn_prev = 0.1, 0.25
    before, after, c, point = _ground_case(v=(1.0, -0.5, -0.2), w=(0.3, 0.2, 0.1), mu=mu, jn_prev=jn_prev)
    t = _rel(before, point).copy()
    t[2] = 0.0
    t /= np.linalg.norm(t)
    j_n = float(c["impulses"][0, 0])
    assert j_n > 0
    dv = after[1][1, :3].astype(np.float64) - before[1][1, :3]
    # linear velocity change along t: -mu * (jn_prev + j_n) / m, and nothing across t
    np.testing.assert_allclose(np.dot(dv, t), -mu * (jn_prev + j_n) * 0.5, rtol=1e-5)
    across = dv - np.dot(dv, t) * t
    np.testing.assert_allclose(across[:2], [0.0, 0.0], atol=1e-6)
    # the slip leaves tangential speed in the original direction
    vt1 = _rel(after, point)
    assert np.dot(vt1, t) > 0


def test_friction_uses_the_stored_impulse_when_the_slot_adds_none():
    """At the bias velocity the slot's own normal impulse is 0, yet friction still acts with
    mu * impulses.x, and the slot then stores 0 (the last impulse, not a sum)."""
    mu, jn_prev = 0.2, 0.5
    before, after, c, point = _ground_case(v=(0.4, 0.0, 0.0), mu=mu, jn_prev=jn_prev)
    assert c["impulses"][0, 0] == 0.0
    dvx = float(after[1][1, 0]) - float(before[1][1, 0])
    np.testing.assert_allclose(dvx, -mu * jn_prev * 0.5, rtol=1e-5)


def _pair_case(va, vb, mu, wa=(0, 0, 0), wb=(0, 0, 0), jn_prev=0.0):
    """Two dynamic spheres (m 2 and 3, radius 0.1, s 125 and 80), b stacked on a with 0.01
    overlap; the normal -z points from b to a."""
    imi, pos, vel, ang = _bodies([(0.0, 0.0, (0, 0, 0), (0, 0, 0), (0, 0, 0)),
                                  (0.5, 125.0, (0, 0, 0.1), va, wa),
                                  (1 / 3, 80.0, (0, 0, 0.29), vb, wb)])
    point = (0.0, 0.0, 0.195)
    c = _contact(1, 2, point, (0, 0, -1), 0.01, mu, jn_prev)
    before = (pos.copy(), vel.copy(), ang.copy())
    O.solve_contact_slot(imi, pos, vel, ang, c, BETA, SLOP, DT)
    return before, (pos, vel, ang), c, point


@pytest.mark.parametrize("mu", [0.05, 10.0])
def test_two_bodies_conserve_momentum(mu):
    before, after, c, point = _pair_case((0.5, 0.0, 1.0), (-0.3, 0.2, -1.0), mu, wa=(0.1, -0.2, 0.3))
    m = np.array([0.0, 2.0, 3.0])
    p0 = (m[:, None] * before[1][:, :3]).sum(0)
    p1 = (m[:, None] * after[1][:, :3].astype(np.float64)).sum(0)
    np.testing.assert_allclose(p1, p0, atol=1e-5)
    # normal: relative normal velocity reaches the bias velocity beta (pen - slop) / dt
    bias = BETA * (0.01 - SLOP) / DT
    np.testing.assert_allclose(np.dot(_rel(after, point, 1, 2, levers=before[0]), [0, 0, -1]), bias, atol=1e-5)
    # the stored impulse is body a's normal momentum change
    np.testing.assert_allclose(c["impulses"][0, 0], -2.0 * (after[1][1, 2] - before[1][1, 2]), rtol=1e-5)


def test_two_bodies_stick_and_slip():
    va, vb = (0.5, 0.0, 1.0), (-0.3, 0.2, -1.0)
    before, after, _, point = _pair_case(va, vb, 10.0)
    assert np.linalg.norm(_rel(before, point, 1, 2)[:2]) > 0.5
    np.testing.assert_allclose(_rel(after, point, 1, 2, levers=before[0])[:2], [0.0, 0.0], atol=1e-5)
    before, after, c, point = _pair_case(va, vb, 0.05, jn_prev=0.1)
    t = _rel(before, point, 1, 2).copy()
    t[2] = 0.0
    t /= np.linalg.norm(t)
    jt = 0.05 * (0.1 + float(c["impulses"][0, 0]))
    dva = after[1][1, :3].astype(np.float64) - before[1][1, :3]
    dvb = after[1][2, :3].astype(np.float64) - before[1][2, :3]
    np.testing.assert_allclose(np.dot(dva, t), -jt * 0.5, rtol=1e-5)
    np.testing.assert_allclose(np.dot(dvb, t), +jt / 3, rtol=1e-5)


BALL_ON_WORLD = """<mujoco><option timestep="0.01"/><worldbody>
<body name="b" pos="0 0 1"><joint type="ball"/><geom type="sphere" size="0.1" mass="2"/></body>
</worldbody></mujoco>"""


def test_warm_start_lambda_closed_form():
    """Ball joint to the world, anchor at the body's centre, no gravity. Moved 0.3 off its
    anchor, the body is pulled back in the first iteration with lambda = -C / w = -0.3 * 2;
    with the velocities then zeroed, every later step finds the constraint satisfied and
    only the warm start acts: lambda_k = 0.8^(k-1) lambda_1."""
    m = load_model(mjcf_string=BALL_ON_WORLD)
    w = O.OracleWorld(m, 1)
    w.gravity = [0.0, 0.0, 0.0]
    k = int(np.flatnonzero((m["constraints"]["indices"][:, 3] & 0xFF) == C_POSITIONAL)[0])
    p = w.positions.copy()
    p[0, 1, 0] += 0.3
    w.reset_to_state(p, w.quaternions.copy())
    lams = []
    for _ in range(4):
        w.step(None)
        lams.append(float(w.lambdas()[0, k]))
        np.testing.assert_allclose(w.positions[0, 1, :3], [0, 0, 1], atol=1e-6)
        w.velocities[:] = 0
        w.angular_velocities[:] = 0
    np.testing.assert_allclose(lams[0], -0.6, rtol=1e-6)
    np.testing.assert_allclose(lams[1:], [-0.6 * 0.8, -0.6 * 0.64, -0.6 * 0.512], rtol=1e-6)


FREE_WITH_IMU = """<mujoco><option timestep="0.01"/><worldbody>
<body name="b" pos="0 0 1"><joint type="free"/><geom type="sphere" size="0.1" mass="2"/>
<site name="imu"/></body></worldbody>
<sensor><accelerometer site="imu"/><gyro site="imu"/></sensor></mujoco>"""


def test_accelerometer_and_gyro_in_body_frame():
    """The MJCF parser leaves the accelerometer's and gyro's object at body 0 (objname is
    ignored); pointed at the free body here. The body is turned +90 degrees about x and spins
    about its centre (no torque): the accelerometer reports R^T g with R the body's rotation
    matrix, i.e. (0, -9.81, 0) up to rounding, and the gyro the angular velocity the step
    leaves in the state."""
    m = load_model(mjcf_string=FREE_WITH_IMU)
    types = m["sensors"]["type_object"][:, 0]
    assert list(types) == [2, 3]
    m["sensors"]["type_object"][:, 1] = 1
    w = O.OracleWorld(m, 1)
    h = np.sqrt(0.5)
    q = w.quaternions.copy()
    q[0, 1] = [h, 0, 0, h]
    av = w.angular_velocities.copy()
    av[0, 1, :3] = [0.0, 0.0, 0.5]
    w.reset_to_state(w.positions.copy(), q, None, av)
    w.step(None)
    qx, qy, qz, qw = w.quaternions[0, 1].astype(np.float64)
    R = np.array([[1 - 2 * (qy * qy + qz * qz), 2 * (qx * qy - qz * qw), 2 * (qx * qz + qy * qw)],
                  [2 * (qx * qy + qz * qw), 1 - 2 * (qx * qx + qz * qz), 2 * (qy * qz - qx * qw)],
                  [2 * (qx * qz - qy * qw), 2 * (qy * qz + qx * qw), 1 - 2 * (qx * qx + qy * qy)]])
    g = np.array([0.0, 0.0, -9.81])
    np.testing.assert_allclose(w.observations[0, :3], R.T @ g, atol=1e-4)
    np.testing.assert_allclose(w.observations[0, :3], [0.0, -9.81, 0.0], atol=0.05)
    np.testing.assert_allclose(w.observations[0, 3:6], w.angular_velocities[0, 1, :3])
    np.testing.assert_allclose(w.observations[0, 3:6], [0.0, 0.0, 0.5 * 0.999], rtol=1e-3)
