"""Pins the oracle's extended narrow phase (narrow_phase.detectCollision,
src/collision/narrow_phase.zig:28-512) with checks that do not restate its code:

  sphere-sphere, sphere-plane   the reference's KATs (tests/test_collision.zig:54-80,
                                173-199, 220-233)
  sphere-capsule                float64 distance to the segment by dense sampling
  sphere-box                    float64 closest point in the box frame; inside the box the
                                normal is the farthest face's (boxFaceNormal keeps the
                                largest distance), a closed form
  capsule-capsule               closed forms (crossing, parallel overlap, collinear) and
                                float64 segment-segment distance by dense sampling
  capsule-plane, box-plane      float64 endpoint / corner heights
  box-box                       axis-aligned overlaps (closed form) and a float64 separating
                                axis test over the 15 axes for rotated boxes
  dispatch                      swapped operands give the flipped contact; pairs the
                                reference does not handle (capsule-box, cylinder, mesh) give none
  points and anchors            every pair's contact point and local anchors from float64
                                geometry with geom offsets, rotated and offset planes, the
                                farthest-face normal inside a box, parallel and zero-length
                                capsule axes; closest points by ternary search
"""
import numpy as np
import pytest

from oracle import oracle as O


def collider(kind, size, pos=(0, 0, 0), quat=(0, 0, 0, 1), local=(0, 0, 0)):
    r = np.zeros(1, O.COLLIDER_DTYPE)
    r["type"] = {"sphere": 0, "capsule": 1, "box": 2, "plane": 3, "cylinder": 4, "mesh": 5}[kind]
    s = list(size) + [0.0] * (3 - len(size))
    r["size"][0] = s
    r["position"][0, :3] = pos
    r["quaternion"][0] = quat
    r["local_pos"][0, :3] = local
    return r


def detect(a, b):
    return O.detect_collisions(a, b)[0]


def rot64(q):
    x, y, z, w = (float(v) for v in q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                     [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                     [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])


def rand_quat(rng):
    q = rng.normal(size=4)
    return (q / np.linalg.norm(q)).astype(np.float32)


# ---- reference KATs ----------------------------------------------------------------

def test_sphere_sphere_kats():
    r = detect(collider("sphere", [0.5]), collider("sphere", [0.5], pos=(0.8, 0, 0)))
    assert r["valid"] == 1 and abs(r["penetration"] - 0.2) < 0.01 and abs(r["normal"][0] - 1.0) < 0.01
    assert detect(collider("sphere", [0.5]), collider("sphere", [0.5], pos=(2.0, 0, 0)))["valid"] == 0
    touch = detect(collider("sphere", [0.5]), collider("sphere", [0.5], pos=(1.0, 0, 0)))
    assert touch["valid"] == 0 or touch["penetration"] <= 0.01


def test_sphere_plane_kats():
    plane = collider("plane", [0.0])
    r = detect(collider("sphere", [0.5], pos=(0, 0, 0.3)), plane)
    assert r["valid"] == 1 and abs(r["penetration"] - 0.2) < 0.01
    assert detect(collider("sphere", [0.5], pos=(0, 0, 1.0)), plane)["valid"] == 0


# ---- float64 geometry ----------------------------------------------------------------

def seg_point_dist(p, a, b, n=20001):
    t = np.linspace(0.0, 1.0, n)[:, None]
    pts = a + t * (b - a)
    d = np.linalg.norm(pts - p, axis=1)
    i = int(np.argmin(d))
    return d[i], pts[i]


def test_sphere_capsule_distance():
    rng = np.random.default_rng(0)
    checked = 0
    for _ in range(300):
        cq, cp = rand_quat(rng), rng.uniform(-1, 1, 3).astype(np.float32)
        sp = rng.uniform(-1.5, 1.5, 3).astype(np.float32)
        rs, rc, hl = (float(v) for v in rng.uniform(0.1, 0.6, 3))
        cap = collider("capsule", [rc, hl], pos=cp, quat=cq)
        r = detect(collider("sphere", [rs], pos=sp), cap)
        ax = rot64(cq) @ np.array([0, 0, 1.0])
        dist, closest = seg_point_dist(sp.astype(np.float64), cp - ax * hl, cp + ax * hl)
        if abs(dist - (rs + rc)) < 1e-4:
            continue
        assert r["valid"] == (dist < rs + rc)
        if r["valid"]:
            checked += 1
            assert abs(r["penetration"] - (rs + rc - dist)) < 1e-4
            np.testing.assert_allclose(r["normal"], (sp - closest) / dist, atol=1e-3)
    assert checked > 30


def test_sphere_box_distance_and_inside_normal():
    rng = np.random.default_rng(1)
    checked = 0
    for _ in range(600):
        bq, bp = rand_quat(rng), rng.uniform(-1, 1, 3).astype(np.float32)
        he = rng.uniform(0.2, 0.8, 3).astype(np.float32)
        sp = (bp + rng.uniform(-1.2, 1.2, 3)).astype(np.float32)
        rs = float(rng.uniform(0.1, 0.7))
        r = detect(collider("sphere", [rs], pos=sp), collider("box", he, pos=bp, quat=bq))
        R = rot64(bq)
        local = R.T @ (sp.astype(np.float64) - bp)
        cl = np.clip(local, -he, he)
        dist = np.linalg.norm(local - cl)
        if abs(dist - rs) < 1e-4 or dist < 1e-3:
            continue
        assert r["valid"] == (dist < rs)
        if r["valid"]:
            checked += 1
            assert abs(r["penetration"] - (rs - dist)) < 1e-4
            np.testing.assert_allclose(r["normal"], R @ ((local - cl) / dist), atol=1e-3)
            np.testing.assert_allclose(r["local_b"][:3], cl, atol=1e-4)
    assert checked > 30
    # Centre inside the box: boxFaceNormal keeps the largest face distance -> the far -x face.
    r = detect(collider("sphere", [0.2], pos=(0.1, 0, 0)), collider("box", [1, 1, 1]))
    assert r["valid"] == 1 and list(r["normal"]) == [-1.0, 0.0, 0.0] and r["penetration"] == np.float32(0.2)


def test_capsule_capsule_closed_forms():
    x90 = (0.0, np.sqrt(0.5), 0.0, np.sqrt(0.5))  # z axis -> x axis
    # crossing: A along z at the origin, B along x at y = 0.3 -> closest points 0.3 apart
    r = detect(collider("capsule", [0.2, 1.0]), collider("capsule", [0.2, 1.0], pos=(0, 0.3, 0), quat=x90))
    assert r["valid"] == 1 and abs(r["penetration"] - 0.1) < 1e-6
    np.testing.assert_allclose(r["normal"], [0, 1, 0], atol=1e-6)
    # parallel, overlapping along the axis, 0.35 apart
    r = detect(collider("capsule", [0.2, 1.0]), collider("capsule", [0.25, 1.0], pos=(0.35, 0, 1.5)))
    assert r["valid"] == 1 and abs(r["penetration"] - 0.1) < 1e-6
    # collinear, end caps 0.3 apart (gap 2.3 - 2.0)
    r = detect(collider("capsule", [0.2, 1.0]), collider("capsule", [0.2, 1.0], pos=(0, 0, 2.3)))
    assert r["valid"] == 1 and abs(r["penetration"] - 0.1) < 1e-6
    np.testing.assert_allclose(r["normal"], [0, 0, 1], atol=1e-6)


def test_capsule_capsule_distance():
    rng = np.random.default_rng(2)
    s = np.linspace(0, 1, 801)
    checked = 0
    for _ in range(60):
        qa, qb = rand_quat(rng), rand_quat(rng)
        pa, pb = rng.uniform(-0.6, 0.6, 3).astype(np.float32), rng.uniform(-0.6, 0.6, 3).astype(np.float32)
        ra, rb, ha, hb = (float(v) for v in rng.uniform(0.1, 0.5, 4))
        r = detect(collider("capsule", [ra, ha], pos=pa, quat=qa), collider("capsule", [rb, hb], pos=pb, quat=qb))
        xa, xb = rot64(qa) @ [0, 0, 1.0], rot64(qb) @ [0, 0, 1.0]
        A = (pa - xa * ha) + s[:, None] * (2 * ha * xa)
        Bp = (pb - xb * hb) + s[:, None] * (2 * hb * xb)
        d = np.sqrt(((A[:, None, :] - Bp[None, :, :]) ** 2).sum(-1)).min()
        if abs(d - (ra + rb)) < 2e-3 or d < 1e-3:
            continue
        assert r["valid"] == (d < ra + rb)
        if r["valid"]:
            checked += 1
            assert abs(r["penetration"] - (ra + rb - d)) < 2e-3
    assert checked > 10


def test_capsule_plane_and_box_plane_heights():
    rng = np.random.default_rng(3)
    for _ in range(200):
        q, p = rand_quat(rng), rng.uniform(-0.5, 0.5, 3).astype(np.float32)
        p[2] = rng.uniform(-0.2, 1.2)
        radius, hl = (float(v) for v in rng.uniform(0.1, 0.5, 2))
        plane = collider("plane", [0.0])
        r = detect(collider("capsule", [radius, hl], pos=p, quat=q), plane)
        ax = rot64(q) @ [0, 0, 1.0]
        low = min((p - ax * hl)[2], (p + ax * hl)[2]) - radius
        if abs(low) > 1e-4:
            assert r["valid"] == (low < 0)
            if r["valid"]:
                assert abs(r["penetration"] + low) < 1e-4
        he = rng.uniform(0.1, 0.5, 3).astype(np.float32)
        rb = detect(collider("box", he, pos=p, quat=q), plane)
        corners = np.array([[sx * he[0], sy * he[1], sz * he[2]] for sz in (-1, 1) for sy in (-1, 1) for sx in (-1, 1)])
        zmin = (corners @ rot64(q).T + p)[:, 2].min()
        if abs(zmin) > 1e-4:
            assert rb["valid"] == (zmin < 0)
            if rb["valid"]:
                assert abs(rb["penetration"] + zmin) < 1e-4
                np.testing.assert_allclose(rb["normal"], [0, 0, 1], atol=1e-6)


def test_box_box_axis_aligned_closed_form():
    r = detect(collider("box", [1, 1, 1]), collider("box", [0.5, 0.5, 0.5], pos=(1.3, 0.2, -0.1)))
    assert r["valid"] == 1 and abs(r["penetration"] - 0.2) < 1e-6
    np.testing.assert_allclose(r["normal"], [1, 0, 0], atol=1e-6)
    np.testing.assert_allclose(r["point"], [0.65, 0.1, -0.05], atol=1e-6)
    r = detect(collider("box", [1, 1, 1]), collider("box", [0.5, 0.5, 0.5], pos=(0.2, -1.4, 0.0)))
    assert r["valid"] == 1 and abs(r["penetration"] - 0.1) < 1e-6
    np.testing.assert_allclose(r["normal"], [0, -1, 0], atol=1e-6)
    assert detect(collider("box", [1, 1, 1]), collider("box", [0.5, 0.5, 0.5], pos=(1.6, 0, 0)))["valid"] == 0


def sat64(pa, Ra, ha, pb, Rb, hb):
    """float64 separating-axis test: None if separated, else (min overlap, axis A->B)."""
    axes = [Ra[:, i] for i in range(3)] + [Rb[:, i] for i in range(3)]
    for i in range(3):
        for j in range(3):
            c = np.cross(Ra[:, i], Rb[:, j])
            if np.linalg.norm(c) > 1e-6:
                axes.append(c / np.linalg.norm(c))
    d = pb - pa
    best, best_ax = np.inf, None
    for ax in axes:
        ra = sum(ha[k] * abs(ax @ Ra[:, k]) for k in range(3))
        rb = sum(hb[k] * abs(ax @ Rb[:, k]) for k in range(3))
        ov = ra + rb - abs(d @ ax)
        if ov < 0:
            return None
        if ov < best:
            best, best_ax = ov, ax
    return best, best_ax if best_ax @ d >= 0 else -best_ax


def test_box_box_rotated_sat():
    rng = np.random.default_rng(4)
    hits = 0
    for _ in range(300):
        qa, qb = rand_quat(rng), rand_quat(rng)
        pa, pb = rng.uniform(-0.8, 0.8, 3).astype(np.float32), rng.uniform(-0.8, 0.8, 3).astype(np.float32)
        ha, hb = rng.uniform(0.2, 0.6, 3).astype(np.float32), rng.uniform(0.2, 0.6, 3).astype(np.float32)
        r = detect(collider("box", ha, pos=pa, quat=qa), collider("box", hb, pos=pb, quat=qb))
        ref = sat64(pa.astype(np.float64), rot64(qa), ha, pb.astype(np.float64), rot64(qb), hb)
        if ref is not None and ref[0] < 1e-4:
            continue
        assert r["valid"] == (ref is not None)
        if ref is not None:
            hits += 1
            assert abs(r["penetration"] - ref[0]) < 1e-4
            np.testing.assert_allclose(r["point"], (pa + pb) / 2, atol=1e-5)
    assert hits > 50


# ---- dispatch ------------------------------------------------------------------------

@pytest.mark.parametrize("other", [("capsule", [0.3, 0.5]), ("box", [0.4, 0.3, 0.5]), ("plane", [0.05])])
def test_swapped_operands_flip(other):
    rng = np.random.default_rng(5)
    n_hit = 0
    for _ in range(100):
        s = collider("sphere", [0.4], pos=rng.uniform(-0.6, 0.6, 3))
        o = collider(other[0], other[1], pos=rng.uniform(-0.3, 0.3, 3), quat=rand_quat(rng))
        ab, ba = detect(s, o), detect(o, s)
        assert ab["valid"] == ba["valid"]
        if ab["valid"]:
            n_hit += 1
            assert np.array_equal(ab["point"], ba["point"]) and ab["penetration"] == ba["penetration"]
            assert np.array_equal(ab["normal"], -ba["normal"])
            assert np.array_equal(ab["local_a"], ba["local_b"]) and np.array_equal(ab["local_b"], ba["local_a"])
    assert n_hit > 10


def test_unhandled_pairs_give_no_contact():
    cap, box = collider("capsule", [0.5, 0.5]), collider("box", [0.5, 0.5, 0.5])
    assert detect(cap, box)["valid"] == 0 and detect(box, cap)["valid"] == 0
    for kind in ("cylinder", "mesh"):
        assert detect(collider(kind, [0.5, 0.5]), collider("sphere", [0.5]))["valid"] == 0
    assert detect(collider("plane", [0.0]), collider("plane", [0.0]))["valid"] == 0


# ---- contact points, anchors and frames ------------------------------------------------
# Each pair's point and local anchors from float64 geometry, with geom offsets, rotated
# planes and plane offsets, following the ContactResult each pair builds
# (narrow_phase.zig:125-423). Closest points come from ternary searches (the distance from
# a point to a segment, and from one segment to another, is convex along the segments), not
# from the projection formulas the oracle uses.

def world_point(pos, quat, local=(0, 0, 0)):
    return np.asarray(pos, np.float64) + rot64(quat) @ np.asarray(local, np.float64)


def ternary(f, lo=0.0, hi=1.0, iters=90):
    for _ in range(iters):
        m1, m2 = lo + (hi - lo) / 3, hi - (hi - lo) / 3
        if f(m1) <= f(m2):
            hi = m2
        else:
            lo = m1
    return 0.5 * (lo + hi)


def seg_closest(p, a, b):
    t = ternary(lambda t: np.linalg.norm(a + t * (b - a) - p))
    return a + t * (b - a)


def segseg_closest(a1, a2, b1, b2):
    inner = lambda s: ternary(lambda t: np.linalg.norm(a1 + s * (a2 - a1) - b1 - t * (b2 - b1)), iters=60)
    s = ternary(lambda s: np.linalg.norm(a1 + s * (a2 - a1) - b1 - inner(s) * (b2 - b1)), iters=60)
    t = inner(s)
    return a1 + s * (a2 - a1), b1 + t * (b2 - b1)


def anchors(r):
    return np.asarray(r["local_a"], np.float64), np.asarray(r["local_b"], np.float64)


def test_sphere_sphere_point_midway_between_the_surfaces():
    """point = midpoint of A's surface point toward B and B's surface point toward A;
    local_a = n ra, local_b = -n rb, n from A to B; centres include each geom's offset
    (narrow_phase.zig:41-43,125-153)."""
    rng = np.random.default_rng(6)
    checked = 0
    for _ in range(300):
        qa, qb = rand_quat(rng), rand_quat(rng)
        pa, pb = rng.uniform(-0.3, 0.3, 3), rng.uniform(-0.3, 0.3, 3)
        la, lb = rng.uniform(-0.25, 0.25, 3), rng.uniform(-0.25, 0.25, 3)
        ra, rb = (float(v) for v in rng.uniform(0.15, 0.5, 2))
        r = detect(collider("sphere", [ra], pa, qa, la), collider("sphere", [rb], pb, qb, lb))
        ca, cb = world_point(pa, qa, la), world_point(pb, qb, lb)
        d = np.linalg.norm(cb - ca)
        if abs(d - (ra + rb)) < 1e-4 or d < 1e-3:
            continue
        assert r["valid"] == (d < ra + rb)
        if r["valid"]:
            checked += 1
            n = (cb - ca) / d
            np.testing.assert_allclose(r["normal"], n, atol=2e-5)
            np.testing.assert_allclose(r["point"], 0.5 * ((ca + n * ra) + (cb - n * rb)), atol=2e-5)
            la_, lb_ = anchors(r)
            np.testing.assert_allclose(la_, np.r_[n * ra, 0], atol=2e-5)
            np.testing.assert_allclose(lb_, np.r_[-n * rb, 0], atol=2e-5)
    assert checked > 50


def test_sphere_capsule_point_and_anchors():
    """n from the capsule's axis point to the sphere centre; point = midpoint of the capsule's
    surface point (closest + n cr) and the sphere's surface point toward it (centre - n sr);
    local_a = n sr, local_b = -n cr (narrow_phase.zig:156-197)."""
    rng = np.random.default_rng(7)
    checked = 0
    for _ in range(300):
        cq, cp, cl = rand_quat(rng), rng.uniform(-0.5, 0.5, 3), rng.uniform(-0.2, 0.2, 3)
        sq, sp, sl = rand_quat(rng), rng.uniform(-1.0, 1.0, 3), rng.uniform(-0.2, 0.2, 3)
        rs, rc, hl = (float(v) for v in rng.uniform(0.1, 0.6, 3))
        r = detect(collider("sphere", [rs], sp, sq, sl), collider("capsule", [rc, hl], cp, cq, cl))
        s, c = world_point(sp, sq, sl), world_point(cp, cq, cl)
        ax = rot64(cq) @ [0, 0, 1.0]
        closest = seg_closest(s, c - ax * hl, c + ax * hl)
        d = np.linalg.norm(s - closest)
        if abs(d - (rs + rc)) < 1e-4 or d < 1e-3:
            continue
        assert r["valid"] == (d < rs + rc)
        if r["valid"]:
            checked += 1
            n = (s - closest) / d
            np.testing.assert_allclose(r["normal"], n, atol=1e-4)
            np.testing.assert_allclose(r["point"], 0.5 * ((closest + n * rc) + (s - n * rs)), atol=1e-4)
            la_, lb_ = anchors(r)
            np.testing.assert_allclose(la_, np.r_[n * rs, 0], atol=1e-4)
            np.testing.assert_allclose(lb_, np.r_[-n * rc, 0], atol=1e-4)
    assert checked > 50


def test_sphere_plane_offset_frame_and_point():
    """The plane's normal is its body's z axis and its point the body's transform of the geom
    offset; the signed distance subtracts the plane's offset (size[0]); point = midpoint of
    the sphere's deepest point and its projection on the plane; local_a = -n r
    (narrow_phase.zig:200-228)."""
    rng = np.random.default_rng(8)
    checked = 0
    for _ in range(300):
        pq, pp, pl = rand_quat(rng), rng.uniform(-0.5, 0.5, 3), rng.uniform(-0.3, 0.3, 3)
        off = float(rng.uniform(-0.3, 0.3))
        n = rot64(pq) @ [0, 0, 1.0]
        base = world_point(pp, pq, pl)
        sp = base + n * rng.uniform(-0.5, 1.0) + rng.uniform(-0.5, 0.5, 3)
        rs = float(rng.uniform(0.1, 0.6))
        r = detect(collider("sphere", [rs], sp.astype(np.float32)), collider("plane", [off], pp, pq, pl))
        s = sp.astype(np.float32).astype(np.float64)
        sd = (s - base) @ n - off
        if abs(sd - rs) < 1e-4:
            continue
        assert r["valid"] == (sd < rs)
        if r["valid"]:
            checked += 1
            assert abs(r["penetration"] - (rs - sd)) < 2e-5
            np.testing.assert_allclose(r["normal"], n, atol=2e-6)
            np.testing.assert_allclose(r["point"], 0.5 * ((s - n * rs) + (s - n * sd)), atol=2e-5)
            la_, lb_ = anchors(r)
            np.testing.assert_allclose(la_, np.r_[-n * rs, 0], atol=2e-6)
            assert not lb_.any()
    assert checked > 50


def test_sphere_box_point_and_anchors_in_the_body_frame():
    """The box frame is its body's transform (narrow_phase.zig:239-251): the clamp is about the
    body origin, and the geom offset enters only local_b = clamped - offset. point = world
    closest point + n pen/2; local_a = -n r (narrow_phase.zig:256-276)."""
    rng = np.random.default_rng(9)
    checked = 0
    for _ in range(600):
        bq, bp, bl = rand_quat(rng), rng.uniform(-0.5, 0.5, 3), rng.uniform(-0.3, 0.3, 3)
        he = rng.uniform(0.2, 0.7, 3).astype(np.float32)
        sq, sl = rand_quat(rng), rng.uniform(-0.2, 0.2, 3)
        sp = bp + rng.uniform(-1.2, 1.2, 3)
        rs = float(rng.uniform(0.1, 0.6))
        r = detect(collider("sphere", [rs], sp, sq, sl), collider("box", he, bp, bq, bl))
        s = world_point(sp.astype(np.float32), sq, sl)
        R = rot64(bq)
        local = R.T @ (s - bp.astype(np.float32))
        cl = np.clip(local, -he, he)
        d = np.linalg.norm(local - cl)
        if abs(d - rs) < 1e-4 or d < 1e-3:
            continue
        assert r["valid"] == (d < rs)
        if r["valid"]:
            checked += 1
            n = R @ ((local - cl) / d)
            wc = bp.astype(np.float32) + R @ cl
            np.testing.assert_allclose(r["point"], wc + n * (rs - d) / 2, atol=5e-5)
            la_, lb_ = anchors(r)
            np.testing.assert_allclose(la_, np.r_[-n * rs, 0], atol=5e-5)
            np.testing.assert_allclose(lb_, np.r_[cl - bl.astype(np.float32), 0], atol=5e-5)
    assert checked > 50


def test_sphere_centre_inside_a_box_takes_the_farthest_face():
    """With the centre inside the box (distance 0) the normal is the face direction of largest
    face distance: face +i at he_i - p_i gives +e_i, face -i at he_i + p_i gives -e_i
    (boxFaceNormal, narrow_phase.zig:890-910); the point is the centre + n r/2."""
    rng = np.random.default_rng(10)
    for _ in range(200):
        bq, bp = rand_quat(rng), rng.uniform(-0.5, 0.5, 3)
        he = rng.uniform(0.3, 0.8, 3)
        lp = rng.uniform(-0.9, 0.9, 3) * he
        dist = np.r_[he - lp, he + lp]
        if np.sort(dist)[-1] - np.sort(dist)[-2] < 1e-3:
            continue
        k = int(np.argmax(dist))
        ln = np.zeros(3)
        ln[k % 3] = 1.0 if k < 3 else -1.0
        R = rot64(bq)
        sp = (bp + R @ lp).astype(np.float32)
        rs = float(rng.uniform(0.1, 0.5))
        r = detect(collider("sphere", [rs], sp), collider("box", he.astype(np.float32), bp, bq))
        assert r["valid"] == 1
        np.testing.assert_allclose(r["normal"], R @ ln, atol=2e-6)
        assert abs(r["penetration"] - rs) < 1e-5
        np.testing.assert_allclose(r["point"], sp + R @ ln * rs / 2, atol=2e-5)


def test_capsule_capsule_point_and_anchors():
    """point = midpoint of A's surface point (qa + n ra) and B's (qb - n rb) over the closest
    points qa, qb of the two axes; local_a = n ra, local_b = -n rb (narrow_phase.zig:280-331)."""
    rng = np.random.default_rng(11)
    checked = 0
    for _ in range(80):
        qa, qb = rand_quat(rng), rand_quat(rng)
        pa, pb = rng.uniform(-0.6, 0.6, 3).astype(np.float32), rng.uniform(-0.6, 0.6, 3).astype(np.float32)
        ra, rb, ha, hb = (float(v) for v in rng.uniform(0.1, 0.5, 4))
        r = detect(collider("capsule", [ra, ha], pos=pa, quat=qa), collider("capsule", [rb, hb], pos=pb, quat=qb))
        xa, xb = rot64(qa) @ [0, 0, 1.0], rot64(qb) @ [0, 0, 1.0]
        if abs(xa @ xb) > 0.99:
            continue
        ca, cb = segseg_closest(pa - xa * ha, pa + xa * ha, pb - xb * hb, pb + xb * hb)
        d = np.linalg.norm(cb - ca)
        if abs(d - (ra + rb)) < 1e-4 or d < 1e-2:
            continue
        assert r["valid"] == (d < ra + rb)
        if r["valid"]:
            checked += 1
            n = (cb - ca) / d
            np.testing.assert_allclose(r["normal"], n, atol=1e-4)
            np.testing.assert_allclose(r["point"], 0.5 * ((ca + n * ra) + (cb - n * rb)), atol=1e-4)
            la_, lb_ = anchors(r)
            np.testing.assert_allclose(la_, np.r_[n * ra, 0], atol=1e-4)
            np.testing.assert_allclose(lb_, np.r_[-n * rb, 0], atol=1e-4)
    assert checked > 10


def test_capsule_capsule_parallel_takes_the_start_of_a():
    """Parallel axes leave s at 0 (denominator 0): A's contact axis point is its start
    a1 = centre - axis h, and B's is the point of B's axis nearest a1
    (closestPointsBetweenSegments, narrow_phase.zig:852-864)."""
    # A along z at the origin (a1 = (0,0,-1)), B parallel at x = 0.35 spanning z in [-1.5, 0.5]
    r = detect(collider("capsule", [0.2, 1.0]), collider("capsule", [0.25, 1.0], pos=(0.35, 0, -0.5)))
    assert r["valid"] == 1 and abs(r["penetration"] - 0.1) < 1e-6
    np.testing.assert_allclose(r["normal"], [1, 0, 0], atol=1e-6)
    np.testing.assert_allclose(r["point"], [0.5 * (0.2 + 0.10), 0, -1.0], atol=1e-6)


@pytest.mark.parametrize("which", ["a", "b"])
def test_zero_length_capsule_is_a_sphere(which):
    """A capsule of half-length 0 has a degenerate axis segment (length below EPSILON) and
    meets another capsule as a sphere of its radius would (narrow_phase.zig:840-851)."""
    rng = np.random.default_rng(12 if which == "a" else 13)
    checked = 0
    for _ in range(200):
        q, p = rand_quat(rng), rng.uniform(-0.4, 0.4, 3).astype(np.float32)
        c = rng.uniform(-0.8, 0.8, 3).astype(np.float32)
        rc, rs, hl = (float(v) for v in rng.uniform(0.1, 0.5, 3))
        long_cap = collider("capsule", [rc, hl], pos=p, quat=q)
        point_cap = collider("capsule", [rs, 0.0], pos=c, quat=rand_quat(rng))
        r = detect(point_cap, long_cap) if which == "a" else detect(long_cap, point_cap)
        ax = rot64(q) @ [0, 0, 1.0]
        closest = seg_closest(c.astype(np.float64), p - ax * hl, p + ax * hl)
        d = np.linalg.norm(c - closest)
        if abs(d - (rs + rc)) < 1e-4 or d < 1e-3:
            continue
        assert r["valid"] == (d < rs + rc)
        if r["valid"]:
            checked += 1
            assert abs(r["penetration"] - (rs + rc - d)) < 1e-4
            n = (closest - c) / d if which == "a" else (c - closest) / d
            np.testing.assert_allclose(r["normal"], n, atol=1e-4)
    assert checked > 30


def test_capsule_plane_point_anchor_and_no_offset():
    """Endpoint heights are measured from the plane body's transform of the geom offset, with
    no plane offset (size[0] is not read); point = midpoint of the deepest surface point and
    its projection on the plane; local_a = -n r (narrow_phase.zig:334-370)."""
    rng = np.random.default_rng(14)
    checked = 0
    for _ in range(300):
        pq, pp, pl = rand_quat(rng), rng.uniform(-0.5, 0.5, 3), rng.uniform(-0.3, 0.3, 3)
        n = rot64(pq) @ [0, 0, 1.0]
        base = world_point(pp, pq, pl)
        cq, hl, rad = rand_quat(rng), float(rng.uniform(0.1, 0.5)), float(rng.uniform(0.1, 0.4))
        cp = (base + n * rng.uniform(-0.3, 1.0) + rng.uniform(-0.5, 0.5, 3)).astype(np.float32)
        r = detect(collider("capsule", [rad, hl], cp, cq), collider("plane", [0.4], pp, pq, pl))
        ax = rot64(cq) @ [0, 0, 1.0]
        ends = [cp - ax * hl, cp + ax * hl]
        h = [(e - base) @ n - rad for e in ends]
        if min(abs(h[0]), abs(h[1])) < 1e-4 or abs(h[0] - h[1]) < 1e-4:
            continue
        assert r["valid"] == (min(h) < 0)
        if r["valid"]:
            checked += 1
            k = int(np.argmin(h))
            assert abs(r["penetration"] + h[k]) < 2e-5
            surface = ends[k] - n * rad
            np.testing.assert_allclose(r["point"], 0.5 * (surface + (surface - n * h[k])), atol=2e-5)
            la_, lb_ = anchors(r)
            np.testing.assert_allclose(la_, np.r_[-n * rad, 0], atol=2e-6)
            assert not lb_.any()
    assert checked > 50


def test_box_plane_corner_point_anchor_and_no_offset():
    """The deepest of the box's corners about its body origin (the box's geom offset is not
    read), measured from the plane body's transform of its geom offset with no plane offset;
    the point is that corner in the world and local_a the corner in the box frame
    (narrow_phase.zig:373-423)."""
    rng = np.random.default_rng(15)
    checked = 0
    signs = np.array([[sx, sy, sz] for sz in (-1, 1) for sy in (-1, 1) for sx in (-1, 1)], np.float64)
    for _ in range(300):
        pq, pp, pl = rand_quat(rng), rng.uniform(-0.5, 0.5, 3), rng.uniform(-0.3, 0.3, 3)
        n = rot64(pq) @ [0, 0, 1.0]
        base = world_point(pp, pq, pl)
        bq, he, bl = rand_quat(rng), rng.uniform(0.1, 0.5, 3).astype(np.float32), rng.uniform(-0.3, 0.3, 3)
        bp = (base + n * rng.uniform(-0.3, 0.8) + rng.uniform(-0.5, 0.5, 3)).astype(np.float32)
        r = detect(collider("box", he, bp, bq, bl), collider("plane", [0.4], pp, pq, pl))
        corners = signs * he
        world = corners @ rot64(bq).T + bp
        h = (world - base) @ n
        order = np.argsort(h)
        if abs(h[order[0]]) < 1e-4 or h[order[1]] - h[order[0]] < 1e-4:
            continue
        assert r["valid"] == (h[order[0]] < 0)
        if r["valid"]:
            checked += 1
            k = order[0]
            assert abs(r["penetration"] + h[k]) < 2e-5
            np.testing.assert_allclose(r["point"], world[k], atol=2e-5)
            la_, lb_ = anchors(r)
            np.testing.assert_allclose(la_, np.r_[corners[k], 0], atol=0)
            assert not lb_.any()
    assert checked > 50


@pytest.mark.parametrize("other", [("capsule", [0.3, 0.5]), ("box", [0.4, 0.3, 0.5])])
def test_plane_first_flips(other):
    """plane-capsule and plane-box are the capsule-plane and box-plane contacts flipped
    (narrow_phase.zig:104-120, flipContact :912-920)."""
    rng = np.random.default_rng(16)
    n_hit = 0
    for _ in range(100):
        plane = collider("plane", [0.0], pos=rng.uniform(-0.2, 0.2, 3), quat=rand_quat(rng))
        o = collider(other[0], other[1], pos=rng.uniform(-0.4, 0.4, 3), quat=rand_quat(rng))
        ab, ba = detect(o, plane), detect(plane, o)
        assert ab["valid"] == ba["valid"]
        if ab["valid"]:
            n_hit += 1
            assert np.array_equal(ab["point"], ba["point"]) and ab["penetration"] == ba["penetration"]
            assert np.array_equal(ab["normal"], -ba["normal"])
            assert np.array_equal(ab["local_a"], ba["local_b"]) and np.array_equal(ab["local_b"], ba["local_a"])
    assert n_hit > 10
