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
