// Extended narrow phase, device side: narrow_phase.detectCollision and the primitive pairs
// it dispatches to (src/collision/narrow_phase.zig:28-512, helpers :786-925). Used by the
// batched collision kernel (collide.hip) and, in the opt-in extended-contact mode, by the
// step kernel's narrow phase.
//
// Arithmetic follows the reference's operation order with no FMA contraction and correctly
// rounded sqrt and division (the library's build flags); std.math.clamp is @max(lo, @min(x,
// hi)) with @min/@max returning the non-NaN operand and, between +0 and -0, the second one.
// Axes come from the body transform only, as in the reference. Heightfield, mesh and
// cylinder pairs (GJK/EPA) report no contact.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/zeno_amd_ext.h"
#include "dmath.h"

namespace za {
namespace np {

constexpr float kNpEps = 1e-6f;  // constants.EPSILON (src/physics/constants.zig:13)

struct Side {
    uint32_t type;
    f3 size, local;
    f3 pos;
    q4 q;
};

// A ZenoAmdCollider record as its four 16-B quads.
__device__ __forceinline__ Side side_from(float4 r0, float4 r1, float4 r2, float4 r3) {
    Side s;
    s.type = __float_as_uint(r0.x);
    s.size = mk3(r0.y, r0.z, r0.w);
    s.local = mk3(r1.x, r1.y, r1.z);
    s.pos = mk3(r2.x, r2.y, r2.z);
    s.q = mk4(r3.x, r3.y, r3.z, r3.w);
    return s;
}
__device__ __forceinline__ Side load_side(const ZenoAmdCollider* c) {
    const float4* p = reinterpret_cast<const float4*>(c);
    return side_from(p[0], p[1], p[2], p[3]);
}

__device__ __forceinline__ float np_min(float a, float b) { return a != a ? b : (b != b ? a : (a < b ? a : b)); }
__device__ __forceinline__ float np_max(float a, float b) { return a != a ? b : (b != b ? a : (a > b ? a : b)); }
__device__ __forceinline__ float np_clamp(float x, float lo, float hi) { return np_max(lo, np_min(x, hi)); }

// Transform.transformPoint / transformVector (body.zig:192-203); rotateByQuat is qrot.
__device__ __forceinline__ f3 tpoint(const Side& s, f3 local) {
    const f3 r = qrot(local, s.q);
    return mk3(r.x + s.pos.x, r.y + s.pos.y, r.z + s.pos.z);
}
__device__ __forceinline__ f3 taxis(const Side& s, float x, float y, float z) { return qrot(mk3(x, y, z), s.q); }

struct Result {
    f3 point, normal, la, lb;
    float pen;
    bool valid;
};

__device__ __forceinline__ Result hit(f3 point, f3 normal, float pen, f3 la, f3 lb) {
    Result r;
    r.point = point; r.normal = normal; r.pen = pen; r.la = la; r.lb = lb; r.valid = true;
    return r;
}
__device__ __forceinline__ Result miss() {
    Result r;
    r.point = r.normal = r.la = r.lb = mk3(0.0f, 0.0f, 0.0f);
    r.pen = 0.0f;
    r.valid = false;
    return r;
}
// flipContact (:912-920)
__device__ __forceinline__ Result flip(Result r) {
    if (!r.valid) return r;
    const f3 t = r.la;
    r.normal = scale(r.normal, -1.0f);
    r.la = r.lb;
    r.lb = t;
    return r;
}

// sphereSphere (:125-153)
__device__ inline Result sphere_sphere(f3 pa, float ra, f3 pb, float rb) {
    const f3 diff = sub(pb, pa);
    const float dist_sq = dot(diff, diff);
    const float min_dist = ra + rb;
    if (dist_sq >= min_dist * min_dist) return miss();
    const float dist = __builtin_sqrtf(dist_sq);
    const f3 n = dist > kNpEps ? scale(diff, 1.0f / dist) : mk3(0.0f, 0.0f, 1.0f);
    const float pen = min_dist - dist;
    return hit(add(pa, scale(n, ra - pen * 0.5f)), n, pen, scale(n, ra), scale(n, -rb));
}

// closestPointOnSegment (:815-825)
__device__ __forceinline__ f3 closest_on_segment(f3 p, f3 s, f3 e) {
    const f3 seg = sub(e, s);
    const float len_sq = dot(seg, seg);
    if (len_sq < kNpEps) return s;
    const float t = np_clamp(dot(sub(p, s), seg) / len_sq, 0.0f, 1.0f);
    return add(s, scale(seg, t));
}

// sphereCapsule (:156-197)
__device__ inline Result sphere_capsule(f3 sp, float sr, f3 cp, const Side& cap) {
    const float cr = cap.size.x, hl = cap.size.y;
    const f3 axis = taxis(cap, 0.0f, 0.0f, 1.0f);
    const f3 p1 = sub(cp, scale(axis, hl));
    const f3 p2 = add(cp, scale(axis, hl));
    const f3 closest = closest_on_segment(sp, p1, p2);
    const f3 diff = sub(sp, closest);
    const float dist_sq = dot(diff, diff);
    const float min_dist = sr + cr;
    if (dist_sq >= min_dist * min_dist) return miss();
    const float dist = __builtin_sqrtf(dist_sq);
    const f3 n = dist > kNpEps ? scale(diff, 1.0f / dist) : mk3(0.0f, 0.0f, 1.0f);
    const float pen = min_dist - dist;
    return hit(add(closest, scale(n, cr - pen * 0.5f)), n, pen, scale(n, sr), scale(n, -cr));
}

// spherePlane (:200-228)
__device__ inline Result sphere_plane(f3 sp, float sr, const Side& pl) {
    const f3 n = taxis(pl, 0.0f, 0.0f, 1.0f);
    const f3 pp = tpoint(pl, pl.local);
    const float signed_dist = dot(sub(sp, pp), n) - pl.size.x;
    if (signed_dist >= sr) return miss();
    const float pen = sr - signed_dist;
    return hit(sub(sp, scale(n, signed_dist + pen * 0.5f)), n, pen, scale(n, -sr), mk3(0.0f, 0.0f, 0.0f));
}

// boxFaceNormal (:890-910): the face with the largest distance from the point.
__device__ __forceinline__ f3 box_face_normal(f3 p, f3 he) {
    float maxd = -__builtin_inff();
    f3 nrm = mk3(0.0f, 0.0f, 1.0f);
    const float pc[3] = {p.x, p.y, p.z}, hc[3] = {he.x, he.y, he.z};
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float dpos = hc[i] - pc[i];
        const float dneg = hc[i] + pc[i];
        if (dpos > maxd) { maxd = dpos; nrm = mk3(i == 0 ? 1.0f : 0.0f, i == 1 ? 1.0f : 0.0f, i == 2 ? 1.0f : 0.0f); }
        if (dneg > maxd) { maxd = dneg; nrm = mk3(i == 0 ? -1.0f : 0.0f, i == 1 ? -1.0f : 0.0f, i == 2 ? -1.0f : 0.0f); }
    }
    return nrm;
}

// sphereBox (:231-277), with Transform.inverse (body.zig:223-235)
__device__ inline Result sphere_box(f3 sp, float sr, const Side& box) {
    const q4 iq = mk4(-box.q.x, -box.q.y, -box.q.z, box.q.w);
    const f3 ipos = qrot(mk3(-box.pos.x, -box.pos.y, -box.pos.z), iq);
    const f3 r = qrot(sp, iq);
    const f3 ls = mk3(r.x + ipos.x, r.y + ipos.y, r.z + ipos.z);
    const f3 he = box.size;
    const f3 cl = mk3(np_clamp(ls.x, -he.x, he.x), np_clamp(ls.y, -he.y, he.y), np_clamp(ls.z, -he.z, he.z));
    const f3 diff = sub(ls, cl);
    const float dist_sq = dot(diff, diff);
    if (dist_sq >= sr * sr) return miss();
    const float dist = __builtin_sqrtf(dist_sq);
    const f3 ln = dist > kNpEps ? scale(diff, 1.0f / dist) : box_face_normal(ls, he);
    const f3 wc = tpoint(box, cl);
    const f3 n = qrot(ln, box.q);
    const float pen = sr - dist;
    return hit(add(wc, scale(n, pen * 0.5f)), n, pen, scale(n, -sr), sub(cl, box.local));
}

// closestPointsBetweenSegments (:832-888)
__device__ inline void closest_between_segments(f3 a1, f3 a2, f3 b1, f3 b2, f3& pa, f3& pb) {
    const f3 d1 = sub(a2, a1), d2 = sub(b2, b1), r = sub(a1, b1);
    const float a = dot(d1, d1), e = dot(d2, d2), f = dot(d2, r);
    float s = 0.0f, t = 0.0f;
    if (a < kNpEps && e < kNpEps) { pa = a1; pb = b1; return; }
    if (a < kNpEps) {
        t = np_clamp(f / e, 0.0f, 1.0f);
    } else {
        const float c = dot(d1, r);
        if (e < kNpEps) {
            s = np_clamp(-c / a, 0.0f, 1.0f);
        } else {
            const float b = dot(d1, d2);
            const float denom = a * e - b * b;
            if (denom != 0.0f) s = np_clamp((b * f - c * e) / denom, 0.0f, 1.0f);
            t = (b * s + f) / e;
            if (t < 0.0f) {
                t = 0.0f;
                s = np_clamp(-c / a, 0.0f, 1.0f);
            } else if (t > 1.0f) {
                t = 1.0f;
                s = np_clamp((b - c) / a, 0.0f, 1.0f);
            }
        }
    }
    pa = add(a1, scale(d1, s));
    pb = add(b1, scale(d2, t));
}

// capsuleCapsule (:280-331)
__device__ inline Result capsule_capsule(f3 pa, const Side& ca, f3 pb, const Side& cb) {
    const float ra = ca.size.x, rb = cb.size.x, ha = ca.size.y, hb = cb.size.y;
    const f3 xa = taxis(ca, 0.0f, 0.0f, 1.0f), xb = taxis(cb, 0.0f, 0.0f, 1.0f);
    const f3 a1 = sub(pa, scale(xa, ha)), a2 = add(pa, scale(xa, ha));
    const f3 b1 = sub(pb, scale(xb, hb)), b2 = add(pb, scale(xb, hb));
    f3 qa, qb;
    closest_between_segments(a1, a2, b1, b2, qa, qb);
    const f3 diff = sub(qb, qa);
    const float dist_sq = dot(diff, diff);
    const float min_dist = ra + rb;
    if (dist_sq >= min_dist * min_dist) return miss();
    const float dist = __builtin_sqrtf(dist_sq);
    const f3 n = dist > kNpEps ? scale(diff, 1.0f / dist) : mk3(0.0f, 0.0f, 1.0f);
    const float pen = min_dist - dist;
    const f3 wa = add(qa, scale(n, ra));
    const f3 wb = sub(qb, scale(n, rb));
    return hit(scale(add(wa, wb), 0.5f), n, pen, scale(n, ra), scale(n, -rb));
}

// capsulePlane (:334-370)
__device__ inline Result capsule_plane(f3 cp, const Side& cap, const Side& pl) {
    const float radius = cap.size.x, hl = cap.size.y;
    const f3 axis = taxis(cap, 0.0f, 0.0f, 1.0f);
    const f3 n = taxis(pl, 0.0f, 0.0f, 1.0f);
    const f3 pp = tpoint(pl, pl.local);
    const f3 p1 = sub(cp, scale(axis, hl));
    const f3 p2 = add(cp, scale(axis, hl));
    const float d1 = dot(sub(p1, pp), n) - radius;
    const float d2 = dot(sub(p2, pp), n) - radius;
    if (d1 >= 0.0f && d2 >= 0.0f) return miss();
    const f3 deepest = d1 < d2 ? p1 : p2;
    const float dist = np_min(d1, d2);
    return hit(sub(deepest, scale(n, dist * 0.5f + radius)), n, -dist, scale(n, -radius), mk3(0.0f, 0.0f, 0.0f));
}

// boxPlane (:373-423): the eight corners in the reference's order.
__device__ inline Result box_plane(const Side& box, const Side& pl) {
    const f3 h = box.size;
    const f3 n = taxis(pl, 0.0f, 0.0f, 1.0f);
    const f3 pp = tpoint(pl, pl.local);
    float min_dist = __builtin_inff();
    f3 dc = mk3(0.0f, 0.0f, 0.0f), dw = dc;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const f3 corner = mk3((k & 1) ? h.x : -h.x, (k & 2) ? h.y : -h.y, (k & 4) ? h.z : -h.z);
        const f3 wc = tpoint(box, corner);
        const float dist = dot(sub(wc, pp), n);
        if (dist < min_dist) { min_dist = dist; dc = corner; dw = wc; }
    }
    if (min_dist >= 0.0f) return miss();
    return hit(dw, n, -min_dist, dc, mk3(0.0f, 0.0f, 0.0f));
}

// testAxis (:788-813): false for a separating axis.
__device__ __forceinline__ bool test_axis(f3 axis, f3 d, const f3* xa, f3 ha, const f3* xb, f3 hb, float& overlap) {
    const float proj_a = ha.x * __builtin_fabsf(dot(axis, xa[0])) + ha.y * __builtin_fabsf(dot(axis, xa[1])) +
                         ha.z * __builtin_fabsf(dot(axis, xa[2]));
    const float proj_b = hb.x * __builtin_fabsf(dot(axis, xb[0])) + hb.y * __builtin_fabsf(dot(axis, xb[1])) +
                         hb.z * __builtin_fabsf(dot(axis, xb[2]));
    const float dist = __builtin_fabsf(dot(d, axis));
    if (dist > proj_a + proj_b) return false;
    overlap = proj_a + proj_b - dist;
    return true;
}

// boxBox, separating axes (:426-512)
__device__ inline Result box_box(f3 pa, const Side& ba, f3 pb, const Side& bb) {
    const f3 xa[3] = {taxis(ba, 1.0f, 0.0f, 0.0f), taxis(ba, 0.0f, 1.0f, 0.0f), taxis(ba, 0.0f, 0.0f, 1.0f)};
    const f3 xb[3] = {taxis(bb, 1.0f, 0.0f, 0.0f), taxis(bb, 0.0f, 1.0f, 0.0f), taxis(bb, 0.0f, 0.0f, 1.0f)};
    const f3 d = sub(pb, pa);
    float min_overlap = __builtin_inff(), ov = 0.0f;
    f3 best = mk3(0.0f, 0.0f, 1.0f);
    for (int i = 0; i < 3; ++i) {
        if (!test_axis(xa[i], d, xa, ba.size, xb, bb.size, ov)) return miss();
        if (ov < min_overlap) { min_overlap = ov; best = xa[i]; }
    }
    for (int i = 0; i < 3; ++i) {
        if (!test_axis(xb[i], d, xa, ba.size, xb, bb.size, ov)) return miss();
        if (ov < min_overlap) { min_overlap = ov; best = xb[i]; }
    }
    for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j) {
            const f3 edge = cross(xa[i], xb[j]);
            const float len = __builtin_sqrtf(dot(edge, edge));
            if (len < kNpEps) continue;
            const f3 nrm = scale(edge, 1.0f / len);
            if (!test_axis(nrm, d, xa, ba.size, xb, bb.size, ov)) return miss();
            if (ov < min_overlap) { min_overlap = ov; best = nrm; }
        }
    }
    if (dot(best, d) < 0.0f) best = scale(best, -1.0f);
    return hit(add(pa, scale(d, 0.5f)), best, min_overlap, mk3(0.0f, 0.0f, 0.0f), mk3(0.0f, 0.0f, 0.0f));
}

// detectCollision (:28-123): types 0 sphere, 1 capsule, 2 box, 3 plane.
__device__ inline Result detect(const Side& a, const Side& b) {
    const f3 pa = tpoint(a, a.local);
    const f3 pb = tpoint(b, b.local);
    switch (a.type) {
        case 0:
            if (b.type == 0) return sphere_sphere(pa, a.size.x, pb, b.size.x);
            if (b.type == 1) return sphere_capsule(pa, a.size.x, pb, b);
            if (b.type == 2) return sphere_box(pa, a.size.x, b);
            if (b.type == 3) return sphere_plane(pa, a.size.x, b);
            return miss();
        case 1:
            if (b.type == 0) return flip(sphere_capsule(pb, b.size.x, pa, a));
            if (b.type == 1) return capsule_capsule(pa, a, pb, b);
            if (b.type == 3) return capsule_plane(pa, a, b);
            return miss();
        case 2:
            if (b.type == 0) return flip(sphere_box(pb, b.size.x, a));
            if (b.type == 3) return box_plane(a, b);
            if (b.type == 2) return box_box(pa, a, pb, b);
            return miss();
        case 3:
            if (b.type == 0) return flip(sphere_plane(pb, b.size.x, a));
            if (b.type == 1) return flip(capsule_plane(pb, b, a));
            if (b.type == 2) return flip(box_plane(b, a));
            return miss();
        default:
            return miss();
    }
}

}  // namespace np
}  // namespace za
