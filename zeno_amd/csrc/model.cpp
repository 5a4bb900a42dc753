// Scene -> device-ready model.
#include "model.h"

#include <algorithm>
#include <cstring>

namespace za {
namespace {

// World.quatConjugate / quatMultiply / rotateByQuat, world.zig:180-212. The host-side
// rotation uses its own operation order (t = 2 (q.xyz x v); v + w t + q.xyz x t).
void quat_conj(const float q[4], float o[4]) { o[0] = -q[0]; o[1] = -q[1]; o[2] = -q[2]; o[3] = q[3]; }

void quat_mul(const float a[4], const float b[4], float o[4]) {
    float r[4] = {
        a[3] * b[0] + a[0] * b[3] + a[1] * b[2] - a[2] * b[1],
        a[3] * b[1] - a[0] * b[2] + a[1] * b[3] + a[2] * b[0],
        a[3] * b[2] + a[0] * b[1] - a[1] * b[0] + a[2] * b[3],
        a[3] * b[3] - a[0] * b[0] - a[1] * b[1] - a[2] * b[2],
    };
    std::memcpy(o, r, sizeof r);
}

void host_rotate(const float v[3], const float q[4], float o[3]) {
    float t0 = 2.0f * (q[1] * v[2] - q[2] * v[1]);
    float t1 = 2.0f * (q[2] * v[0] - q[0] * v[2]);
    float t2 = 2.0f * (q[0] * v[1] - q[1] * v[0]);
    float r[3] = {
        v[0] + q[3] * t0 + (q[1] * t2 - q[2] * t1),
        v[1] + q[3] * t1 + (q[2] * t0 - q[0] * t2),
        v[2] + q[3] * t2 + (q[0] * t1 - q[1] * t0),
    };
    std::memcpy(o, r, sizeof r);
}

// Primitive constraint kinds of joint.zig:169-187.
enum PrimKind { P_DISTANCE, P_POINT, P_HINGE, P_SLIDER, P_CONE_LIMIT, P_ANGULAR_LIMIT, P_LINEAR_LIMIT, P_WELD };

struct Prim {
    PrimKind kind;
    uint32_t a, b;
    float anchor_a[3], anchor_b[3], axis[3];
    float damping = 0, lower = 0, upper = 0;
};

Prim make_prim(PrimKind k, const JointDef& j, const float axis[3]) {
    Prim p;
    p.kind = k;
    p.a = j.parent_body;
    p.b = j.child_body;
    std::memcpy(p.anchor_a, j.anchor_parent, sizeof p.anchor_a);
    std::memcpy(p.anchor_b, j.anchor_child, sizeof p.anchor_b);
    std::memcpy(p.axis, axis, sizeof p.axis);
    return p;
}

// joint.zig:202-350
void decompose_joint(const JointDef& j, std::vector<Prim>& out) {
    const float zero[3] = {0, 0, 0};
    switch (j.joint_type) {
        case JOINT_FIXED: out.push_back(make_prim(P_WELD, j, zero)); break;
        case JOINT_REVOLUTE: {
            out.push_back(make_prim(P_POINT, j, zero));
            Prim h = make_prim(P_HINGE, j, j.axis);
            h.damping = j.damping;
            out.push_back(h);
            if (j.has_limits()) {
                Prim l = make_prim(P_ANGULAR_LIMIT, j, j.axis);
                l.lower = j.limit_lower;
                l.upper = j.limit_upper;
                out.push_back(l);
            }
            break;
        }
        case JOINT_PRISMATIC: {
            Prim s = make_prim(P_SLIDER, j, j.axis);
            s.damping = j.damping;
            out.push_back(s);
            if (j.has_limits()) {
                Prim l = make_prim(P_LINEAR_LIMIT, j, j.axis);
                l.lower = j.limit_lower;
                l.upper = j.limit_upper;
                out.push_back(l);
            }
            break;
        }
        case JOINT_BALL: {
            out.push_back(make_prim(P_POINT, j, zero));
            if (j.has_limits()) {
                Prim c = make_prim(P_CONE_LIMIT, j, j.axis);
                c.upper = j.limit_upper;
                out.push_back(c);
            }
            break;
        }
        case JOINT_FREE: break;
        case JOINT_UNIVERSAL:
            out.push_back(make_prim(P_POINT, j, zero));
            out.push_back(make_prim(P_HINGE, j, j.axis));
            out.push_back(make_prim(P_HINGE, j, j.axis2));
            break;
        default: break;
    }
}

void set4(float d[4], float a, float b, float c, float e) { d[0] = a; d[1] = b; d[2] = c; d[3] = e; }

// world.zig:315-445. Compliance is always 0 because decomposeJoint never sets one
// (world.zig:323).
bool prim_to_template(const Prim& p, const Scene& s, ConstraintRec& c) {
    std::memset(&c, 0, sizeof c);
    const float compliance = 0.0f;
    c.indices[0] = p.a;
    c.indices[1] = p.b;
    c.indices[2] = 0;
    switch (p.kind) {
        case P_POINT:  // xpbd.zig:213-228
            c.indices[3] = C_POSITIONAL;
            set4(c.anchor_a, p.anchor_a[0], p.anchor_a[1], p.anchor_a[2], compliance);
            set4(c.anchor_b, p.anchor_b[0], p.anchor_b[1], p.anchor_b[2], 0);
            return true;
        case P_HINGE: {  // world.zig:331-351, xpbd.zig:231-250
            float aw[3], qbi[4], ab[3];
            host_rotate(p.axis, s.bodies[p.a].quaternion, aw);
            quat_conj(s.bodies[p.b].quaternion, qbi);
            host_rotate(aw, qbi, ab);
            c.indices[3] = C_ANGULAR;
            set4(c.anchor_a, p.axis[0], p.axis[1], p.axis[2], compliance);
            set4(c.anchor_b, ab[0], ab[1], ab[2], p.damping);
            return true;
        }
        case P_WELD: {  // world.zig:353-371, xpbd.zig:310-330
            float qai[4], rel[4];
            quat_conj(s.bodies[p.a].quaternion, qai);
            quat_mul(qai, s.bodies[p.b].quaternion, rel);
            c.indices[3] = C_WELD;
            set4(c.anchor_a, p.anchor_a[0], p.anchor_a[1], p.anchor_a[2], compliance);
            set4(c.anchor_b, p.anchor_b[0], p.anchor_b[1], p.anchor_b[2], 0);
            std::memcpy(c.axis_target, rel, sizeof rel);
            return true;
        }
        case P_ANGULAR_LIMIT:  // xpbd.zig:253-272
            c.indices[3] = C_ANGULAR_LIMIT;
            set4(c.anchor_a, p.axis[0], p.axis[1], p.axis[2], compliance);
            set4(c.limits, p.lower, p.upper, 0, 0);
            return true;
        case P_CONE_LIMIT:  // world.zig:416-429
            c.indices[3] = C_ANGULAR_LIMIT;
            set4(c.anchor_a, p.axis[0], p.axis[1], p.axis[2], compliance);
            set4(c.limits, -p.upper, p.upper, 0, 0);
            return true;
        case P_LINEAR_LIMIT:  // world.zig:385-396
            c.indices[3] = C_LINEAR_LIMIT;
            set4(c.anchor_a, p.axis[0], p.axis[1], p.axis[2], compliance);
            set4(c.anchor_b, p.anchor_b[0], p.anchor_b[1], p.anchor_b[2], 0);
            set4(c.limits, p.lower, p.upper, 0, 0);
            return true;
        case P_SLIDER: {  // world.zig:397-415
            float qai[4], rel[4];
            quat_conj(s.bodies[p.a].quaternion, qai);
            quat_mul(qai, s.bodies[p.b].quaternion, rel);
            c.indices[3] = C_SLIDER;
            set4(c.anchor_a, p.anchor_a[0], p.anchor_a[1], p.anchor_a[2], compliance);
            set4(c.anchor_b, p.anchor_b[0], p.anchor_b[1], p.anchor_b[2], p.damping);
            set4(c.axis_target, p.axis[0], p.axis[1], p.axis[2], 0);
            std::memcpy(c.limits, rel, sizeof rel);
            return true;
        }
        case P_DISTANCE:  // never produced by decompose_joint; world.zig:430-442
            c.indices[3] = C_CONNECT;
            set4(c.anchor_a, p.anchor_a[0], p.anchor_a[1], p.anchor_a[2], compliance);
            set4(c.anchor_b, p.anchor_b[0], p.anchor_b[1], p.anchor_b[2], 0);
            return true;
    }
    return false;
}

}  // namespace

uint32_t color_constraints(std::vector<ConstraintRec>& cs, uint32_t num_bodies) {
    const size_t n = cs.size();
    if (n == 0) return 0;
    std::vector<std::vector<uint32_t>> per_body(num_bodies);
    for (size_t i = 0; i < n; ++i) {
        uint32_t a = cs[i].indices[0], b = cs[i].indices[1];
        if (a < num_bodies) per_body[a].push_back((uint32_t)i);
        if (b < num_bodies && b != a) per_body[b].push_back((uint32_t)i);
    }
    uint32_t max_color = 0;
    bool used[256];
    for (size_t i = 0; i < n; ++i) {
        std::memset(used, 0, sizeof used);
        uint32_t a = cs[i].indices[0], b = cs[i].indices[1];
        auto mark = [&](uint32_t body) {
            for (uint32_t nb : per_body[body])
                if (nb < i) used[(cs[nb].indices[3] >> 8) & 0xFF] = true;
        };
        if (a < num_bodies) mark(a);
        if (b < num_bodies && b != a) mark(b);
        uint32_t color = 0;
        while (color < 255 && used[color]) ++color;
        cs[i].indices[3] = (cs[i].indices[3] & 0xFFu) | (color << 8);
        max_color = std::max(max_color, color);
    }
    return max_color + 1;
}

void build_model(const Scene& s, Model& m) {
    m = Model{};
    m.physics = s.physics;
    m.num_bodies = (uint32_t)s.bodies.size();
    m.num_joints = (uint32_t)s.joints.size();
    m.num_geoms = (uint32_t)s.geoms.size();
    m.num_actuators = (uint32_t)s.actuators.size();
    m.num_sensors = (uint32_t)s.sensors.size();
    m.obs_dim = s.obs_dim;

    // Bodies (world.zig:1580-1596) and the per-env initial state (world.zig:663-691).
    const uint32_t B = m.num_bodies;
    m.bodies.resize(B);
    m.init_pos.assign(4 * B, 0.0f);
    m.init_quat.assign(4 * B, 0.0f);
    m.init_vel.assign(4 * B, 0.0f);
    m.init_angvel.assign(4 * B, 0.0f);
    m.inv_mass_inertia.assign(4 * B, 0.0f);
    for (uint32_t i = 0; i < B; ++i) {
        const BodyDef& b = s.bodies[i];
        BodyRec& r = m.bodies[i];
        float invi[3];
        b.inv_inertia(invi);
        float invm = b.inv_mass();
        set4(r.position, b.position[0], b.position[1], b.position[2], 0);
        std::memcpy(r.quaternion, b.quaternion, sizeof r.quaternion);
        set4(r.inv_mass_inertia, invm, invi[0], invi[1], invi[2]);
        set4(r.params, (float)b.parent_id, (float)b.body_type, b.gravity_scale, b.linear_damping);
        set4(r.com_offset, b.com_offset[0], b.com_offset[1], b.com_offset[2], 0);
        set4(&m.init_pos[4 * i], b.position[0], b.position[1], b.position[2], 0);
        std::memcpy(&m.init_quat[4 * i], b.quaternion, 4 * sizeof(float));
        set4(&m.init_vel[4 * i], b.linear_velocity[0], b.linear_velocity[1], b.linear_velocity[2], 0);
        set4(&m.init_angvel[4 * i], b.angular_velocity[0], b.angular_velocity[1], b.angular_velocity[2], 0);
        set4(&m.inv_mass_inertia[4 * i], invm, invi[0], invi[1], invi[2]);
    }

    // Joints (world.zig:1606-1619).
    m.joints.resize(m.num_joints);
    m.joint_limited.resize(m.num_joints);
    for (uint32_t i = 0; i < m.num_joints; ++i) {
        const JointDef& j = s.joints[i];
        JointRec& r = m.joints[i];
        set4(r.anchor_parent, j.anchor_parent[0], j.anchor_parent[1], j.anchor_parent[2], 0);
        set4(r.anchor_child, j.anchor_child[0], j.anchor_child[1], j.anchor_child[2], 0);
        set4(r.axis, j.axis[0], j.axis[1], j.axis[2], 0);
        set4(r.params, (float)j.joint_type, (float)j.parent_body, (float)j.child_body, j.limit_lower);
        set4(r.params2, j.limit_upper, j.damping, j.stiffness, j.ref_position);
        m.joint_limited[i] = j.limited ? 1 : 0;
    }

    // Geoms (primitives.zig:433-441).
    m.geoms.resize(m.num_geoms);
    for (uint32_t i = 0; i < m.num_geoms; ++i) {
        const GeomDef& g = s.geoms[i];
        GeomRec& r = m.geoms[i];
        r.type_body[0] = g.geom_type;
        r.type_body[1] = g.body_id;
        r.type_body[2] = g.mask;
        r.type_body[3] = g.group;
        set4(r.pos_size0, g.local_pos[0], g.local_pos[1], g.local_pos[2], g.size[0]);
        std::memcpy(r.quat, g.local_quat, sizeof r.quat);
        set4(r.params, g.size[1], g.size[2], g.friction, g.restitution);
    }

    // Actuators (world.zig:1626-1636) and sensors with running output offsets
    // (world.zig:646-655).
    m.actuators.resize(m.num_actuators);
    for (uint32_t i = 0; i < m.num_actuators; ++i) {
        const ActuatorDef& a = s.actuators[i];
        set4(m.actuators[i].params, (float)a.joint, a.ctrl_min, a.ctrl_max, a.gear);
        set4(m.actuators[i].params2, a.force_min, a.force_max, a.kp, a.kv);
    }
    m.sensors.resize(m.num_sensors);
    uint32_t offset = 0;
    for (uint32_t i = 0; i < m.num_sensors; ++i) {
        const SensorDef& sd = s.sensors[i];
        SensorRec& r = m.sensors[i];
        r.type_object[0] = sd.sensor_type;
        r.type_object[1] = sd.object_id;
        r.type_object[2] = sd.dim;
        r.type_object[3] = 0;
        set4(r.params, sd.noise, sd.cutoff, (float)sd.dim, (float)offset);
        offset += sd.dim;
    }

    // Constraint templates, colouring, stable sort by colour, colour ranges.
    std::vector<Prim> prims;
    for (const JointDef& j : s.joints) decompose_joint(j, prims);
    m.templates.clear();
    for (const Prim& p : prims) {
        ConstraintRec c;
        if (prim_to_template(p, s, c)) m.templates.push_back(c);
    }
    m.num_constraints = (uint32_t)m.templates.size();
    if (m.num_constraints > 0) {
        m.num_colors = color_constraints(m.templates, B);
        std::stable_sort(m.templates.begin(), m.templates.end(), [](const ConstraintRec& x, const ConstraintRec& y) {
            return ((x.indices[3] >> 8) & 0xFF) < ((y.indices[3] >> 8) & 0xFF);
        });
        // xpbd.zig:619-640
        m.color_ranges.assign(2 * m.num_colors, 0);
        uint32_t cur = (m.templates[0].indices[3] >> 8) & 0xFF;
        uint32_t start = 0;
        for (uint32_t i = 0; i < m.num_constraints; ++i) {
            uint32_t col = (m.templates[i].indices[3] >> 8) & 0xFF;
            if (col != cur) {
                m.color_ranges[2 * cur] = start;
                m.color_ranges[2 * cur + 1] = i - start;
                cur = col;
                start = i;
            }
        }
        m.color_ranges[2 * cur] = start;
        m.color_ranges[2 * cur + 1] = m.num_constraints - start;
        for (uint32_t c = 0; c < m.num_colors; ++c) m.max_color_size = std::max(m.max_color_size, m.color_ranges[2 * c + 1]);
    }

    // Candidate geom pairs: the broad phase's static filters (same body, contype /
    // conaffinity, all_shaders.metal:494-506) depend only on the model, so they are
    // applied once here. The list keeps (g, g') lexicographic order. Scenes above
    // kHashMinGeoms geoms use the spatial hash instead (world.zig:534) and keep no list.
    m.pairs.clear();
    const uint32_t listed = m.num_geoms > kHashMinGeoms ? 0u : m.num_geoms;
    for (uint32_t g = 0; g < listed; ++g) {
        for (uint32_t h = g + 1; h < listed; ++h) {
            const GeomRec& a = m.geoms[g];
            const GeomRec& b = m.geoms[h];
            if (a.type_body[1] == b.type_body[1]) continue;
            if ((a.type_body[3] & b.type_body[2]) == 0 && (b.type_body[3] & a.type_body[2]) == 0) continue;
            m.pairs.push_back(g | (h << 16));
        }
    }
    m.num_pairs = (uint32_t)m.pairs.size();
}

}  // namespace za
