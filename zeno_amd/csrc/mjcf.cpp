// MJCF subset parser producing a za::Scene.
//
// The reference's parser (src/mjcf/parser.zig) is not a conforming XML/MJCF reader, and
// the physics step depends on several of its quirks, so this parser reproduces them
// deliberately:
//   * self-closing tags produce a start token only (parser.zig:1390-1396);
//   * attribute lookup, number and vector parsing split on single spaces
//     (parser.zig:1440-1558);
//   * `<default>` handling stops at the first closing tag (parser.zig:774-821);
//   * body world position is the sum of relative positions with no rotation
//     composition, and the body quaternion is the local one (parser.zig:898-922);
//   * joint `range` is used as given (radians), `anchor_parent = body.pos + joint.pos`
//     (parser.zig:964-994);
//   * a body without joints gets a fixed joint to its parent (parser.zig:953-962);
//   * a `fromto` capsule keeps the default quaternion; mass and COM use the geom `pos`
//     attribute, not the fromto midpoint (parser.zig:1031-1081, 1213-1243);
//   * frame sensors ignore `objname` and read object 0 (parser.zig:1277-1330).
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <optional>
#include <sstream>

#include "scene.h"

namespace za {

// ----------------------------------------------------------------------------------
// Scene container (world/scene.zig:43-117, sensors.zig:170-207)
// ----------------------------------------------------------------------------------
uint32_t Scene::add_body(const BodyDef& b) {
    uint32_t id = (uint32_t)bodies.size();
    bodies.push_back(b);
    if (!b.name.empty()) body_names[b.name] = id;
    return id;
}
uint32_t Scene::add_joint(const JointDef& j) {
    uint32_t id = (uint32_t)joints.size();
    joints.push_back(j);
    if (!j.name.empty()) joint_names[j.name] = id;
    return id;
}
uint32_t Scene::add_geom(const std::string& name, const GeomDef& g) {
    uint32_t id = (uint32_t)geoms.size();
    geoms.push_back(g);
    if (!name.empty()) geom_names[name] = id;
    return id;
}
uint32_t Scene::add_actuator(const ActuatorDef& a) {
    uint32_t id = (uint32_t)actuators.size();
    actuators.push_back(a);
    if (!a.name.empty()) actuator_names[a.name] = id;
    return id;
}
void Scene::add_sensor(const SensorDef& s) {
    sensors.push_back(s);
    obs_dim += s.dim;
}
void Scene::auto_add_sensors() {
    // Root = first dynamic body with a negative parent. The parser gives every body a
    // parent >= 0, so for MJCF scenes this stays body 0 (the static world).
    uint32_t root = 0;
    for (size_t i = 0; i < bodies.size(); ++i) {
        if (bodies[i].body_type == BODY_DYNAMIC && bodies[i].parent_id < 0) { root = (uint32_t)i; break; }
    }
    const uint32_t frame_types[4] = {S_FRAMEPOS, S_FRAMEQUAT, S_FRAMELINVEL, S_FRAMEANGVEL};
    const uint32_t frame_dims[4] = {3, 4, 3, 3};
    for (int k = 0; k < 4; ++k) {
        SensorDef s; s.sensor_type = frame_types[k]; s.object_id = root; s.dim = frame_dims[k];
        add_sensor(s);
    }
    for (uint32_t j = 0; j < (uint32_t)joints.size(); ++j) {
        SensorDef p; p.sensor_type = 0; p.object_id = j; p.dim = 1; add_sensor(p);
        SensorDef v; v.sensor_type = 1; v.object_id = j; v.dim = 1; add_sensor(v);
    }
}

namespace {

// ----------------------------------------------------------------------------------
// Tokenizer (parser.zig:1341-1438)
// ----------------------------------------------------------------------------------
enum TokKind { TOK_START, TOK_END, TOK_TEXT, TOK_COMMENT };
struct Token {
    TokKind kind;
    std::string_view name;
    std::string_view attrs;
};

inline bool is_ws(char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r'; }

struct Tokenizer {
    std::string_view src;
    size_t pos = 0;

    void skip_ws() { while (pos < src.size() && is_ws(src[pos])) ++pos; }

    bool next(Token& t) {
        skip_ws();
        if (pos >= src.size()) return false;
        if (src[pos] == '<') return parse_tag(t);
        size_t start = pos;
        while (pos < src.size() && src[pos] != '<') ++pos;
        t = {TOK_TEXT, src.substr(start, pos - start), {}};
        return true;
    }

    bool parse_tag(Token& t) {
        ++pos;  // '<'
        if (pos >= src.size()) return false;
        if (src.size() - pos >= 3 && src.compare(pos, 3, "!--") == 0) {
            while (pos + 2 < src.size()) {
                if (src[pos] == '-' && src[pos + 1] == '-' && src[pos + 2] == '>') { pos += 3; break; }
                ++pos;
            }
            t = {TOK_COMMENT, {}, {}};
            return true;
        }
        bool is_end = src[pos] == '/';
        if (is_end) ++pos;
        size_t name_start = pos;
        while (pos < src.size() && !is_ws(src[pos]) && src[pos] != '>' && src[pos] != '/') ++pos;
        std::string_view name = src.substr(name_start, pos - name_start);
        skip_ws();
        size_t attrs_start = pos;
        while (pos < src.size() && src[pos] != '>') ++pos;
        size_t attrs_end = pos;
        if (!is_end) {
            size_t check = pos;
            while (check > attrs_start && is_ws(src[check - 1])) --check;
            if (check > attrs_start && src[check - 1] == '/') attrs_end = check - 1;
        }
        std::string_view attrs = src.substr(attrs_start, attrs_end - attrs_start);
        if (pos < src.size()) ++pos;  // '>'
        if (is_end) t = {TOK_END, name, {}};
        else t = {TOK_START, name, attrs};
        return true;
    }
};

// parser.zig:1440-1484
std::optional<std::string_view> get_attr(std::string_view attrs, std::string_view name) {
    size_t pos = 0;
    while (pos < attrs.size()) {
        while (pos < attrs.size() && is_ws(attrs[pos])) ++pos;
        size_t ns = pos;
        while (pos < attrs.size() && attrs[pos] != '=' && !is_ws(attrs[pos])) ++pos;
        std::string_view attr_name = attrs.substr(ns, pos - ns);
        while (pos < attrs.size() && (is_ws(attrs[pos]) || attrs[pos] == '=')) ++pos;
        if (pos >= attrs.size()) break;
        char q = attrs[pos];
        if (q != '"' && q != '\'') continue;
        ++pos;
        size_t vs = pos;
        while (pos < attrs.size() && attrs[pos] != q) ++pos;
        std::string_view value = attrs.substr(vs, pos - vs);
        ++pos;
        if (attr_name == name) return value;
    }
    return std::nullopt;
}

// Whole-string f32 parse; fails on empty input, leading blanks or trailing characters,
// as std.fmt.parseFloat does (parser.zig:1486-1488).
std::optional<float> parse_float(std::string_view s) {
    if (s.empty() || is_ws(s[0])) return std::nullopt;
    std::string tmp(s);
    char* end = nullptr;
    errno = 0;
    float v = std::strtof(tmp.c_str(), &end);
    if (end != tmp.c_str() + tmp.size()) return std::nullopt;
    return v;
}

// Base-10 u32 parse with an optional '+' and '_' digit separators (parser.zig:1490-1492).
std::optional<uint32_t> parse_int(std::string_view s) {
    size_t i = 0;
    if (i < s.size() && s[i] == '+') ++i;
    if (i >= s.size()) return std::nullopt;
    uint64_t v = 0;
    bool prev_digit = false;
    for (; i < s.size(); ++i) {
        char c = s[i];
        if (c == '_') {
            if (!prev_digit || i + 1 >= s.size()) return std::nullopt;
            prev_digit = false;
            continue;
        }
        if (c < '0' || c > '9') return std::nullopt;
        v = v * 10 + (uint64_t)(c - '0');
        if (v > 0xFFFFFFFFull) return std::nullopt;
        prev_digit = true;
    }
    if (!prev_digit) return std::nullopt;
    return (uint32_t)v;
}

// Splits on single spaces, keeping empty fields (std.mem.splitScalar semantics).
struct SpaceSplit {
    std::string_view s;
    size_t pos = 0;
    bool done = false;
    bool next(std::string_view& out) {
        if (done) return false;
        size_t sp = s.find(' ', pos);
        if (sp == std::string_view::npos) { out = s.substr(pos); done = true; return true; }
        out = s.substr(pos, sp - pos);
        pos = sp + 1;
        return true;
    }
};

template <int N>
bool parse_vecn(std::string_view s, float* out) {
    SpaceSplit it{s};
    for (int i = 0; i < N; ++i) {
        std::string_view part;
        if (!it.next(part)) return false;
        auto v = parse_float(part);
        if (!v) return false;
        out[i] = *v;
    }
    return true;
}

// parser.zig:1537-1547: up to three fields, each failed field reads as 0.
void parse_size(std::string_view s, float out[3]) {
    out[0] = out[1] = out[2] = 0.0f;
    SpaceSplit it{s};
    std::string_view part;
    int i = 0;
    while (it.next(part)) {
        if (i >= 3) break;
        auto v = parse_float(part);
        out[i] = v ? *v : 0.0f;
        ++i;
    }
}

// ----------------------------------------------------------------------------------
// Parsed MJCF model (mjcf/schema.zig:100-223)
// ----------------------------------------------------------------------------------
enum MJointType { MJ_FREE, MJ_BALL, MJ_SLIDE, MJ_HINGE };
enum MGeomType { MG_PLANE, MG_SPHERE, MG_CAPSULE, MG_CYLINDER, MG_BOX, MG_MESH, MG_HFIELD };
enum MActType { MA_MOTOR, MA_POSITION, MA_VELOCITY, MA_GENERAL };

struct MJoint {
    std::string name;
    MJointType type = MJ_HINGE;
    float pos[3] = {0, 0, 0};
    float axis[3] = {0, 0, 1};
    bool has_range = false;
    float range[2] = {0, 0};
    bool limited = false;
    float damping = 0, stiffness = 0, armature = 0, ref = 0;
};

struct MGeom {
    std::string name;
    MGeomType type = MG_SPHERE;
    float pos[3] = {0, 0, 0};
    float quat[4] = {1, 0, 0, 0};  // wxyz
    float size[3] = {0.05f, 0, 0};
    bool has_fromto = false;
    float fromto[6] = {0, 0, 0, 0, 0, 0};
    bool has_mass = false;
    float mass = 0;
    float density = 1000.0f;
    float friction[3] = {1.0f, 0.005f, 0.0001f};
    uint32_t contype = 1;
    uint32_t conaffinity = 1;
};

struct MInertial {
    float mass = 1.0f;
    float pos[3] = {0, 0, 0};
    bool has_diag = false;
    float diag[3] = {0, 0, 0};
    bool has_full = false;
    float full[6] = {0, 0, 0, 0, 0, 0};
};

struct MBody {
    std::string name;
    float pos[3] = {0, 0, 0};
    float quat[4] = {1, 0, 0, 0};  // wxyz
    bool has_euler = false;
    float euler[3] = {0, 0, 0};
    std::string childclass;
    bool has_inertial = false;
    MInertial inertial;
    std::vector<MJoint> joints;
    std::vector<MGeom> geoms;
    std::vector<MBody> children;
};

struct MActuator {
    std::string name;
    MActType type = MA_MOTOR;
    std::string joint;
    bool has_ctrlrange = false;
    float ctrlrange[2] = {0, 0};
    bool has_forcerange = false;
    float forcerange[2] = {0, 0};
    float gear = 1.0f;
    float kp = 0, kv = 0;
};

struct MSensor {
    std::string name;
    int type = 0;  // index into kSensorNames
    std::string joint;
    float noise = 0;
    float cutoff = 0;
};

struct MDefault {
    MJoint joint;
    MGeom geom;
};

struct MModel {
    float timestep = 0.002f;
    float gravity[3] = {0, 0, -9.81f};
    std::map<std::string, MDefault> defaults;
    MBody worldbody;
    std::vector<MActuator> actuators;
    std::vector<MSensor> sensors;
};

const char* kSensorNames[] = {"jointpos", "jointvel", "accelerometer", "gyro", "touch", "force",
                              "torque", "framepos", "framequat", "framelinvel", "frameangvel",
                              "subtreecom"};

std::optional<MJointType> joint_type_from(std::string_view s) {
    if (s == "free") return MJ_FREE;
    if (s == "ball") return MJ_BALL;
    if (s == "slide") return MJ_SLIDE;
    if (s == "hinge") return MJ_HINGE;
    return std::nullopt;
}
std::optional<MGeomType> geom_type_from(std::string_view s) {
    if (s == "plane") return MG_PLANE;
    if (s == "sphere") return MG_SPHERE;
    if (s == "capsule") return MG_CAPSULE;
    if (s == "cylinder") return MG_CYLINDER;
    if (s == "box") return MG_BOX;
    if (s == "mesh") return MG_MESH;
    if (s == "hfield") return MG_HFIELD;
    return std::nullopt;
}

// parser.zig:412-451
void apply_joint_attrs(MJoint& j, std::string_view a) {
    if (auto v = get_attr(a, "name")) j.name = std::string(*v);
    if (auto v = get_attr(a, "type")) { if (auto t = joint_type_from(*v)) j.type = *t; }
    if (auto v = get_attr(a, "pos")) { float t[3]; if (parse_vecn<3>(*v, t)) std::memcpy(j.pos, t, sizeof t); }
    if (auto v = get_attr(a, "axis")) { float t[3]; if (parse_vecn<3>(*v, t)) std::memcpy(j.axis, t, sizeof t); }
    if (auto v = get_attr(a, "range")) {
        float t[2];
        j.has_range = parse_vecn<2>(*v, t);
        if (j.has_range) std::memcpy(j.range, t, sizeof t);
        j.limited = j.has_range;
    }
    if (auto v = get_attr(a, "damping")) { if (auto f = parse_float(*v)) j.damping = *f; }
    if (auto v = get_attr(a, "stiffness")) { if (auto f = parse_float(*v)) j.stiffness = *f; }
    if (auto v = get_attr(a, "armature")) { if (auto f = parse_float(*v)) j.armature = *f; }
    if (auto v = get_attr(a, "ref")) { if (auto f = parse_float(*v)) j.ref = *f; }
}

// parser.zig:469-526
void apply_geom_attrs(MGeom& g, std::string_view a) {
    if (auto v = get_attr(a, "name")) g.name = std::string(*v);
    if (auto v = get_attr(a, "type")) { if (auto t = geom_type_from(*v)) g.type = *t; }
    if (auto v = get_attr(a, "pos")) { float t[3]; if (parse_vecn<3>(*v, t)) std::memcpy(g.pos, t, sizeof t); }
    if (auto v = get_attr(a, "quat")) { float t[4]; if (parse_vecn<4>(*v, t)) std::memcpy(g.quat, t, sizeof t); }
    if (auto v = get_attr(a, "size")) parse_size(*v, g.size);
    if (auto v = get_attr(a, "fromto")) {
        float t[6];
        g.has_fromto = parse_vecn<6>(*v, t);
        if (g.has_fromto) std::memcpy(g.fromto, t, sizeof t);
    }
    if (auto v = get_attr(a, "mass")) {
        auto f = parse_float(*v);
        g.has_mass = (bool)f;
        g.mass = f ? *f : 0.0f;
    }
    if (auto v = get_attr(a, "density")) { if (auto f = parse_float(*v)) g.density = *f; }
    if (auto v = get_attr(a, "friction")) { float t[3]; if (parse_vecn<3>(*v, t)) std::memcpy(g.friction, t, sizeof t); }
    if (auto v = get_attr(a, "contype")) { if (auto n = parse_int(*v)) g.contype = *n; }
    if (auto v = get_attr(a, "conaffinity")) { if (auto n = parse_int(*v)) g.conaffinity = *n; }
    if (auto v = get_attr(a, "mesh")) { (void)v; g.type = MG_MESH; }
}

MJoint joint_with_defaults(std::string_view a, const std::map<std::string, MDefault>& defs, const std::string& cls) {
    std::string use = cls;
    if (auto v = get_attr(a, "class")) use = std::string(*v);
    MJoint j;
    auto it = defs.find(use);
    if (it != defs.end()) j = it->second.joint;
    apply_joint_attrs(j, a);
    return j;
}

MGeom geom_with_defaults(std::string_view a, const std::map<std::string, MDefault>& defs, const std::string& cls) {
    std::string use = cls;
    if (auto v = get_attr(a, "class")) use = std::string(*v);
    MGeom g;
    auto it = defs.find(use);
    if (it != defs.end()) g = it->second.geom;
    apply_geom_attrs(g, a);
    return g;
}

// parser.zig:371-396
MInertial parse_inertial(std::string_view a) {
    MInertial in;
    if (auto v = get_attr(a, "mass")) { auto f = parse_float(*v); in.mass = f ? *f : 1.0f; }
    if (auto v = get_attr(a, "pos")) { float t[3] = {0, 0, 0}; if (!parse_vecn<3>(*v, t)) { t[0] = t[1] = t[2] = 0; } std::memcpy(in.pos, t, sizeof t); }
    if (auto v = get_attr(a, "diaginertia")) in.has_diag = parse_vecn<3>(*v, in.diag);
    if (auto v = get_attr(a, "fullinertia")) in.has_full = parse_vecn<6>(*v, in.full);
    return in;
}

// parser.zig:326-369
void parse_body_content(Tokenizer& tk, MBody& body, std::string_view end_tag,
                        const std::map<std::string, MDefault>& defs, const std::string& parent_class) {
    Token t;
    while (tk.next(t)) {
        if (t.kind == TOK_END && t.name == end_tag) break;
        if (t.kind != TOK_START) continue;
        if (t.name == "body") {
            MBody child;
            if (auto v = get_attr(t.attrs, "name")) child.name = std::string(*v);
            if (auto v = get_attr(t.attrs, "pos")) { float p[3]; if (parse_vecn<3>(*v, p)) std::memcpy(child.pos, p, sizeof p); else child.pos[0] = child.pos[1] = child.pos[2] = 0; }
            if (auto v = get_attr(t.attrs, "quat")) { float q[4]; if (parse_vecn<4>(*v, q)) std::memcpy(child.quat, q, sizeof q); else { child.quat[0] = 1; child.quat[1] = child.quat[2] = child.quat[3] = 0; } }
            if (auto v = get_attr(t.attrs, "euler")) child.has_euler = parse_vecn<3>(*v, child.euler);
            std::string cc = parent_class;
            if (auto v = get_attr(t.attrs, "childclass")) cc = std::string(*v);
            child.childclass = cc;
            parse_body_content(tk, child, "body", defs, cc);
            body.children.push_back(std::move(child));
        } else if (t.name == "joint") {
            body.joints.push_back(joint_with_defaults(t.attrs, defs, parent_class));
        } else if (t.name == "geom") {
            body.geoms.push_back(geom_with_defaults(t.attrs, defs, parent_class));
        } else if (t.name == "inertial") {
            body.inertial = parse_inertial(t.attrs);
            body.has_inertial = true;
        }
    }
}

// parser.zig:774-821
void parse_defaults(Tokenizer& tk, std::map<std::string, MDefault>& defs) {
    std::string cls = "main";
    MDefault cur;
    Token t;
    while (tk.next(t)) {
        if (t.kind == TOK_END && t.name == "default") {
            if (!cls.empty()) defs[cls] = cur;
            break;
        }
        if (t.kind != TOK_START) continue;
        if (t.name == "default") {
            if (!cls.empty()) defs[cls] = cur;
            auto v = get_attr(t.attrs, "class");
            cls = v ? std::string(*v) : std::string("main");
            cur = MDefault{};
        } else if (t.name == "geom") {
            cur.geom = MGeom{};
            apply_geom_attrs(cur.geom, t.attrs);
        } else if (t.name == "joint") {
            cur.joint = MJoint{};
            apply_joint_attrs(cur.joint, t.attrs);
        }
    }
}

// parser.zig:529-552
void parse_actuators(Tokenizer& tk, std::vector<MActuator>& out) {
    Token t;
    while (tk.next(t)) {
        if (t.kind == TOK_END && t.name == "actuator") break;
        if (t.kind != TOK_START) continue;
        if (t.name == "motor" || t.name == "position" || t.name == "velocity" || t.name == "general") {
            MActuator a;
            if (auto v = get_attr(t.attrs, "name")) a.name = std::string(*v);
            a.type = t.name == "motor" ? MA_MOTOR : t.name == "position" ? MA_POSITION
                   : t.name == "velocity" ? MA_VELOCITY : MA_GENERAL;
            if (auto v = get_attr(t.attrs, "joint")) a.joint = std::string(*v);
            if (auto v = get_attr(t.attrs, "ctrlrange")) a.has_ctrlrange = parse_vecn<2>(*v, a.ctrlrange);
            if (auto v = get_attr(t.attrs, "forcerange")) a.has_forcerange = parse_vecn<2>(*v, a.forcerange);
            if (auto v = get_attr(t.attrs, "gear")) { auto f = parse_float(*v); a.gear = f ? *f : 1.0f; }
            if (auto v = get_attr(t.attrs, "kp")) { auto f = parse_float(*v); a.kp = f ? *f : 0.0f; }
            if (auto v = get_attr(t.attrs, "kv")) { auto f = parse_float(*v); a.kv = f ? *f : 0.0f; }
            out.push_back(a);
        }
    }
}

// parser.zig:588-609
void parse_sensors(Tokenizer& tk, std::vector<MSensor>& out) {
    Token t;
    while (tk.next(t)) {
        if (t.kind == TOK_END && t.name == "sensor") break;
        if (t.kind != TOK_START) continue;
        MSensor s;
        if (auto v = get_attr(t.attrs, "name")) s.name = std::string(*v);
        s.type = 0;
        for (int k = 0; k < 12; ++k) if (t.name == kSensorNames[k]) { s.type = k; break; }
        if (auto v = get_attr(t.attrs, "joint")) s.joint = std::string(*v);
        if (auto v = get_attr(t.attrs, "noise")) { auto f = parse_float(*v); s.noise = f ? *f : 0.0f; }
        out.push_back(s);
    }
}

// Consumes a section the scene does not use, up to its closing tag.
void skip_section(Tokenizer& tk, std::string_view end_tag) {
    Token t;
    while (tk.next(t)) if (t.kind == TOK_END && t.name == end_tag) break;
}

// parser.zig:190-218
void parse_xml(std::string_view xml, MModel& m) {
    Tokenizer tk{xml};
    Token t;
    while (tk.next(t)) {
        if (!(t.kind == TOK_START && t.name == "mujoco")) continue;
        while (tk.next(t)) {
            if (t.kind == TOK_END && t.name == "mujoco") break;
            if (t.kind != TOK_START) continue;
            if (t.name == "option") {
                // parser.zig:304-317: a fresh option record each time.
                m.timestep = 0.002f;
                m.gravity[0] = 0; m.gravity[1] = 0; m.gravity[2] = -9.81f;
                if (auto v = get_attr(t.attrs, "timestep")) { auto f = parse_float(*v); m.timestep = f ? *f : 0.002f; }
                if (auto v = get_attr(t.attrs, "gravity")) {
                    float g[3];
                    if (parse_vecn<3>(*v, g)) std::memcpy(m.gravity, g, sizeof g);
                    else { m.gravity[0] = 0; m.gravity[1] = 0; m.gravity[2] = -9.81f; }
                }
            } else if (t.name == "default") {
                parse_defaults(tk, m.defaults);
            } else if (t.name == "asset") {
                skip_section(tk, "asset");
            } else if (t.name == "worldbody") {
                parse_body_content(tk, m.worldbody, "worldbody", m.defaults, "main");
            } else if (t.name == "actuator") {
                parse_actuators(tk, m.actuators);
            } else if (t.name == "sensor") {
                parse_sensors(tk, m.sensors);
            } else if (t.name == "tendon") {
                skip_section(tk, "tendon");
            } else if (t.name == "equality") {
                skip_section(tk, "equality");
            }
        }
        break;
    }
}

// ----------------------------------------------------------------------------------
// Includes (parser.zig:62-188)
// ----------------------------------------------------------------------------------
std::optional<std::string_view> extract_attr(std::string_view tag, std::string_view name) {
    size_t search = 0;
    while (true) {
        size_t np = tag.find(name, search);
        if (np == std::string_view::npos) return std::nullopt;
        size_t pos = np + name.size();
        while (pos < tag.size() && (tag[pos] == ' ' || tag[pos] == '=' || tag[pos] == '\t')) ++pos;
        if (pos >= tag.size()) return std::nullopt;
        char q = tag[pos];
        if (q != '"' && q != '\'') { search = pos; continue; }
        ++pos;
        size_t vs = pos;
        while (pos < tag.size() && tag[pos] != q) ++pos;
        return tag.substr(vs, pos - vs);
    }
}

std::string path_join(const std::string& a, std::string_view b) {
    if (a.empty()) return std::string(b);
    std::string out = a;
    while (out.size() > 1 && out.back() == '/') out.pop_back();
    size_t i = 0;
    while (i < b.size() && b[i] == '/') ++i;
    out += '/';
    out += b.substr(i);
    return out;
}

std::string path_dirname(const std::string& p, const std::string& fallback) {
    std::string s = p;
    while (s.size() > 1 && s.back() == '/') s.pop_back();
    size_t slash = s.rfind('/');
    if (slash == std::string::npos) return fallback;
    if (slash == 0) return "/";
    return s.substr(0, slash);
}

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::ostringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return true;
}

std::string_view strip_mujoco_tags(std::string_view c) {
    size_t st = c.find("<mujoco");
    if (st == std::string_view::npos) return c;
    size_t gt = c.find('>', st);
    if (gt == std::string_view::npos) return c;
    size_t start = gt + 1;
    size_t end = c.rfind("</mujoco>");
    if (end == std::string_view::npos || end < start) return c;
    return c.substr(start, end - start);
}

std::string process_includes(const std::string& xml, const std::string& dir, int depth = 0) {
    if (xml.find("<include") == std::string::npos || depth > 32) return xml;
    std::string result;
    size_t pos = 0;
    while (pos < xml.size()) {
        size_t inc = xml.find("<include", pos);
        if (inc == std::string::npos) { result.append(xml, pos, std::string::npos); break; }
        result.append(xml, pos, inc - pos);
        size_t rel = xml.find("/>", inc);
        if (rel == std::string::npos) rel = xml.find('>', inc);
        if (rel == std::string::npos) { pos = inc + 8; continue; }
        size_t tag_end = rel - inc;
        std::string_view tag = std::string_view(xml).substr(inc, std::min(tag_end + 2, xml.size() - inc));
        if (auto file = extract_attr(tag, "file")) {
            std::string full = path_join(dir, *file);
            std::string content;
            if (!read_file(full, content)) {
                std::fprintf(stderr, "zeno_amd: could not include file '%s'\n", full.c_str());
                pos = inc + tag_end + 2;
                continue;
            }
            std::string sub = process_includes(content, path_dirname(full, dir), depth + 1);
            std::string_view stripped = strip_mujoco_tags(sub);
            result.append(stripped.data(), stripped.size());
        }
        pos = inc + tag_end + 2;
    }
    if (result.empty()) return xml;
    return result;
}

// ----------------------------------------------------------------------------------
// Mass and inertia (parser.zig:1026-1211), evaluated in f32 in the reference's order.
// ----------------------------------------------------------------------------------
constexpr float kPi = 3.14159265358979323846f;
constexpr float kFourThirds = 4.0f / 3.0f;

float fromto_half_len(const MGeom& g, float dflt) {
    if (!g.has_fromto) return dflt;
    float dx = g.fromto[3] - g.fromto[0];
    float dy = g.fromto[4] - g.fromto[1];
    float dz = g.fromto[5] - g.fromto[2];
    return std::sqrt(dx * dx + dy * dy + dz * dz) * 0.5f;
}

float geom_volume(const MGeom& g) {
    switch (g.type) {
        case MG_SPHERE: return kFourThirds * kPi * g.size[0] * g.size[0] * g.size[0];
        case MG_BOX: return 8.0f * g.size[0] * g.size[1] * g.size[2];
        case MG_CAPSULE: {
            float r = g.size[0];
            float hl = fromto_half_len(g, g.size[1]);
            float cyl = kPi * r * r * (2.0f * hl);
            float sph = kFourThirds * kPi * r * r * r;
            return cyl + sph;
        }
        case MG_CYLINDER: {
            float r = g.size[0];
            float hl = fromto_half_len(g, g.size[1]);
            return kPi * r * r * (2.0f * hl);
        }
        case MG_PLANE: return 1.0f;
        case MG_MESH: { float r = g.size[0]; return kFourThirds * kPi * r * r * r; }
        case MG_HFIELD: return 1.0f;
    }
    return 1.0f;
}

float geom_mass(const MGeom& g) {
    if (g.has_mass) return g.mass;
    return g.density * geom_volume(g);
}

void geom_inertia(const MGeom& g, float mass, float out[3]) {
    switch (g.type) {
        case MG_SPHERE: case MG_MESH: {
            float r = g.size[0];
            float i = 0.4f * mass * r * r;
            out[0] = out[1] = out[2] = i;
            return;
        }
        case MG_BOX: {
            float m12 = mass / 12.0f;
            float sx = g.size[0] * 2.0f, sy = g.size[1] * 2.0f, sz = g.size[2] * 2.0f;
            out[0] = m12 * (sy * sy + sz * sz);
            out[1] = m12 * (sx * sx + sz * sz);
            out[2] = m12 * (sx * sx + sy * sy);
            return;
        }
        case MG_CAPSULE: {
            float r = g.size[0];
            float hl = fromto_half_len(g, g.size[1]);
            float r2 = r * r;
            float h = 2.0f * hl;
            float h2 = h * h;
            float total_h = h + kFourThirds * r;
            float m_cyl = total_h > 0 ? mass * h / total_h : mass;
            float m_hem = (mass - m_cyl) * 0.5f;
            float i_cyl_axial = 0.5f * m_cyl * r2;
            float i_cyl_trans = m_cyl * (3.0f * r2 + h2) / 12.0f;
            float i_hem = 0.4f * m_hem * r2;
            float offset = h * 0.5f + 0.375f * r;
            float i_hem_trans = i_hem + m_hem * offset * offset;
            out[0] = i_cyl_trans + 2.0f * i_hem_trans;
            out[1] = i_cyl_trans + 2.0f * i_hem_trans;
            out[2] = i_cyl_axial + 2.0f * i_hem;
            return;
        }
        case MG_CYLINDER: {
            float r = g.size[0];
            float hl = fromto_half_len(g, g.size[1]);
            float r2 = r * r;
            float h = 2.0f * hl;
            out[0] = mass * (3.0f * r2 + h * h) / 12.0f;
            out[1] = mass * (3.0f * r2 + h * h) / 12.0f;
            out[2] = 0.5f * mass * r2;
            return;
        }
        default:
            out[0] = out[1] = out[2] = 0.0f;
            return;
    }
}

struct MassInertia {
    float mass;
    float inertia[3];
    float com[3];
};

MassInertia body_mass_inertia(const MBody& b) {
    MassInertia mi{1.0f, {0, 0, 0}, {0, 0, 0}};
    if (b.has_inertial) {
        const MInertial& in = b.inertial;
        if (in.has_diag) { mi.inertia[0] = in.diag[0]; mi.inertia[1] = in.diag[1]; mi.inertia[2] = in.diag[2]; }
        else if (in.has_full) { mi.inertia[0] = in.full[0]; mi.inertia[1] = in.full[1]; mi.inertia[2] = in.full[2]; }
        else {
            const float r = 0.05f;
            float i = 0.4f * in.mass * r * r;
            mi.inertia[0] = mi.inertia[1] = mi.inertia[2] = i;
        }
        mi.mass = in.mass;
        return mi;
    }
    if (b.geoms.empty()) return mi;
    float total_mass = 0.0f;
    float ti[3] = {0, 0, 0};
    float com[3] = {0, 0, 0};
    for (const MGeom& g : b.geoms) {
        float gm = geom_mass(g);
        float gi[3];
        geom_inertia(g, gm, gi);
        const float* d = g.pos;
        float dsq[3] = {d[0] * d[0], d[1] * d[1], d[2] * d[2]};
        ti[0] += gi[0] + gm * (dsq[1] + dsq[2]);
        ti[1] += gi[1] + gm * (dsq[0] + dsq[2]);
        ti[2] += gi[2] + gm * (dsq[0] + dsq[1]);
        com[0] += gm * d[0];
        com[1] += gm * d[1];
        com[2] += gm * d[2];
        total_mass += gm;
    }
    if (total_mass <= 0) total_mass = 1.0f;
    mi.mass = total_mass;
    for (int k = 0; k < 3; ++k) { mi.inertia[k] = ti[k]; mi.com[k] = com[k] / total_mass; }
    return mi;
}

// parser.zig:1213-1275
GeomDef convert_geom(const MGeom& mg) {
    GeomDef g;
    g.local_pos[0] = mg.pos[0]; g.local_pos[1] = mg.pos[1]; g.local_pos[2] = mg.pos[2];
    g.local_quat[0] = mg.quat[1]; g.local_quat[1] = mg.quat[2]; g.local_quat[2] = mg.quat[3]; g.local_quat[3] = mg.quat[0];
    g.friction = mg.friction[0];
    g.group = mg.contype;
    g.mask = mg.conaffinity;
    switch (mg.type) {
        case MG_SPHERE: g.geom_type = GEOM_SPHERE; g.size[0] = mg.size[0]; g.size[1] = 0; g.size[2] = 0; break;
        case MG_CAPSULE:
            g.geom_type = GEOM_CAPSULE;
            if (mg.has_fromto) {
                const float* f = mg.fromto;
                float dx = f[3] - f[0], dy = f[4] - f[1], dz = f[5] - f[2];
                float len = std::sqrt(dx * dx + dy * dy + dz * dz);
                g.local_pos[0] = (f[0] + f[3]) * 0.5f;
                g.local_pos[1] = (f[1] + f[4]) * 0.5f;
                g.local_pos[2] = (f[2] + f[5]) * 0.5f;
                g.size[0] = mg.size[0]; g.size[1] = len * 0.5f; g.size[2] = 0;
            } else {
                g.size[0] = mg.size[0]; g.size[1] = mg.size[1]; g.size[2] = 0;
            }
            break;
        case MG_BOX: g.geom_type = GEOM_BOX; g.size[0] = mg.size[0]; g.size[1] = mg.size[1]; g.size[2] = mg.size[2]; break;
        case MG_CYLINDER: g.geom_type = GEOM_CYLINDER; g.size[0] = mg.size[0]; g.size[1] = mg.size[1]; g.size[2] = 0; break;
        case MG_PLANE: g.geom_type = GEOM_PLANE; g.size[0] = g.size[1] = g.size[2] = 0; break;
        case MG_MESH: g.geom_type = GEOM_MESH; g.size[0] = 0.1f; g.size[1] = g.size[2] = 0; break;
        case MG_HFIELD: g.geom_type = GEOM_HFIELD; g.size[0] = g.size[1] = g.size[2] = 1; break;
    }
    return g;
}

// parser.zig:1333-1339, with f32 sin/cos.
void euler_to_quat(const float e[3], float q[4]) {
    float cr = std::cos(e[0] * 0.5f), sr = std::sin(e[0] * 0.5f);
    float cp = std::cos(e[1] * 0.5f), sp = std::sin(e[1] * 0.5f);
    float cy = std::cos(e[2] * 0.5f), sy = std::sin(e[2] * 0.5f);
    q[0] = sr * cp * cy - cr * sp * sy;
    q[1] = cr * sp * cy + sr * cp * sy;
    q[2] = cr * cp * sy - sr * sp * cy;
    q[3] = cr * cp * cy + sr * sp * sy;
}

// parser.zig:898-1009
void process_body(Scene& scene, const MBody& mb, int32_t parent_id, const float parent_pos[3]) {
    for (const MBody& child : mb.children) {
        float pos[3] = {child.pos[0] + parent_pos[0], child.pos[1] + parent_pos[1], child.pos[2] + parent_pos[2]};
        float quat[4];
        if (child.has_euler) euler_to_quat(child.euler, quat);
        else { quat[0] = child.quat[1]; quat[1] = child.quat[2]; quat[2] = child.quat[3]; quat[3] = child.quat[0]; }
        bool has_joints = !child.joints.empty();
        MassInertia mi = body_mass_inertia(child);
        BodyDef bd;
        bd.name = child.name;
        bd.parent_id = parent_id;
        bd.body_type = BODY_DYNAMIC;
        std::memcpy(bd.position, pos, sizeof pos);
        std::memcpy(bd.quaternion, quat, sizeof quat);
        bd.mass = mi.mass;
        std::memcpy(bd.inertia, mi.inertia, sizeof mi.inertia);
        std::memcpy(bd.com_offset, mi.com, sizeof mi.com);
        uint32_t body_id = scene.add_body(bd);

        if (!has_joints && parent_id >= 0) {
            JointDef jd;
            jd.joint_type = JOINT_FIXED;
            jd.parent_body = (uint32_t)parent_id;
            jd.child_body = body_id;
            std::memcpy(jd.anchor_parent, child.pos, sizeof child.pos);
            scene.add_joint(jd);
        }
        for (const MJoint& mj : child.joints) {
            JointDef jd;
            jd.name = mj.name;
            jd.parent_body = parent_id >= 0 ? (uint32_t)parent_id : 0u;
            jd.child_body = body_id;
            for (int k = 0; k < 3; ++k) jd.anchor_parent[k] = child.pos[k] + mj.pos[k];
            std::memcpy(jd.anchor_child, mj.pos, sizeof mj.pos);
            std::memcpy(jd.axis, mj.axis, sizeof mj.axis);
            jd.damping = mj.damping;
            jd.stiffness = mj.stiffness;
            jd.armature = mj.armature;
            jd.ref_position = mj.ref;
            switch (mj.type) {
                case MJ_FREE: jd.joint_type = JOINT_FREE; break;
                case MJ_BALL: jd.joint_type = JOINT_BALL; break;
                case MJ_SLIDE: jd.joint_type = JOINT_PRISMATIC; break;
                case MJ_HINGE: jd.joint_type = JOINT_REVOLUTE; break;
            }
            if (mj.has_range) {
                jd.limit_lower = mj.range[0];
                jd.limit_upper = mj.range[1];
                jd.limited = true;
            }
            scene.add_joint(jd);
        }
        for (const MGeom& mg : child.geoms) {
            GeomDef g = convert_geom(mg);
            g.body_id = body_id;
            scene.add_geom(mg.name, g);
        }
        process_body(scene, child, (int32_t)body_id, pos);
    }
}

// parser.zig:826-896
void convert_to_scene(const MModel& m, Scene& scene) {
    scene.physics.timestep = m.timestep;
    std::memcpy(scene.physics.gravity, m.gravity, sizeof m.gravity);
    BodyDef world;
    world.name = "world";
    world.body_type = BODY_STATIC;
    scene.add_body(world);
    for (const MGeom& mg : m.worldbody.geoms) {
        GeomDef g = convert_geom(mg);
        g.body_id = 0;
        scene.add_geom(mg.name, g);
    }
    const float zero[3] = {0, 0, 0};
    process_body(scene, m.worldbody, 0, zero);

    for (const MActuator& ma : m.actuators) {
        auto it = scene.joint_names.find(ma.joint);
        if (ma.joint.empty() || it == scene.joint_names.end()) continue;
        ActuatorDef a;
        a.name = ma.name;
        a.joint = it->second;
        a.gear = ma.gear;
        a.kp = ma.kp;
        a.kv = ma.kv;
        if (ma.has_ctrlrange) { a.ctrl_min = ma.ctrlrange[0]; a.ctrl_max = ma.ctrlrange[1]; }
        if (ma.has_forcerange) { a.force_min = ma.forcerange[0]; a.force_max = ma.forcerange[1]; }
        a.actuator_type = ma.type == MA_POSITION ? 1u : ma.type == MA_VELOCITY ? 2u : 0u;
        scene.add_actuator(a);
    }

    // Sensor conversion, parser.zig:1277-1330. Dimensions per type.
    static const uint32_t kTypeMap[12] = {S_JOINT_POS, S_JOINT_VEL, S_ACCELEROMETER, S_GYRO, S_TOUCH, S_FORCE,
                                          S_TORQUE, S_FRAMEPOS, S_FRAMEQUAT, S_FRAMELINVEL, S_FRAMEANGVEL,
                                          S_SUBTREECOM};
    static const uint32_t kDims[12] = {1, 1, 3, 3, 1, 3, 3, 3, 4, 3, 3, 3};
    for (const MSensor& ms : m.sensors) {
        SensorDef s;
        s.name = ms.name;
        s.noise = ms.noise;
        s.cutoff = ms.cutoff;
        s.sensor_type = kTypeMap[ms.type];
        s.dim = kDims[ms.type];
        if (ms.type == 0 || ms.type == 1) {
            auto it = scene.joint_names.find(ms.joint);
            s.object_id = (ms.joint.empty() || it == scene.joint_names.end()) ? 0u : it->second;
        }
        scene.add_sensor(s);
    }
    if (scene.sensors.empty()) scene.auto_add_sensors();
}

ParseResult parse_with_dir(const std::string& xml, const std::string& dir, Scene& out) {
    std::string merged = process_includes(xml, dir);
    MModel m;
    parse_xml(merged, m);
    out = Scene{};
    convert_to_scene(m, out);
    return {};
}

}  // namespace

ParseResult parse_mjcf_file(const std::string& path, Scene& out) {
    std::string content;
    if (!read_file(path, content)) return {-2, "file not found: " + path};
    return parse_with_dir(content, path_dirname(path, "."), out);
}

ParseResult parse_mjcf_string(const std::string& xml, Scene& out) {
    return parse_with_dir(xml, ".", out);
}

}  // namespace za
