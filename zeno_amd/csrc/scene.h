// Scene description built from MJCF: bodies, joints, geoms, actuators, sensors.
//
// Field meanings and defaults follow the reference's scene types:
//   BodyDef      src/physics/body.zig:17-75
//   JointDef     src/physics/joint.zig:23-69, ActuatorDef :103-116
//   Geom         src/collision/primitives.zig:135-166
//   Sensor       src/world/sensors.zig:36-52
//   PhysicsConfig src/physics/constants.zig:45-89
#pragma once
#include <cmath>
#include <cstdint>
#include <limits>
#include <string>
#include <unordered_map>
#include <vector>

#include "layout.h"

namespace za {

constexpr float kEpsilon = 1e-6f;  // constants.zig:13

enum BodyType : uint8_t { BODY_STATIC = 0, BODY_KINEMATIC = 1, BODY_DYNAMIC = 2 };

struct BodyDef {
    std::string name;
    BodyType body_type = BODY_DYNAMIC;
    float position[3] = {0, 0, 0};
    float quaternion[4] = {0, 0, 0, 1};  // xyzw
    float linear_velocity[3] = {0, 0, 0};
    float angular_velocity[3] = {0, 0, 0};
    float mass = 1.0f;
    float inertia[3] = {0, 0, 0};
    int32_t parent_id = -1;
    float linear_damping = 0.0f;
    float angular_damping = 0.0f;
    float gravity_scale = 1.0f;
    float com_offset[3] = {0, 0, 0};

    // body.zig:53-58: static, kinematic and non-positive mass bodies are immovable.
    float inv_mass() const {
        if (body_type == BODY_STATIC || body_type == BODY_KINEMATIC || mass <= 0.0f) return 0.0f;
        return 1.0f / mass;
    }
    // body.zig:62-75: per-axis inverse, zero for axes at or below EPSILON.
    void inv_inertia(float out[3]) const {
        for (int i = 0; i < 3; ++i) {
            if (body_type == BODY_STATIC || body_type == BODY_KINEMATIC) out[i] = 0.0f;
            else out[i] = inertia[i] > kEpsilon ? 1.0f / inertia[i] : 0.0f;
        }
    }
};

struct JointDef {
    std::string name;
    uint32_t joint_type = 1;  // JointType, default revolute
    uint32_t parent_body = 0;
    uint32_t child_body = 0;
    float anchor_parent[3] = {0, 0, 0};
    float anchor_child[3] = {0, 0, 0};
    float axis[3] = {0, 0, 1};
    float axis2[3] = {0, 1, 0};
    float limit_lower = -std::numeric_limits<float>::infinity();
    float limit_upper = std::numeric_limits<float>::infinity();
    float damping = 0.0f;
    float stiffness = 0.0f;
    float armature = 0.0f;
    float ref_position = 0.0f;
    bool limited = false;

    // joint.zig:72-74
    bool has_limits() const { return limited && limit_lower < limit_upper; }
};

struct GeomDef {
    uint32_t geom_type = 0;
    uint32_t body_id = 0;
    float local_pos[3] = {0, 0, 0};
    float local_quat[4] = {0, 0, 0, 1};
    float size[3] = {1, 1, 1};
    float friction = 1.0f;
    float restitution = 0.0f;
    uint32_t group = 0;           // MJCF contype
    uint32_t mask = 0xFFFFFFFFu;  // MJCF conaffinity
};

struct ActuatorDef {
    std::string name;
    uint32_t joint = 0;
    float ctrl_min = -1.0f;
    float ctrl_max = 1.0f;
    float force_min = -std::numeric_limits<float>::infinity();
    float force_max = std::numeric_limits<float>::infinity();
    float gear = 1.0f;
    uint32_t actuator_type = 0;  // motor, position, velocity
    float kp = 0.0f;
    float kv = 0.0f;
};

struct SensorDef {
    std::string name;
    uint32_t sensor_type = 0;
    uint32_t object_id = 0;
    uint32_t dim = 1;
    float noise = 0.0f;
    float cutoff = 0.0f;
};

struct PhysicsConfig {
    float gravity[3] = {0.0f, 0.0f, -9.81f};
    float timestep = 0.002f;
    float friction = 1.0f;
    float restitution = 0.0f;
    float baumgarte = 0.2f;
    float slop = 0.005f;
};

struct Scene {
    std::vector<BodyDef> bodies;
    std::vector<JointDef> joints;
    std::vector<GeomDef> geoms;
    std::vector<ActuatorDef> actuators;
    std::vector<SensorDef> sensors;
    uint32_t obs_dim = 0;  // sum of sensor dims (sensors.zig SensorConfig.total_dim)
    PhysicsConfig physics;
    std::unordered_map<std::string, uint32_t> body_names, joint_names, geom_names, actuator_names;

    uint32_t add_body(const BodyDef& b);
    uint32_t add_joint(const JointDef& j);
    uint32_t add_geom(const std::string& name, const GeomDef& g);
    uint32_t add_actuator(const ActuatorDef& a);
    void add_sensor(const SensorDef& s);
    // scene.zig:211-226 + sensors.zig:191-207
    void auto_add_sensors();
};

// Parse errors map onto the C ABI error codes (-2 file, -3 parse).
struct ParseResult {
    int error = 0;  // 0 ok, -2 file not found, -3 parse error
    std::string message;
};

// mjcf/parser.zig:22-51: parse a file (includes resolved relative to its directory).
ParseResult parse_mjcf_file(const std::string& path, Scene& out);
// mjcf/parser.zig:39-51: parse a string; includes resolve against ".".
ParseResult parse_mjcf_string(const std::string& xml, Scene& out);

}  // namespace za
