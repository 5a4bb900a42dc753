// Fixed-size records shared by the host engine, the HIP kernels and the C ABI.
//
// Every record keeps the byte layout the reference publishes through its C ABI or
// uploads to its kernels, so that getters return bytes a reference caller can read
// unchanged.  Citations are paths inside Lulzx/zeno.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define ZA_HD __host__ __device__
#else
#define ZA_HD
#endif

namespace za {

// Spatial hash (all_shaders.metal:541-703, world.zig:533-569): used above 512 geoms, over a
// 64^3 grid of unit cells. The step kernel's sort key packs the geom index into 14 bits.
constexpr uint32_t kHashMinGeoms = 512;
constexpr uint32_t kHashMaxGeoms = 1u << 14;

// BodyDataGPU, src/world/world.zig:1573-1597 (80 B):
// position, quaternion (xyzw), inv_mass_inertia (inv_m, invI.xyz),
// params (parent_id, body_type, gravity_scale, linear_damping), com_offset.
struct alignas(16) BodyRec {
    float position[4];
    float quaternion[4];
    float inv_mass_inertia[4];
    float params[4];
    float com_offset[4];
};
static_assert(sizeof(BodyRec) == 80, "BodyRec layout");

// JointDataGPU, src/world/world.zig:1599-1620 (80 B):
// params = (type, parent, child, limit_lower), params2 = (limit_upper, damping, stiffness, ref).
struct alignas(16) JointRec {
    float anchor_parent[4];
    float anchor_child[4];
    float axis[4];
    float params[4];
    float params2[4];
};
static_assert(sizeof(JointRec) == 80, "JointRec layout");

// GeomGPU, src/collision/primitives.zig:424-442 (64 B):
// type_body = (type, body, conaffinity, contype); pos_size0 = (local pos, size0);
// quat = local quat (xyzw); params = (size1, size2, friction, restitution).
struct alignas(16) GeomRec {
    uint32_t type_body[4];
    float pos_size0[4];
    float quat[4];
    float params[4];
};
static_assert(sizeof(GeomRec) == 64, "GeomRec layout");

// ActuatorDataGPU, src/world/world.zig:1622-1637 (32 B):
// params = (joint, ctrl_min, ctrl_max, gear), params2 = (force_min, force_max, kp, kv).
struct alignas(16) ActuatorRec {
    float params[4];
    float params2[4];
};
static_assert(sizeof(ActuatorRec) == 32, "ActuatorRec layout");

// SensorGPU, src/world/sensors.zig:149-161 (32 B):
// type_object = (type, object, dim, 0); params = (noise, cutoff, dim, output offset).
struct alignas(16) SensorRec {
    uint32_t type_object[4];
    float params[4];
};
static_assert(sizeof(SensorRec) == 32, "SensorRec layout");

// XPBDConstraint, src/physics/xpbd.zig:50-121 (96 B):
// indices = (body_a, body_b, env, type | colour << 8).
struct alignas(16) ConstraintRec {
    uint32_t indices[4];
    float anchor_a[4];
    float anchor_b[4];
    float axis_target[4];
    float limits[4];
    float state[4];
};
static_assert(sizeof(ConstraintRec) == 96, "ConstraintRec layout");

// ContactGPU, src/physics/contact.zig:210-247 (64 B).
struct alignas(16) ContactRec {
    float position_pen[4];
    float normal_friction[4];
    uint32_t indices[4];
    float impulses[4];
};
static_assert(sizeof(ContactRec) == 64, "ContactRec layout");

// Geom type codes, src/collision/primitives.zig:124-132.
enum GeomType : uint32_t {
    GEOM_SPHERE = 0, GEOM_CAPSULE = 1, GEOM_BOX = 2, GEOM_PLANE = 3,
    GEOM_CYLINDER = 4, GEOM_MESH = 5, GEOM_HFIELD = 6
};

// Joint type codes, src/physics/joint.zig:7-20.
enum JointType : uint32_t {
    JOINT_FIXED = 0, JOINT_REVOLUTE = 1, JOINT_PRISMATIC = 2, JOINT_BALL = 3,
    JOINT_FREE = 4, JOINT_UNIVERSAL = 5
};

// XPBD constraint type codes, src/physics/xpbd.zig:23-46.
enum ConstraintType : uint32_t {
    C_CONTACT_NORMAL = 0, C_CONTACT_FRICTION = 1, C_POSITIONAL = 2, C_ANGULAR = 3,
    C_ANGULAR_LIMIT = 4, C_LINEAR_LIMIT = 5, C_TENDON = 6, C_WELD = 7, C_CONNECT = 8,
    C_JOINT_EQUALITY = 9, C_SLIDER = 10
};

// Sensor type codes, src/world/sensors.zig:6-33.
enum SensorType : uint32_t {
    S_JOINT_POS = 0, S_JOINT_VEL = 1, S_ACCELEROMETER = 2, S_GYRO = 3, S_TOUCH = 4,
    S_FORCE = 5, S_TORQUE = 6, S_FRAMEPOS = 7, S_FRAMEQUAT = 8, S_FRAMELINVEL = 9,
    S_FRAMEANGVEL = 10, S_SUBTREECOM = 11, S_USER = 12
};

}  // namespace za
