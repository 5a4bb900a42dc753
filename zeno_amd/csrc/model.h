// Device-ready model: the per-scene constant records the step reads, built once per world.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "layout.h"
#include "scene.h"

namespace za {

struct Model {
    uint32_t num_bodies = 0, num_joints = 0, num_geoms = 0, num_actuators = 0, num_sensors = 0;
    uint32_t obs_dim = 0;
    uint32_t num_constraints = 0;  // per env
    uint32_t num_colors = 0;
    uint32_t max_color_size = 0;
    uint32_t num_pairs = 0;        // broad-phase candidate pairs after static filters

    PhysicsConfig physics;

    std::vector<BodyRec> bodies;           // [B]
    std::vector<JointRec> joints;          // [J]
    std::vector<GeomRec> geoms;            // [G]
    std::vector<ActuatorRec> actuators;    // [A]
    std::vector<SensorRec> sensors;        // [S]
    std::vector<ConstraintRec> templates;  // [N], colour-sorted, env field 0
    std::vector<uint32_t> color_ranges;    // [num_colors][2] = (offset, count)
    std::vector<uint32_t> pairs;           // [P] = g | g' << 16, in (g, g') lexicographic order
    std::vector<uint8_t> joint_limited;    // [J] JointDef.limited

    // Initial state of one env (world.zig:663-691), float4 per body.
    std::vector<float> init_pos, init_quat, init_vel, init_angvel, inv_mass_inertia;
};

// Builds the model from a parsed scene: joint decomposition (joint.zig:202-350),
// constraint templates (world.zig:311-445), greedy colouring and stable colour sort
// (xpbd.zig:533-640), GPU records (world.zig:617-660) and the candidate pair list.
void build_model(const Scene& scene, Model& m);

// Greedy constraint colouring over template order (xpbd.zig:533-605). Writes the colour into
// bits 8..15 of indices[3] and returns the number of colours.
uint32_t color_constraints(std::vector<ConstraintRec>& cs, uint32_t num_bodies);

}  // namespace za
