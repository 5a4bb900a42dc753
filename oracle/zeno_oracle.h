/*
 * CPU oracle for the batched physics step of Lulzx/zeno.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the CPU baseline; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The product
 * (zeno_amd/libzeno.so) never links or calls it.
 *
 * It restates, as scalar C, the reference's step: World.step / World.stepOnce
 * (src/world/world.zig:694-792, 934-1293) and every MSL kernel those dispatch
 * (src/shaders/all_shaders.metal). All records use the reference's byte layouts.
 *
 * The reference runs three of its kernels with unordered atomics or unsynchronised
 * parallel writes. The oracle uses the deterministic schedule documented for this build:
 *   S1 broad-phase pairs are appended in (g ascending, g' ascending) order;
 *   S2 joint forces are summed per body in ascending joint order, body_a before body_b;
 *   S3 joint constraints run per colour in colour-sorted template order;
 *   S4 contact slots are solved Gauss-Seidel in ascending slot order.
 * Transcendentals (atan2, asin) use a Cephes-style float routine (zo_atan2f, zo_asinf);
 * the fp32 step is compiled without FMA contraction.
 */
#ifndef ZENO_ORACLE_H
#define ZENO_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reference GPU records (byte layouts of world.zig:1573-1637, primitives.zig:424-442,
 * sensors.zig:149-161, xpbd.zig:50-121, contact.zig:210-247). */
typedef struct { float position[4], quaternion[4], inv_mass_inertia[4], params[4], com_offset[4]; } ZoBody;
typedef struct { float anchor_parent[4], anchor_child[4], axis[4], params[4], params2[4]; } ZoJoint;
typedef struct { uint32_t type_body[4]; float pos_size0[4], quat[4], params[4]; } ZoGeom;
typedef struct { float params[4], params2[4]; } ZoActuator;
typedef struct { uint32_t type_object[4]; float params[4]; } ZoSensor;
typedef struct { uint32_t indices[4]; float anchor_a[4], anchor_b[4], axis_target[4], limits[4], state[4]; } ZoConstraint;
typedef struct { float position_pen[4], normal_friction[4]; uint32_t indices[4]; float impulses[4]; } ZoContact;

/* One side of a pair for the extended narrow phase (narrow_phase.detectCollision,
 * src/collision/narrow_phase.zig:28-123): the geom's type, size and local position
 * (primitives.Geom) and its body's transform (body.Transform). 64 bytes. */
typedef struct {
    uint32_t type;         /* GeomType: 0 sphere, 1 capsule, 2 box, 3 plane; others: no contact */
    float size[3];         /* radius; radius, half length; half extents; plane offset */
    float local_pos[4];    /* w unused */
    float position[4];     /* w unused */
    float quaternion[4];   /* xyzw */
} ZoCollider;

/* narrow_phase.ContactResult (:12-25). All zero when there is no contact. 64 bytes. */
typedef struct {
    float point[3];
    float penetration;
    float normal[3];
    uint32_t valid;
    float local_a[4];      /* w 0 */
    float local_b[4];      /* w 0 */
} ZoContactResult;

/* Per-world constants: SimParams (world.zig:35-56) plus the uploaded scene records. */
typedef struct {
    uint32_t num_envs, num_bodies, num_joints, num_geoms, num_actuators, num_sensors, obs_dim;
    uint32_t num_constraints, num_colors, max_contacts, contact_iterations, config_substeps;
    float timestep; /* WorldConfig.timestep: the full step */
    float gravity[3];
    float friction, restitution, baumgarte, slop;
    const ZoBody* bodies;          /* [B] */
    const ZoJoint* joints;         /* [J] */
    const ZoGeom* geoms;           /* [G] */
    const ZoActuator* actuators;   /* [A] */
    const ZoSensor* sensors;       /* [S] */
    const uint32_t* color_ranges;  /* [num_colors][2] = (offset, count) */
    /* Extended-contact mode (not in the reference's step): 1 sends the pairs that the
     * reference's narrow_phase kernel leaves invalid through zo_detect_collision. */
    uint32_t extended_contacts;
} ZoModel;

/* Per-env state buffers in the reference layout (state.zig:56-117). J' = max(J,1),
 * O' = max(obs_dim,1). */
typedef struct {
    float* positions;           /* [E*B*4] */
    float* quaternions;         /* [E*B*4] */
    float* velocities;          /* [E*B*4] */
    float* angular_velocities;  /* [E*B*4] */
    float* accelerations;       /* [E*B*4] */
    float* inv_mass_inertia;    /* [E*B*4] */
    float* forces;              /* [E*B*4] */
    float* torques;             /* [E*B*4] */
    float* prev_positions;      /* [E*B*4] */
    float* prev_quaternions;    /* [E*B*4] */
    float* prev_velocities;     /* [E*B*4] */
    float* joint_positions;     /* [E*J'] */
    float* joint_velocities;    /* [E*J'] */
    float* joint_torques;       /* [E*J'] */
    float* observations;        /* [E*O'] */
    ZoContact* contacts;        /* [E*M] */
    uint32_t* contact_counts;   /* [E] */
    ZoContact* prev_contacts;   /* [E*M] */
    uint32_t* prev_contact_counts; /* [E] */
    ZoConstraint* constraints;  /* [E*N] */
    uint32_t* cell_ids;         /* [E*G] spatial-hash cell of each geom (G > 512); may be NULL otherwise */
} ZoState;

/* World.step (world.zig:694-746) for envs [env_begin, env_end): copies actions, runs
 * `substeps` (0 = the configured count) stepOnce passes, then writes accelerations.
 * nthreads <= 0 uses the OpenMP default. Returns 0. */
int zo_step(const ZoModel* m, ZoState* s, const float* actions, uint32_t substeps,
            uint32_t env_begin, uint32_t env_end, int nthreads);

/* Joint decomposition + constraint templates + greedy colouring + stable colour sort +
 * colour ranges (joint.zig:202-350, world.zig:311-501, xpbd.zig:533-640), recomputed from
 * the joint records. `limited` is JointDef.limited per joint. `out` must hold 3*J
 * records, `ranges` 512 entries. Returns the number of templates; *num_colors receives
 * the colour count. */
uint32_t zo_build_templates(const ZoJoint* joints, const uint8_t* limited, uint32_t num_joints,
                            const ZoBody* bodies, uint32_t num_bodies,
                            ZoConstraint* out, uint32_t* ranges, uint32_t* num_colors);

/* Math routines shared by the step, exported for their own accuracy tests. */
float zo_atan2f(float y, float x);
float zo_asinf(float x);

/* The O(G^2) broad phase, sort and narrow phase for one env (all_shaders.metal:468-533,
 * 711-894), exposed for unit tests: positions are [B*4] of that env. */
void zo_collide_env(const ZoModel* m, const float* positions, const float* quaternions,
                    ZoContact* contacts, uint32_t* count);

/* The spatial-hash broad phase (all_shaders.metal:556-703) for one env, whatever the geom
 * count, exposed for unit tests: cell_ids receives [G] cell ids; pairs are appended at
 * *count in the sequential order described in zeno_oracle.c. */
void zo_broad_phase_hash(const ZoModel* m, const float* positions, uint32_t* cell_ids,
                         ZoContact* contacts, uint32_t* count);

/* narrow_phase.detectCollision for one pair: 1 and *out filled on contact, else 0. */
int zo_detect_collision(const ZoCollider* a, const ZoCollider* b, ZoContactResult* out);
/* The same over n pairs; nthreads <= 0 uses the OpenMP default. */
void zo_detect_collisions(const ZoCollider* a, const ZoCollider* b, uint32_t n, ZoContactResult* out, int nthreads);

/* match_cached_contacts (all_shaders.metal:1483-1544) on one env, exposed for unit tests. */
void zo_match_cached(uint32_t max_contacts, ZoContact* contacts, uint32_t count,
                     ZoContact* prev_contacts, uint32_t prev_count);

/* solve_contacts (all_shaders.metal:1644-1793) on one slot, exposed for unit tests: the
 * slot's body indices address [num_bodies] float4 records of inverse mass and inertia,
 * positions, velocities and angular velocities; state and contact->impulses[0] are updated
 * in place. */
void zo_solve_contact_slot(uint32_t num_bodies, const float* inv_mass_inertia, float* positions, float* velocities,
                           float* angular_velocities, ZoContact* contact, float baumgarte, float slop, float dt);

/* sort_contacts (all_shaders.metal:711-745) on one env's list, exposed for unit tests. */
void zo_sort_contacts(uint32_t max_contacts, ZoContact* contacts, uint32_t count);

#ifdef __cplusplus
}
#endif
#endif
