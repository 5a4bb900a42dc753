/*
 * zeno_amd_ext.h — extension entry points of libzeno (MI355X build).
 *
 * None of these exist in the reference's C ABI (Lulzx/zeno); they sit beside the reference
 * ABI of zeno.h and serve four callers:
 *   - inspection of the model a world was built from (tests and the CPU oracle read the
 *     constraint templates, colours and records the kernels use), without a GPU;
 *   - device-resident stepping and timing for benchmarks and graph capture;
 *   - solver state that the reference keeps but never exposes (lambda, previous contact
 *     count, spatial-hash cells), used by parity tests;
 *   - the reference's Zig-level collision routine (narrow_phase.detectCollision) for C
 *     callers, batched on the GPU.
 */
#ifndef ZENO_AMD_EXT_H
#define ZENO_AMD_EXT_H

#include <stdint.h>

#include "zeno.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ZenoAmdModelHandle;

/* A parsed scene and the records the step reads. Pointers stay valid until the model (or
 * world) is destroyed. Record layouts are the reference's GPU layouts:
 * bodies 80 B (world.zig:1573-1597), joints 80 B (world.zig:1599-1620),
 * geoms 64 B (primitives.zig:424-442), actuators 32 B (world.zig:1622-1637),
 * sensors 32 B (sensors.zig:149-161), constraint templates 96 B (xpbd.zig:50-121). */
typedef struct {
    uint32_t num_bodies, num_joints, num_geoms, num_actuators, num_sensors, obs_dim;
    uint32_t num_constraints, num_colors, max_color_size, num_pairs;
    float timestep;      /* MJCF <option timestep> */
    float gravity[3];
    float friction, restitution, baumgarte, slop;
    const void* bodies;
    const void* joints;
    const void* geoms;
    const void* actuators;
    const void* sensors;
    const void* constraints;          /* colour-sorted templates (env 0) */
    const uint32_t* color_ranges;     /* [num_colors][2] = (offset, count) */
    const uint32_t* pairs;            /* [num_pairs] = g | g' << 16, broad-phase candidates */
    const uint8_t* joint_limited;     /* [num_joints] JointDef.limited */
    const float* init_positions;      /* [num_bodies*4] initial state of every env */
    const float* init_quaternions;
    const float* init_velocities;
    const float* init_angular_velocities;
    const float* inv_mass_inertia;    /* [num_bodies*4] */
} ZenoAmdModelView;

/* Parse MJCF and build the model on the host only (no GPU needed). NULL on failure; the
 * reason is available from zeno_amd_last_error(). */
ZenoAmdModelHandle zeno_amd_model_create(const char* mjcf_path);
ZenoAmdModelHandle zeno_amd_model_create_from_string(const char* mjcf_string);
void zeno_amd_model_destroy(ZenoAmdModelHandle model);
int zeno_amd_model_view(ZenoAmdModelHandle model, ZenoAmdModelView* out);

/* The model a world runs. */
int zeno_amd_world_model_view(ZenoWorldHandle world, ZenoAmdModelView* out);

/* Message of the last failure on this thread ("" when none). */
const char* zeno_amd_last_error(void);

/* Number of GPUs HIP reports (0 when none or when the runtime is unavailable). */
int zeno_amd_device_count(void);

/* Solver state that the reference keeps in device buffers without a getter:
 * lambda per env and constraint (XPBDConstraint.state.x == state.y after every step),
 * and prev_contact_counts. Copies into caller memory; returns 0 or an error code. */
int zeno_amd_world_get_lambda(ZenoWorldHandle world, float* out /* [E*N] */);
int zeno_amd_world_get_prev_contact_counts(ZenoWorldHandle world, uint32_t* out /* [E] */);

/* Set every env's contact count (u32, never cleared by a step, so it wraps after 2^32
 * appends). Replaces a caller's write through the pointer zeno_world_get_contact_counts
 * returns, which is shared memory in the reference (src/main.zig:557-560). Copies from caller
 * memory; held views follow; returns 0 or an error code. */
int zeno_amd_world_set_contact_counts(ZenoWorldHandle world, const uint32_t* counts /* [E] */);

/* Step with actions already in device memory (d_actions: [E*A] floats on the world's
 * device). Same semantics as zeno_world_step. */
int zeno_amd_world_step_device(ZenoWorldHandle world, const float* d_actions, uint32_t substeps);

/* Waits for all work queued on the world's stream. */
int zeno_amd_world_synchronize(ZenoWorldHandle world);

/* Kernel timing with HIP events on the world's stream. enable = k > 0 records an event pair
 * around every k-th step launch (k = 1: every launch), 0 stops; get returns the summed
 * kernel time in ms of the timed launches and their number (waits for the stream). */
int zeno_amd_world_set_kernel_timing(ZenoWorldHandle world, int enable);
int zeno_amd_world_get_kernel_timing(ZenoWorldHandle world, double* total_ms, uint64_t* launches);

/* Launch configuration chosen for the world: environments per wavefront and LDS bytes
 * per workgroup (with the working sets in HBM, the contact and hash arrays kept in LDS). */
/* No counterpart in the reference: the number of joint-solve phases per solver iteration
 * (same-type runs of one colour, after the constraints that can never act are left out: those
 * with nothing to move and angular limits whose bounds lie beyond +-2 pi). 0 for NULL. */
uint32_t zeno_amd_world_joint_phases(ZenoWorldHandle world);
int zeno_amd_world_launch_config(ZenoWorldHandle world, uint32_t* envs_per_wave, uint32_t* lds_bytes);

/* Environment groups per workgroup of the world's step launches (1..4; with the model records
 * in LDS, the groups of a workgroup share one copy of them), one wave each, or two with split
 * groups. 0 for an invalid handle. */
uint32_t zeno_amd_world_waves_per_group(ZenoWorldHandle world);

/* No counterpart in the reference (a launch-shape query). 1 when each environment group runs
 * on two waves: one solving the joints and contacts, one running the contact pipeline (broad
 * phase to contact levels) meanwhile; 0 when one wave does both; -1 for an invalid handle. */
int zeno_amd_world_split_groups(ZenoWorldHandle world);

/* *placement: where the step kernel keeps the scene's model records and each environment's
 * working set. 0 = both in LDS (several environments per workgroup); 1 = model records read
 * from HBM, working set in LDS; 2 = both in HBM, the contact pipeline's arrays in LDS; 3 = all
 * in HBM, no LDS (contact lists too long for LDS). The world picks, among 0-2, the one that
 * keeps the most environments resident on the GPU (HIP occupancy query), and 3 when none of
 * them fits; ZENO_AMD_PLACEMENT=0/1/2/3 at create forces one.
 * *spatial_hash = 1 when the scene has more than 512 geoms and the spatial-hash broad
 * phase runs (world.zig:534, all_shaders.metal:541-703). Either pointer may be null. */
int zeno_amd_world_modes(ZenoWorldHandle world, int* placement, int* spatial_hash);

/* Extended-contact mode, off by default (the reference's step has no such mode). With
 * enable != 0, the geom pairs that the reference's narrow_phase kernel leaves invalid
 * (all_shaders.metal:794-893: everything but sphere-sphere, sphere-plane and capsule-plane)
 * are tested with narrow_phase.detectCollision (narrow_phase.zig:28-123) on the bodies'
 * poses, so boxes and capsules collide with each other and with spheres; their contacts
 * enter the contact list and the solve like the others. Takes effect at the next step. */
int zeno_amd_world_set_extended_contacts(ZenoWorldHandle world, int enable);

/* Captures num_steps consecutive steps into a HIP graph held by the world (replacing an
 * earlier one); nothing runs until zeno_amd_world_graph_launch. Step k reads its actions
 * at (const char*)d_actions + k * action_stride_bytes (device memory, E x action_dim f32
 * each; ignored for scenes without actuators), with substeps as in zeno_world_step. The
 * graph keeps the kernel arguments of capture time: the setters of timestep, gravity and the
 * extended-contact mode, and the first zeno_world_step_subset (which allocates its buffers),
 * release it. No counterpart in the reference (its loop is one zeno_world_step per step);
 * for callers that replay a fixed device-resident action schedule. */
int zeno_amd_world_capture_steps(ZenoWorldHandle world, const float* d_actions, uint64_t action_stride_bytes,
                                 uint32_t num_steps, uint32_t substeps);
/* Enqueues the captured steps once on the world's stream; returns after enqueueing
 * (zeno_amd_world_synchronize waits). ZENO_INVALID_ARGUMENT when nothing is captured. */
int zeno_amd_world_graph_launch(ZenoWorldHandle world);
int zeno_amd_world_release_graph(ZenoWorldHandle world);

/* The spatial hash's cell of every geom in the last substep, [E*G] u32: x + 64 y + 4096 z
 * of the clamped unit-cell coordinates, the reference's cell_ids buffer
 * (world.zig:140,548; all_shaders.metal:576-582), which it keeps without a getter.
 * ZENO_INVALID_ARGUMENT when the scene does not use the spatial hash. */
int zeno_amd_world_get_cell_ids(ZenoWorldHandle world, uint32_t* out /* [E*G] */);

/* ---- Extended narrow phase ---------------------------------------------------------
 * The reference's host-side collision routine narrow_phase.detectCollision(geom_a,
 * transform_a, geom_b, transform_b) ?ContactResult (src/collision/narrow_phase.zig:28-123,
 * exported through the `zeno` Zig module, src/main.zig:28; it has no C entry point there),
 * batched on the GPU. Pairs handled: sphere-sphere, sphere-capsule, sphere-box,
 * sphere-plane, capsule-capsule, capsule-plane, box-plane, box-box (separating axes), in
 * either operand order; every other pair (capsule-box, cylinder, mesh, heightfield, plane-
 * plane) reports no contact. */

/* One operand: the geom's type, size and local position (primitives.Geom,
 * primitives.zig:135-166) and its body's transform (body.Transform, body.zig:141-143).
 * 64 bytes. */
typedef struct {
    uint32_t type;         /* 0 sphere, 1 capsule, 2 box, 3 plane, 4 cylinder, 5 mesh, 6 heightfield */
    float size[3];         /* radius | radius, half length | half extents | plane offset */
    float local_pos[4];    /* w unused */
    float position[4];     /* w unused */
    float quaternion[4];   /* xyzw */
} ZenoAmdCollider;

/* narrow_phase.ContactResult (narrow_phase.zig:12-25); all zero with valid = 0 where the
 * reference returns null. 64 bytes. */
typedef struct {
    float point[3];
    float penetration;
    float normal[3];       /* from a to b */
    uint32_t valid;
    float local_a[4];      /* w 0 */
    float local_b[4];      /* w 0 */
} ZenoAmdContactResult;

/* detectCollision(a[i], b[i]) -> out[i] for i < n. Device pointers; enqueued on `stream`
 * (a hipStream_t; null = the default stream), returns after enqueueing. */
int zeno_amd_detect_collisions(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n,
                               ZenoAmdContactResult* out, void* stream);

/* The same on host arrays: copies in, runs on the current device, copies back, waits. */
int zeno_amd_detect_collisions_host(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n,
                                    ZenoAmdContactResult* out);

/* No counterpart in the reference. zeno_amd_detect_collisions_host for callers that cannot
 * allocate device memory (serving loops and harnesses that forbid hipMalloc): the operands
 * and results are staged in a static device array of ZENO_AMD_NOALLOC_MAX_PAIRS pairs
 * (3 MiB on each GPU the library runs on, held until the process ends) instead of buffers
 * allocated per call, and nothing is allocated or freed. n above that limit returns
 * ZENO_INVALID_ARGUMENT. Runs on the current device and waits. Every call on one GPU shares
 * that GPU's array, so calls on one GPU from several host threads take turns: each holds a
 * per-device lock from its first copy in until its results are back. */
#define ZENO_AMD_NOALLOC_MAX_PAIRS 16384u
int zeno_amd_detect_collisions_host_noalloc(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n,
                                            ZenoAmdContactResult* out);

/* No counterpart in the reference: a self-check of the device arithmetic the step relies on.
 * q[i] = a[i] / b[i] evaluated the way the step kernel divides several numbers by one divisor
 * (one fp64 reciprocal from v_rcp_f64 and its cubic correction, then fp32(a * y) with exact
 * subnormal ties rounded to even), which must give the bits of the IEEE fp32 division for
 * every input. Host arrays; runs on the current device and waits. */
int zeno_amd_selfcheck_divide(const float* a, const float* b, float* q, uint32_t n);

/* No counterpart in the reference: a self-check of the device arithmetic the step relies on.
 * y[i] = sqrt(x[i]) evaluated the way the step kernel takes the square roots it compares
 * against a threshold (v_sqrt_f32 and the one-ulp correction, without the scaling of inputs
 * below 2^-96), which must give the bits of the IEEE fp32 square root for every x >= 2^-96
 * and for +-0, +inf, NaN and negative x, and a value below 2^-47 for 0 < x < 2^-96. Host
 * arrays; runs on the current device and waits. */
int zeno_amd_selfcheck_sqrt(const float* x, float* y, uint32_t n);

/* No counterpart in the reference: a self-check of the device arithmetic the step relies on.
 * *max_err = the largest |1 - b y| over every finite nonzero fp32 b, with y the fp64
 * reciprocal the step divides by (v_rcp_f64 and its cubic correction). The quotients a * y are
 * the correctly rounded fp32 a / b when this is below about 2^-49.1. Runs on the current
 * device (2^32 divisors, well under a second) and waits. */
int zeno_amd_selfcheck_reciprocal_error(double* max_err);

#ifdef __cplusplus
}
#endif
#endif /* ZENO_AMD_EXT_H */
