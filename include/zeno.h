/*
 * zeno.h — C ABI of libzeno, the MI355X build of Lulzx/zeno's batched physics step.
 *
 * Every declaration here replaces the `export fn` of the same name in the reference's
 * src/main.zig and matches the cffi declaration in python/zeno/_ffi.py:41-301, so the
 * reference's Python bindings can load this library unchanged. Line numbers cite
 * src/main.zig unless stated otherwise.
 *
 * Differences from the reference that a caller can observe:
 *   - State lives in GPU memory. Getters return stable pinned host mirrors (one address per
 *     world for its lifetime) that are refreshed from the GPU each time the getter is
 *     called after a step; writes through these pointers are not propagated — use the
 *     set_* / reset_to_state calls.
 *   - zeno_world_step returns once the step is queued; every getter and setter waits for it.
 *   - zeno_metal_available() returns false; ZenoInfo.metal_available is false.
 *   - The zeno_swarm_* entry points are present for ABI compatibility and return
 *     ZENO_NOT_IMPLEMENTED (-7) or NULL: the swarm subsystem is not part of this build.
 */
#ifndef ZENO_H
#define ZENO_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ZenoWorldHandle;
typedef void* ZenoSwarmHandle;

/* main.zig:75-86 */
typedef struct {
    uint32_t num_envs;
    float timestep;               /* 0 = MJCF <option timestep> */
    uint32_t contact_iterations;  /* solver iterations for joints and contacts */
    uint32_t max_contacts_per_env;
    uint64_t seed;
    uint32_t substeps;
    bool enable_profiling;
    uint32_t max_bodies_per_env;  /* accepted, ignored (main.zig:156-164) */
    uint32_t max_joints_per_env;  /* accepted, ignored */
    uint32_t max_geoms_per_env;   /* accepted, ignored */
} ZenoConfig;

/* main.zig:89-102 */
typedef struct {
    uint32_t num_envs;
    uint32_t num_bodies;
    uint32_t num_joints;
    uint32_t num_actuators;
    uint32_t num_sensors;
    uint32_t num_geoms;
    uint32_t obs_dim;
    uint32_t action_dim;
    float timestep;
    uint64_t memory_usage;
    uint64_t gpu_memory_usage;
    bool metal_available;
} ZenoInfo;

/* main.zig:105-113 */
typedef struct {
    float integrate_ns;
    float collision_broad_ns;
    float collision_narrow_ns;
    float constraint_solve_ns;
    float total_step_ns;
    uint32_t num_contacts;
    uint32_t num_active_constraints;
} ZenoProfilingData;

/* main.zig:116-125 */
typedef enum {
    ZENO_SUCCESS = 0,
    ZENO_INVALID_HANDLE = -1,
    ZENO_FILE_NOT_FOUND = -2,
    ZENO_PARSE_ERROR = -3,
    ZENO_METAL_ERROR = -4, /* any GPU (HIP) failure */
    ZENO_OUT_OF_MEMORY = -5,
    ZENO_INVALID_ARGUMENT = -6,
    ZENO_NOT_IMPLEMENTED = -7
} ZenoError;

/* ---- World lifecycle ---------------------------------------------------------------- */
ZenoWorldHandle zeno_world_create(const char* mjcf_path, const ZenoConfig* config);       /* :139-179 */
ZenoWorldHandle zeno_world_create_from_string(const char* mjcf_string, const ZenoConfig* config); /* :181-216 */
void zeno_world_destroy(ZenoWorldHandle world);                                           /* :218-226 */

/* ---- Simulation ----------------------------------------------------------------------- */
int zeno_world_step(ZenoWorldHandle world, const float* actions, uint32_t substeps);      /* :228-245 */
int zeno_world_step_subset(ZenoWorldHandle world, const float* actions, const uint8_t* env_mask,
                           uint32_t substeps);                                            /* :247-268 */
int zeno_world_reset(ZenoWorldHandle world, const uint8_t* env_mask);                     /* :271-288 */
int zeno_world_reset_to_state(ZenoWorldHandle world, const float* positions, const float* quaternions,
                              const float* velocities, const float* angular_velocities,
                              const uint8_t* env_mask);                                   /* :290-385 */

/* ---- State access (stable host mirrors) ----------------------------------------------- */
float* zeno_world_get_observations(ZenoWorldHandle world);             /* :388-394 */
float* zeno_world_get_rewards(ZenoWorldHandle world);                  /* :396-402 */
uint8_t* zeno_world_get_dones(ZenoWorldHandle world);                  /* :404-410 */
float* zeno_world_get_body_positions(ZenoWorldHandle world);           /* :485-494 */
float* zeno_world_get_body_quaternions(ZenoWorldHandle world);         /* :496-505 */
float* zeno_world_get_body_velocities(ZenoWorldHandle world);          /* :507-513 */
float* zeno_world_get_body_angular_velocities(ZenoWorldHandle world);  /* :515-521 */
float* zeno_world_get_body_accelerations(ZenoWorldHandle world);       /* :523-529 */
float* zeno_world_get_joint_positions(ZenoWorldHandle world);          /* :531-537 */
float* zeno_world_get_joint_velocities(ZenoWorldHandle world);         /* :539-545 */
float* zeno_world_get_joint_forces(ZenoWorldHandle world);             /* :547-555 */
void* zeno_world_get_contacts(ZenoWorldHandle world);                  /* :573-579 */
uint32_t* zeno_world_get_contact_counts(ZenoWorldHandle world);        /* :557-563 */
float* zeno_world_get_sensor_data(ZenoWorldHandle world);              /* :565-571 */

/* ---- State mutation ------------------------------------------------------------------- */
int zeno_world_set_body_positions(ZenoWorldHandle world, const float* positions, const uint8_t* env_mask);   /* :581-606 */
int zeno_world_set_body_velocities(ZenoWorldHandle world, const float* velocities, const uint8_t* env_mask); /* :608-631 */
int zeno_world_set_gravity(ZenoWorldHandle world, float gx, float gy, float gz);                             /* :633-648 */
int zeno_world_set_timestep(ZenoWorldHandle world, float timestep);                                          /* :650-664 */

/* ---- Metadata ------------------------------------------------------------------------- */
uint32_t zeno_world_num_envs(ZenoWorldHandle world);      /* :412-418 */
uint32_t zeno_world_num_bodies(ZenoWorldHandle world);    /* :420-426 */
uint32_t zeno_world_num_joints(ZenoWorldHandle world);    /* :428-434 */
uint32_t zeno_world_num_sensors(ZenoWorldHandle world);   /* :436-442 */
uint32_t zeno_world_obs_dim(ZenoWorldHandle world);       /* :444-450 */
uint32_t zeno_world_action_dim(ZenoWorldHandle world);    /* :452-458 */
int zeno_world_get_info(ZenoWorldHandle world, ZenoInfo* info);  /* :460-483 */

/* ---- Profiling ------------------------------------------------------------------------ */
int zeno_world_get_profiling(ZenoWorldHandle world, ZenoProfilingData* data);  /* :666-684 */
void zeno_world_reset_profiling(ZenoWorldHandle world);                        /* :686-691 */

/* ---- Utility -------------------------------------------------------------------------- */
const char* zeno_version(void);                     /* :721-724 */
bool zeno_metal_available(void);                    /* :733-736 */
const char* zeno_error_string(int error_code);      /* :706-719 */
uint64_t zeno_world_memory_usage(ZenoWorldHandle world);   /* :693-699 */
void zeno_world_compact_memory(ZenoWorldHandle world);     /* :701-704 (no-op) */
uint32_t zeno_world_max_contacts_per_env(ZenoWorldHandle world);  /* :726-731 */

/* ---- Swarm ABI (not built: stubs), _ffi.py:220-301, main.zig:756-910 ------------------ */
typedef struct {
    uint32_t num_agents;
    float communication_range;
    uint32_t max_neighbors;
    uint32_t max_message_bytes;
    uint32_t max_messages_per_step;
    float grid_cell_size;
    uint64_t seed;
    bool enable_physics;
    uint32_t latency_ticks;
    float drop_prob;
    uint32_t max_broadcast_recipients;
    uint32_t max_inbox_per_agent;
    bool strict_determinism;
    uint8_t _pad[2];
} ZenoSwarmConfig;

typedef struct {
    float connectivity_ratio;
    float fragmentation_score;
    uint32_t collision_count;
    uint32_t message_count;
    uint32_t bytes_sent;
    uint32_t total_edges;
    float avg_neighbors;
    uint32_t messages_dropped;
    float convergence_time_ms;
    uint32_t near_miss_count;
    float task_success;
    uint32_t _pad;
} ZenoSwarmMetrics;

typedef struct {
    uint32_t agent_id;
    uint32_t team_id;
    uint32_t status;
    uint32_t flags;
    float local_state[4];
} ZenoAgentState;

typedef struct {
    float score;
    bool complete;
    uint8_t _pad1[3];
    float detail[4];
} ZenoTaskResult;

typedef struct {
    uint32_t attack_type;
    float intensity;
    uint32_t target_agents[16];
    uint32_t num_targets;
    uint32_t seed;
    uint32_t _pad[2];
} ZenoAttackConfig;

typedef struct {
    uint64_t frame_count;
    uint64_t total_bytes;
    bool recording;
    uint8_t _pad[7];
} ZenoReplayStats;

ZenoSwarmHandle zeno_swarm_create(ZenoWorldHandle world, const ZenoSwarmConfig* config);   /* :756-771 */
void zeno_swarm_destroy(ZenoSwarmHandle swarm);                                            /* :773-781 */
int zeno_swarm_step(ZenoSwarmHandle swarm, ZenoWorldHandle world, float* actions);          /* :783-808 */
int zeno_swarm_get_metrics(ZenoSwarmHandle swarm, ZenoSwarmMetrics* metrics);              /* :810-816 */
ZenoAgentState* zeno_swarm_get_agent_states(ZenoSwarmHandle swarm);                        /* :818-824 */
int zeno_swarm_get_neighbor_counts(ZenoSwarmHandle swarm, uint32_t* out, uint32_t count);  /* :826-832 */
void zeno_swarm_set_body_offset(ZenoSwarmHandle swarm, uint32_t offset);                   /* :834-839 */
int zeno_swarm_evaluate_task(ZenoSwarmHandle swarm, void* world, uint32_t task_type,
                             const float params[8], ZenoTaskResult* result);               /* :841-860 */
int zeno_swarm_apply_attack(ZenoSwarmHandle swarm, const ZenoAttackConfig* config);        /* :862-871 */
uint32_t* zeno_swarm_get_neighbor_index_ptr(ZenoSwarmHandle swarm);                        /* :873-879 */
uint32_t* zeno_swarm_get_neighbor_row_ptr(ZenoSwarmHandle swarm);                          /* :881-887 */
int zeno_swarm_start_recording(ZenoSwarmHandle swarm);                                     /* :889-895 */
int zeno_swarm_stop_recording(ZenoSwarmHandle swarm);                                      /* :897-903 */
int zeno_swarm_get_replay_stats(ZenoSwarmHandle swarm, ZenoReplayStats* stats);            /* :905-911 */

#ifdef __cplusplus
}
#endif
#endif /* ZENO_H */
