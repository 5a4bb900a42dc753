// C ABI of libzeno: the reference's zeno_* exports (src/main.zig:139-910) plus the
// zeno_amd_* extensions declared in include/zeno_amd_ext.h.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <new>
#include <string>

#include "../../include/zeno.h"
#include "../../include/zeno_amd_ext.h"
#include "collide.h"
#include "world.h"

using za::World;

namespace {

thread_local std::string g_last_error;

void set_error(const std::string& s) {
    g_last_error = s;
    if (!s.empty()) std::fprintf(stderr, "zeno_amd: %s\n", s.c_str());
}

World* W(ZenoWorldHandle h) { return static_cast<World*>(h); }

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return ZENO_SUCCESS;
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return ZENO_METAL_ERROR;
}

struct ModelBox {
    za::Scene scene;
    za::Model model;
};

void fill_view(const za::Model& m, ZenoAmdModelView* v) {
    std::memset(v, 0, sizeof *v);
    v->num_bodies = m.num_bodies;
    v->num_joints = m.num_joints;
    v->num_geoms = m.num_geoms;
    v->num_actuators = m.num_actuators;
    v->num_sensors = m.num_sensors;
    v->obs_dim = m.obs_dim;
    v->num_constraints = m.num_constraints;
    v->num_colors = m.num_colors;
    v->max_color_size = m.max_color_size;
    v->num_pairs = m.num_pairs;
    v->timestep = m.physics.timestep;
    std::memcpy(v->gravity, m.physics.gravity, sizeof v->gravity);
    v->friction = m.physics.friction;
    v->restitution = m.physics.restitution;
    v->baumgarte = m.physics.baumgarte;
    v->slop = m.physics.slop;
    v->bodies = m.bodies.data();
    v->joints = m.joints.data();
    v->geoms = m.geoms.data();
    v->actuators = m.actuators.data();
    v->sensors = m.sensors.data();
    v->constraints = m.templates.data();
    v->color_ranges = m.color_ranges.data();
    v->pairs = m.pairs.data();
    v->joint_limited = m.joint_limited.data();
    v->init_positions = m.init_pos.data();
    v->init_quaternions = m.init_quat.data();
    v->init_velocities = m.init_vel.data();
    v->init_angular_velocities = m.init_angvel.data();
    v->inv_mass_inertia = m.inv_mass_inertia.data();
}

ZenoWorldHandle create_world(const za::Scene& scene, const ZenoConfig* config) {
    if (!config) { set_error("null config"); return nullptr; }
    std::string err;
    World* w = nullptr;
    try {
        w = World::create(scene, *config, err);
    } catch (const std::bad_alloc&) {
        err = "out of memory";
    }
    if (!w) { set_error("failed to create world: " + err); return nullptr; }
    g_last_error.clear();
    return w;
}

}  // namespace

extern "C" {

// ---- World lifecycle ----------------------------------------------------------------------
ZenoWorldHandle zeno_world_create(const char* mjcf_path, const ZenoConfig* config) {
    if (!mjcf_path) { set_error("null path"); return nullptr; }
    za::Scene scene;
    za::ParseResult r = za::parse_mjcf_file(mjcf_path, scene);
    if (r.error) { set_error("Failed to parse MJCF: " + r.message); return nullptr; }
    return create_world(scene, config);
}

ZenoWorldHandle zeno_world_create_from_string(const char* mjcf_string, const ZenoConfig* config) {
    if (!mjcf_string) { set_error("null MJCF string"); return nullptr; }
    za::Scene scene;
    za::ParseResult r = za::parse_mjcf_string(mjcf_string, scene);
    if (r.error) { set_error("Failed to parse MJCF: " + r.message); return nullptr; }
    return create_world(scene, config);
}

void zeno_world_destroy(ZenoWorldHandle world) {
    if (!world) return;
    delete W(world);
}

// ---- Simulation ---------------------------------------------------------------------------
int zeno_world_step(ZenoWorldHandle world, const float* actions, uint32_t substeps) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    if (!actions && w->A > 0) return ZENO_INVALID_ARGUMENT;
    return hip_status(w->step(actions, substeps, false), "step");
}

int zeno_world_step_subset(ZenoWorldHandle world, const float* actions, const uint8_t* env_mask, uint32_t substeps) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    if (!env_mask || (!actions && w->A > 0)) return ZENO_INVALID_ARGUMENT;
    return hip_status(w->step_subset(actions, env_mask, substeps), "step_subset");
}

int zeno_world_reset(ZenoWorldHandle world, const uint8_t* env_mask) {
    if (!world) return ZENO_INVALID_HANDLE;
    return hip_status(W(world)->reset(env_mask), "reset");
}

int zeno_world_reset_to_state(ZenoWorldHandle world, const float* positions, const float* quaternions,
                              const float* velocities, const float* angular_velocities, const uint8_t* env_mask) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!positions || !quaternions) return ZENO_INVALID_ARGUMENT;
    return hip_status(W(world)->reset_to_state(positions, quaternions, velocities, angular_velocities, env_mask),
                      "reset_to_state");
}

// ---- State access -------------------------------------------------------------------------
float* zeno_world_get_observations(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_OBS) : nullptr;
}
float* zeno_world_get_rewards(ZenoWorldHandle world) { return world ? W(world)->h_rewards : nullptr; }
uint8_t* zeno_world_get_dones(ZenoWorldHandle world) { return world ? W(world)->h_dones : nullptr; }
float* zeno_world_get_body_positions(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_POS) : nullptr;
}
float* zeno_world_get_body_quaternions(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_QUAT) : nullptr;
}
float* zeno_world_get_body_velocities(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_VEL) : nullptr;
}
float* zeno_world_get_body_angular_velocities(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_ANGVEL) : nullptr;
}
float* zeno_world_get_body_accelerations(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_ACC) : nullptr;
}
float* zeno_world_get_joint_positions(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_JPOS) : nullptr;
}
float* zeno_world_get_joint_velocities(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_JVEL) : nullptr;
}
float* zeno_world_get_joint_forces(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_JTRQ) : nullptr;
}
void* zeno_world_get_contacts(ZenoWorldHandle world) {
    if (!world || W(world)->M == 0) return nullptr;
    return W(world)->mirror(za::MIR_CON);
}
uint32_t* zeno_world_get_contact_counts(ZenoWorldHandle world) {
    return world ? (uint32_t*)W(world)->mirror(za::MIR_COUNT) : nullptr;
}
// world.zig:1398-1403: sensor readings live in the observation buffer.
float* zeno_world_get_sensor_data(ZenoWorldHandle world) {
    return world ? (float*)W(world)->mirror(za::MIR_OBS) : nullptr;
}

// ---- State mutation -----------------------------------------------------------------------
int zeno_world_set_body_positions(ZenoWorldHandle world, const float* positions, const uint8_t* env_mask) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!positions) return ZENO_INVALID_ARGUMENT;
    World* w = W(world);
    if (hipSetDevice(w->device) != hipSuccess) return ZENO_METAL_ERROR;
    return hip_status(w->set_state_array(w->d_pos, za::MIR_POS, positions, env_mask), "set_body_positions");
}

int zeno_world_set_body_velocities(ZenoWorldHandle world, const float* velocities, const uint8_t* env_mask) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!velocities) return ZENO_INVALID_ARGUMENT;
    World* w = W(world);
    if (hipSetDevice(w->device) != hipSuccess) return ZENO_METAL_ERROR;
    return hip_status(w->set_state_array(w->d_vel, za::MIR_VEL, velocities, env_mask), "set_body_velocities");
}

int zeno_world_set_gravity(ZenoWorldHandle world, float gx, float gy, float gz) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    w->release_graph();
    w->gravity[0] = gx;
    w->gravity[1] = gy;
    w->gravity[2] = gz;
    return ZENO_SUCCESS;
}

int zeno_world_set_timestep(ZenoWorldHandle world, float timestep) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (timestep <= 0) return ZENO_INVALID_ARGUMENT;  // NaN passes, as in main.zig:655
    World* w = W(world);
    w->release_graph();
    w->timestep = timestep;
    w->dt = timestep / (float)(w->cfg_substeps > 1 ? w->cfg_substeps : 1);
    return ZENO_SUCCESS;
}

// ---- Metadata -----------------------------------------------------------------------------
uint32_t zeno_world_num_envs(ZenoWorldHandle world) { return world ? W(world)->E : 0; }
uint32_t zeno_world_num_bodies(ZenoWorldHandle world) { return world ? W(world)->B : 0; }
uint32_t zeno_world_num_joints(ZenoWorldHandle world) { return world ? W(world)->J : 0; }
uint32_t zeno_world_num_sensors(ZenoWorldHandle world) { return world ? W(world)->model.num_sensors : 0; }
uint32_t zeno_world_obs_dim(ZenoWorldHandle world) { return world ? W(world)->model.obs_dim : 0; }
uint32_t zeno_world_action_dim(ZenoWorldHandle world) { return world ? W(world)->A : 0; }

int zeno_world_get_info(ZenoWorldHandle world, ZenoInfo* info) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!info) return ZENO_INVALID_ARGUMENT;
    World* w = W(world);
    std::memset(info, 0, sizeof *info);
    info->num_envs = w->E;
    info->num_bodies = w->B;
    info->num_joints = w->J;
    info->num_actuators = w->A;
    info->num_sensors = w->model.num_sensors;
    info->num_geoms = w->model.num_geoms;
    info->obs_dim = w->model.obs_dim;
    info->action_dim = w->A;
    info->timestep = w->timestep;
    info->memory_usage = w->state_bytes();
    info->gpu_memory_usage = w->state_bytes();
    info->metal_available = false;
    return ZENO_SUCCESS;
}

// ---- Profiling ----------------------------------------------------------------------------
int zeno_world_get_profiling(ZenoWorldHandle world, ZenoProfilingData* data) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!data) return ZENO_INVALID_ARGUMENT;
    return hip_status(W(world)->get_profiling(data), "get_profiling");
}

void zeno_world_reset_profiling(ZenoWorldHandle world) {
    if (!world) return;
    World* w = W(world);
    w->prof = ZenoProfilingData{};
    w->prof_pending = false;
}

// ---- Utility ------------------------------------------------------------------------------
const char* zeno_version(void) { return "0.1.0"; }
bool zeno_metal_available(void) { return false; }

const char* zeno_error_string(int error_code) {
    switch (error_code) {
        case 0: return "success";
        case -1: return "invalid handle";
        case -2: return "file not found";
        case -3: return "parse error";
        case -4: return "metal error";
        case -5: return "out of memory";
        case -6: return "invalid argument";
        case -7: return "not implemented";
        default: return "unknown error";
    }
}

uint64_t zeno_world_memory_usage(ZenoWorldHandle world) { return world ? W(world)->state_bytes() : 0; }
void zeno_world_compact_memory(ZenoWorldHandle world) { (void)world; }
uint32_t zeno_world_max_contacts_per_env(ZenoWorldHandle world) { return world ? W(world)->M : 0; }

// ---- Swarm ABI: not part of this build --------------------------------------------------
ZenoSwarmHandle zeno_swarm_create(ZenoWorldHandle world, const ZenoSwarmConfig* config) {
    (void)world; (void)config;
    set_error("swarm subsystem not implemented");
    return nullptr;
}
void zeno_swarm_destroy(ZenoSwarmHandle swarm) { (void)swarm; }
int zeno_swarm_step(ZenoSwarmHandle swarm, ZenoWorldHandle world, float* actions) {
    (void)swarm; (void)world; (void)actions;
    return ZENO_NOT_IMPLEMENTED;
}
int zeno_swarm_get_metrics(ZenoSwarmHandle swarm, ZenoSwarmMetrics* metrics) {
    (void)swarm; (void)metrics;
    return ZENO_NOT_IMPLEMENTED;
}
ZenoAgentState* zeno_swarm_get_agent_states(ZenoSwarmHandle swarm) { (void)swarm; return nullptr; }
int zeno_swarm_get_neighbor_counts(ZenoSwarmHandle swarm, uint32_t* out, uint32_t count) {
    (void)swarm; (void)out; (void)count;
    return ZENO_NOT_IMPLEMENTED;
}
void zeno_swarm_set_body_offset(ZenoSwarmHandle swarm, uint32_t offset) { (void)swarm; (void)offset; }
int zeno_swarm_evaluate_task(ZenoSwarmHandle swarm, void* world, uint32_t task_type, const float params[8],
                             ZenoTaskResult* result) {
    (void)swarm; (void)world; (void)task_type; (void)params; (void)result;
    return ZENO_NOT_IMPLEMENTED;
}
int zeno_swarm_apply_attack(ZenoSwarmHandle swarm, const ZenoAttackConfig* config) {
    (void)swarm; (void)config;
    return ZENO_NOT_IMPLEMENTED;
}
uint32_t* zeno_swarm_get_neighbor_index_ptr(ZenoSwarmHandle swarm) { (void)swarm; return nullptr; }
uint32_t* zeno_swarm_get_neighbor_row_ptr(ZenoSwarmHandle swarm) { (void)swarm; return nullptr; }
int zeno_swarm_start_recording(ZenoSwarmHandle swarm) { (void)swarm; return ZENO_NOT_IMPLEMENTED; }
int zeno_swarm_stop_recording(ZenoSwarmHandle swarm) { (void)swarm; return ZENO_NOT_IMPLEMENTED; }
int zeno_swarm_get_replay_stats(ZenoSwarmHandle swarm, ZenoReplayStats* stats) {
    (void)swarm; (void)stats;
    return ZENO_NOT_IMPLEMENTED;
}

// ---- Extensions (include/zeno_amd_ext.h) --------------------------------------------------
ZenoAmdModelHandle zeno_amd_model_create(const char* mjcf_path) {
    if (!mjcf_path) { set_error("null path"); return nullptr; }
    ModelBox* box = new ModelBox();
    za::ParseResult r = za::parse_mjcf_file(mjcf_path, box->scene);
    if (r.error) { set_error("Failed to parse MJCF: " + r.message); delete box; return nullptr; }
    za::build_model(box->scene, box->model);
    g_last_error.clear();
    return box;
}

ZenoAmdModelHandle zeno_amd_model_create_from_string(const char* mjcf_string) {
    if (!mjcf_string) { set_error("null MJCF string"); return nullptr; }
    ModelBox* box = new ModelBox();
    za::ParseResult r = za::parse_mjcf_string(mjcf_string, box->scene);
    if (r.error) { set_error("Failed to parse MJCF: " + r.message); delete box; return nullptr; }
    za::build_model(box->scene, box->model);
    g_last_error.clear();
    return box;
}

void zeno_amd_model_destroy(ZenoAmdModelHandle model) { delete static_cast<ModelBox*>(model); }

int zeno_amd_model_view(ZenoAmdModelHandle model, ZenoAmdModelView* out) {
    if (!model) return ZENO_INVALID_HANDLE;
    if (!out) return ZENO_INVALID_ARGUMENT;
    fill_view(static_cast<ModelBox*>(model)->model, out);
    return ZENO_SUCCESS;
}

int zeno_amd_world_model_view(ZenoWorldHandle world, ZenoAmdModelView* out) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!out) return ZENO_INVALID_ARGUMENT;
    fill_view(W(world)->model, out);
    return ZENO_SUCCESS;
}

const char* zeno_amd_last_error(void) { return g_last_error.c_str(); }

int zeno_amd_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int zeno_amd_world_get_lambda(ZenoWorldHandle world, float* out) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!out) return ZENO_INVALID_ARGUMENT;
    World* w = W(world);
    if (w->N == 0) return ZENO_SUCCESS;
    hipError_t e = hipSetDevice(w->device);
    if (e == hipSuccess) e = hipMemcpyAsync(out, w->d_lam, (size_t)w->E * w->N * 4, hipMemcpyDeviceToHost, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    return hip_status(e, "get_lambda");
}

int zeno_amd_world_get_prev_contact_counts(ZenoWorldHandle world, uint32_t* out) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!out) return ZENO_INVALID_ARGUMENT;
    World* w = W(world);
    hipError_t e = hipSetDevice(w->device);
    if (e == hipSuccess) e = hipMemcpyAsync(out, w->d_pcounts, (size_t)w->E * 4, hipMemcpyDeviceToHost, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    return hip_status(e, "get_prev_contact_counts");
}

int zeno_amd_world_set_contact_counts(ZenoWorldHandle world, const uint32_t* counts) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!counts) return ZENO_INVALID_ARGUMENT;
    return hip_status(W(world)->set_contact_counts(counts), "set_contact_counts");
}

int zeno_amd_world_step_device(ZenoWorldHandle world, const float* d_actions, uint32_t substeps) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    if (!d_actions && w->A > 0) return ZENO_INVALID_ARGUMENT;
    return hip_status(w->step(d_actions ? d_actions : w->d_actions, substeps, true), "step_device");
}

int zeno_amd_world_synchronize(ZenoWorldHandle world) {
    if (!world) return ZENO_INVALID_HANDLE;
    return hip_status(W(world)->sync(), "synchronize");
}

int zeno_amd_world_set_kernel_timing(ZenoWorldHandle world, int enable) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    hipError_t e = w->sync();
    w->timing = enable > 0 ? enable : 0;
    w->t_used = 0;
    w->t_launch = 0;
    return hip_status(e, "set_kernel_timing");
}

int zeno_amd_world_get_kernel_timing(ZenoWorldHandle world, double* total_ms, uint64_t* launches) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (!total_ms || !launches) return ZENO_INVALID_ARGUMENT;
    return hip_status(W(world)->kernel_timing(total_ms, launches), "get_kernel_timing");
}

uint32_t zeno_amd_world_joint_phases(ZenoWorldHandle world) {
    if (!world) return 0;
    return W(world)->njph;
}

int zeno_amd_world_launch_config(ZenoWorldHandle world, uint32_t* envs_per_wave, uint32_t* lds_bytes) {
    if (!world) return ZENO_INVALID_HANDLE;
    const World* w = W(world);
    if (envs_per_wave) *envs_per_wave = (uint32_t)w->epw;
    if (lds_bytes) {
        *lds_bytes = w->placement == za::PL_WORK_HBM ? 0u
                   : w->placement == za::PL_ALL_HBM ? w->lds_small.bytes
                   : w->lds.bytes * (uint32_t)(w->epw * w->waves) + (w->placement == za::PL_LDS ? w->ml.bytes : 0u);
    }
    return ZENO_SUCCESS;
}

uint32_t zeno_amd_world_waves_per_group(ZenoWorldHandle world) { return world ? (uint32_t)W(world)->waves : 0u; }
int zeno_amd_world_split_groups(ZenoWorldHandle world) { return world ? (W(world)->split ? 1 : 0) : -1; }

int zeno_amd_world_modes(ZenoWorldHandle world, int* placement, int* spatial_hash) {
    if (!world) return ZENO_INVALID_HANDLE;
    if (placement) *placement = (int)W(world)->placement;
    if (spatial_hash) *spatial_hash = W(world)->hash ? 1 : 0;
    return ZENO_SUCCESS;
}

int zeno_amd_world_set_extended_contacts(ZenoWorldHandle world, int enable) {
    if (!world) return ZENO_INVALID_HANDLE;
    W(world)->set_extended_contacts(enable != 0);
    return ZENO_SUCCESS;
}

int zeno_amd_world_capture_steps(ZenoWorldHandle world, const float* d_actions, uint64_t action_stride_bytes,
                                 uint32_t num_steps, uint32_t substeps) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    if (num_steps == 0 || (w->A > 0 && !d_actions)) return ZENO_INVALID_ARGUMENT;
    if (w->A > 0 && num_steps > 1 && action_stride_bytes < (uint64_t)w->E * w->A * sizeof(float)) return ZENO_INVALID_ARGUMENT;
    return hip_status(w->capture_steps(d_actions, action_stride_bytes, num_steps, substeps), "capture_steps");
}

int zeno_amd_world_graph_launch(ZenoWorldHandle world) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    if (!w->graph_exec) return ZENO_INVALID_ARGUMENT;
    return hip_status(w->graph_launch(), "graph_launch");
}

int zeno_amd_world_release_graph(ZenoWorldHandle world) {
    if (!world) return ZENO_INVALID_HANDLE;
    W(world)->release_graph();
    return ZENO_SUCCESS;
}

int zeno_amd_world_get_cell_ids(ZenoWorldHandle world, uint32_t* out) {
    if (!world) return ZENO_INVALID_HANDLE;
    World* w = W(world);
    if (!out || !w->hash) return ZENO_INVALID_ARGUMENT;
    hipError_t e = hipSetDevice(w->device);
    if (e == hipSuccess) e = hipMemcpyAsync(out, w->d_cell_ids, (size_t)w->E * w->model.num_geoms * 4, hipMemcpyDeviceToHost, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    return hip_status(e, "get_cell_ids");
}

int zeno_amd_detect_collisions(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n, ZenoAmdContactResult* out,
                               void* stream) {
    if (n == 0) return ZENO_SUCCESS;
    if (!a || !b || !out) return ZENO_INVALID_ARGUMENT;
    return hip_status(za::launch_detect_collisions(a, b, n, out, (hipStream_t)stream), "detect_collisions");
}

int zeno_amd_detect_collisions_host(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n,
                                    ZenoAmdContactResult* out) {
    if (n == 0) return ZENO_SUCCESS;
    if (!a || !b || !out) return ZENO_INVALID_ARGUMENT;
    const size_t in_bytes = (size_t)n * sizeof(ZenoAmdCollider), out_bytes = (size_t)n * sizeof(ZenoAmdContactResult);
    void *da = nullptr, *db = nullptr, *dout = nullptr;
    hipError_t e = hipMalloc(&da, in_bytes);
    if (e == hipSuccess) e = hipMalloc(&db, in_bytes);
    if (e == hipSuccess) e = hipMalloc(&dout, out_bytes);
    if (e == hipSuccess) e = hipMemcpy(da, a, in_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db, b, in_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = za::launch_detect_collisions((const ZenoAmdCollider*)da, (const ZenoAmdCollider*)db, n,
                                                          (ZenoAmdContactResult*)dout, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, dout, out_bytes, hipMemcpyDeviceToHost);
    if (da) hipFree(da);
    if (db) hipFree(db);
    if (dout) hipFree(dout);
    return hip_status(e, "detect_collisions_host");
}

int zeno_amd_detect_collisions_host_noalloc(const ZenoAmdCollider* a, const ZenoAmdCollider* b, uint32_t n,
                                            ZenoAmdContactResult* out) {
    if (n == 0) return ZENO_SUCCESS;
    if (!a || !b || !out) return ZENO_INVALID_ARGUMENT;
    if (n > ZENO_AMD_NOALLOC_MAX_PAIRS) {
        set_error("detect_collisions_host_noalloc: " + std::to_string(n) + " pairs exceed its static staging array of " +
                  std::to_string(ZENO_AMD_NOALLOC_MAX_PAIRS) + " pairs (zeno_amd_detect_collisions_host takes any n)");
        return ZENO_INVALID_ARGUMENT;
    }
    return hip_status(za::detect_collisions_host_noalloc(a, b, n, out), "detect_collisions_host_noalloc");
}

int zeno_amd_selfcheck_divide(const float* a, const float* b, float* q, uint32_t n) {
    if (n == 0) return ZENO_SUCCESS;
    if (!a || !b || !q) return ZENO_INVALID_ARGUMENT;
    return hip_status(za::selfcheck_divide_host(a, b, q, n), "selfcheck_divide");
}

int zeno_amd_selfcheck_sqrt(const float* x, float* y, uint32_t n) {
    if (n == 0) return ZENO_SUCCESS;
    if (!x || !y) return ZENO_INVALID_ARGUMENT;
    return hip_status(za::selfcheck_sqrt_host(x, y, n), "selfcheck_sqrt");
}

int zeno_amd_selfcheck_reciprocal_error(double* max_err) {
    if (!max_err) return ZENO_INVALID_ARGUMENT;
    return hip_status(za::selfcheck_rcp_error_host(max_err), "selfcheck_reciprocal_error");
}

}  // extern "C"
