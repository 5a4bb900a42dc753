// World: one batched simulation on one GPU (the MI355X counterpart of src/world/world.zig).
#pragma once
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../include/zeno.h"
#include "model.h"
#include "step.h"

namespace za {

// Host mirror ids: one pinned host buffer each. A mirror whose pointer a getter has handed
// out ("exposed") is brought up to date before every call that changes device state returns,
// so a view the caller holds follows the simulation like the reference's shared-memory
// buffers; the others are refreshed when their getter is next called.
enum MirrorId {
    MIR_POS, MIR_QUAT, MIR_VEL, MIR_ANGVEL, MIR_ACC, MIR_JPOS, MIR_JVEL, MIR_JTRQ, MIR_OBS,
    MIR_CON, MIR_COUNT, MIR_COUNT_ALL
};

struct World {
    Model model;
    uint32_t E = 0, B = 0, J = 0, Jp = 1, A = 0, Ap = 1, obsp = 1, N = 0, M = 0;
    uint32_t nrec = 0, njph = 0;  // joint solve records and phases
    uint32_t iters = 4, cfg_substeps = 1, adaptive_substeps = 1;
    uint64_t seed = 42;
    bool profiling = false;
    float timestep = 0.002f;  // WorldConfig.timestep (full step)
    float dt = 0.002f;        // SimParams.dt of the last step
    float gravity[3] = {0, 0, -9.81f};
    int device = 0;
    int epw = 1;
    int waves = 1;  // environment groups (waves) per workgroup (model records in LDS: one copy per workgroup)
    bool split = false;  // two waves per group: the solver and the helper (step_kernel SPLIT)
    // The launch shape chosen at creation (extended-contact mode may switch to another one),
    // whether a ZENO_AMD_* variable forced it, and the device's CU count.
    int base_epw = 1, base_waves = 1;
    bool base_split = false, shape_forced = false;
    int cus = 256;
    EnvLds lds{};
    EnvLds lds_small{};  // placement 2: the arrays kept in LDS
    bool hash = false;  // spatial-hash broad phase (more than kHashMinGeoms geoms)
    bool hrows = false;  // hash filter classes fit the model's rows (build_hash_words)
    uint32_t placement = PL_LDS;  // where the step kernel keeps model records and working sets
    bool ext_contacts = false;    // extended-contact mode (zeno_amd_world_set_extended_contacts)
    bool resort = false;          // counts set by the host: the next launch sorts unconditionally
    hipStream_t stream = nullptr;
    size_t device_bytes = 0;

    // Model on device: one blob laid out by `ml` (copied into LDS by the step kernel).
    ModelLayout ml{};
    uint4* d_model = nullptr;
    float4 *d_init_pos = nullptr, *d_init_quat = nullptr, *d_init_vel = nullptr, *d_init_angvel = nullptr;

    // State on device (reference layouts).
    float4 *d_pos = nullptr, *d_quat = nullptr, *d_vel = nullptr, *d_angvel = nullptr, *d_acc = nullptr;
    float *d_jpos = nullptr, *d_jvel = nullptr, *d_jtrq = nullptr, *d_obs = nullptr, *d_lam = nullptr;
    float* d_actions = nullptr;
    ContactRec* d_con = nullptr;
    uint32_t *d_counts = nullptr, *d_pcounts = nullptr;
    uint32_t* d_cell_ids = nullptr;       // [E*G] hash mode
    // Count-only sweep of a full list: the non-plane geoms (at most 64; none when the scene
    // is hashed or has more) and the number of listed pairs with a plane.
    uint32_t* d_sweep = nullptr;
    uint32_t sweep_n = 0, sweep_planes = 0;
    bool b0_static = false;  // body 0 is static and not kinematic (the per-body stages may skip it)
    unsigned char* d_work = nullptr;      // [E * lds.bytes] HBM working sets
    // step_subset support, allocated on first use.
    ContactRec* d_prev_con = nullptr;
    uint8_t* d_prev_detached = nullptr;
    uint8_t* d_mask = nullptr;
    float4* d_stage = nullptr;  // [E*B] staging for masked state writes

    // Host mirrors. Exposed mirrors are refreshed by device-to-host copies on view_stream,
    // which waits for the step stream through view_evt.
    void* h_mirror[MIR_COUNT_ALL] = {};
    size_t mirror_bytes[MIR_COUNT_ALL] = {};
    bool dirty[MIR_COUNT_ALL] = {};
    bool exposed[MIR_COUNT_ALL] = {};
    void* d_view[MIR_COUNT_ALL] = {};  // device addresses of the mirrors (mapped pinned memory)
    bool views_pending = false;        // the last launch stores held views; wait for the stream
    hipStream_t view_stream = nullptr;
    hipEvent_t view_evt = nullptr;
    float* h_rewards = nullptr;
    uint8_t* h_dones = nullptr;

    // Host actions: a ring of pinned, coherent host buffers that the step kernel reads in
    // place over PCIe (with the rest of its input, at the start of the launch), so a step on
    // host actions needs no separate copy. One event marks the end of every kActGroup
    // host-action steps; before the first step of a group the host waits for the event of
    // the group two back, whose steps used the slots this group refills.
    static constexpr int kStage = 8;
    static constexpr int kActGroup = kStage / 2;
    float* h_act[kStage] = {};
    const float* d_act_view[kStage] = {};  // device addresses of h_act
    hipEvent_t act_evt[2] = {};
    bool act_evt_used[2] = {};
    uint64_t act_steps = 0;  // host-action steps staged and launched
    uint8_t* h_mask_stage = nullptr;

    // Profiling and kernel timing.
    hipEvent_t prof_start = nullptr, prof_stop = nullptr;
    bool prof_pending = false;
    unsigned long long* d_phase = nullptr;  // [kPhaseCount] wall-clock ticks of workgroup 0
    double wall_clock_hz = 100e6;
    ZenoProfilingData prof{};
    int timing = 0;                    // 0 off, k > 0: event pair around every k-th launch
    uint64_t t_launch = 0;             // launches since timing was set
    std::vector<hipEvent_t> t_events;  // pairs
    size_t t_used = 0;                 // events used (2 per timed launch)

    // A captured multi-step launch sequence (zeno_amd_world_capture_steps). Its kernel
    // arguments are those of capture time, so the setters that change them release it.
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    uint32_t graph_steps = 0;
    bool capturing = false;

    ~World();
    static World* create(const Scene& scene, const ZenoConfig& cfg, std::string& err);

    hipError_t step(const float* actions, uint32_t substeps, bool actions_on_device);
    hipError_t step_subset(const float* actions, const uint8_t* mask, uint32_t substeps);
    hipError_t reset(const uint8_t* mask);
    hipError_t reset_to_state(const float* pos, const float* quat, const float* vel, const float* angvel,
                              const uint8_t* mask);
    hipError_t set_state_array(float4* dst, MirrorId mid, const float* src, const uint8_t* mask);
    // Host mirror of `id`, current with the device. expose: the pointer goes to a caller, who
    // may hold it across later steps (internal reads pass false).
    void* mirror(MirrorId id, bool expose = true);
    // Brings every exposed mirror up to date after device work; returns once the copies are
    // done. A no-op when no mirror has been handed out.
    hipError_t refresh_views();
    hipError_t set_contact_counts(const uint32_t* counts);
    hipError_t sync();
    hipError_t get_profiling(ZenoProfilingData* out);
    hipError_t kernel_timing(double* ms, uint64_t* launches);
    uint64_t state_bytes() const;
    hipError_t capture_steps(const float* d_actions, uint64_t stride_bytes, uint32_t steps, uint32_t substeps);
    hipError_t graph_launch();
    void release_graph();
    // Extended-contact mode on or off. With the model records and working sets in LDS and
    // a long contact list (M >= 64), the mode runs one environment per wave without split
    // groups, the shape whose narrow phase visits the slots grouped by geom-type pair.
    void set_extended_contacts(bool on);

   private:
    hipError_t launch(const float* d_act, uint32_t substeps, const uint8_t* d_step_mask);
    hipError_t stage_actions(const float* actions, const float** d_out);
    hipError_t mark_actions_used();
    hipError_t upload_mask(const uint8_t* mask, uint8_t** d_out);
    hipError_t ensure_subset_buffers();
    hipError_t write_state_array(float4* dst, MirrorId mid, const float* src, const uint8_t* mask);
    const void* device_src(MirrorId id) const;
    void mark_all_dirty();
};

}  // namespace za
