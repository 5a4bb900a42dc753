// World lifecycle, stepping and state access on one GPU.
//
// Mirrors World in src/world/world.zig: init (:215-691), step (:694-792), stepSubset
// (:833-929), reset (:1296-1314), setters (:1413-1478), and the reset_to_state path of
// src/main.zig:290-385. State stays in HBM; host pointers handed to callers are pinned
// mirrors. Once handed out, a mirror is refreshed before every state-changing call returns
// (the reference's buffers are shared memory that World.step has finished writing when it
// returns, world.zig:733); the others are refreshed when their getter is called.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "world.h"

#define ZA_TRY(x)                                   \
    do {                                            \
        hipError_t _e = (x);                        \
        if (_e != hipSuccess) return _e;            \
    } while (0)

namespace za {
namespace {

// reset (world.zig:1296-1310 with state.zig:390-411): restore the captured initial body
// state and zero joint positions / velocities of the selected envs.
__global__ void reset_envs_kernel(uint32_t E, uint32_t B, uint32_t J, uint32_t Jp, const uint8_t* mask,
                                  const float4* ipos, const float4* iquat, const float4* ivel, const float4* iang,
                                  float4* pos, float4* quat, float4* vel, float4* ang, float* jpos, float* jvel) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;  // E (B + J) may pass 2^32
    const uint32_t per = B + J;
    if (i >= (uint64_t)E * per) return;
    const uint32_t e = (uint32_t)(i / per), k = (uint32_t)(i % per);
    if (mask && !mask[e]) return;
    if (k < B) {
        const size_t o = (size_t)e * B + k;
        pos[o] = ipos[k];
        quat[o] = iquat[k];
        vel[o] = ivel[k];
        ang[o] = iang[k];
    } else {
        const size_t o = (size_t)e * Jp + (k - B);
        jpos[o] = 0.0f;
        jvel[o] = 0.0f;
    }
}

// Copies src into dst for the envs selected by mask (all envs when mask is null).
__global__ void masked_copy_kernel(uint32_t E, uint32_t B, const uint8_t* mask, const float4* src, float4* dst) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)E * B) return;
    if (mask && !mask[i / B]) return;
    dst[i] = src[i];
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t n, uint32_t v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void fill_u8_kernel(uint8_t* p, uint32_t n, uint8_t v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

inline uint32_t blocks_for(uint64_t n, uint32_t t) { return (uint32_t)((n + t - 1) / t); }

template <typename T>
hipError_t dalloc(World* w, T** p, size_t count) {
    size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
    hipError_t e = hipMalloc((void**)p, bytes);
    if (e == hipSuccess) w->device_bytes += bytes;
    return e;
}

template <typename T>
hipError_t upload(World* w, T** p, const T* src, size_t count) {
    ZA_TRY(dalloc(w, p, count));
    if (count) ZA_TRY(hipMemcpy(*p, src, count * sizeof(T), hipMemcpyHostToDevice));
    return hipSuccess;
}

hipError_t fill_u32(hipStream_t s, uint32_t* p, uint32_t n, uint32_t v) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

}  // namespace

World::~World() {
    if (stream) hipStreamSynchronize(stream);
    release_graph();
    void* dev[] = {d_model, d_phase, d_init_pos, d_init_quat, d_init_vel, d_init_angvel, d_pos, d_quat, d_vel, d_angvel, d_acc,
                   d_jpos, d_jvel, d_jtrq, d_obs, d_lam, d_actions, d_con, d_counts, d_pcounts, d_prev_con,
                   d_prev_detached, d_mask, d_stage, d_cell_ids, d_work, d_sweep};
    for (void* p : dev) if (p) hipFree(p);
    for (int i = 0; i < MIR_COUNT_ALL; ++i) if (h_mirror[i]) hipHostFree(h_mirror[i]);
    for (int i = 0; i < kStage; ++i) {
        if (h_act[i]) hipHostFree(h_act[i]);
    }
    for (hipEvent_t ev : act_evt) if (ev) hipEventDestroy(ev);
    if (h_mask_stage) hipHostFree(h_mask_stage);
    std::free(h_rewards);
    std::free(h_dones);
    if (view_stream) hipStreamSynchronize(view_stream);
    if (view_evt) hipEventDestroy(view_evt);
    if (view_stream) hipStreamDestroy(view_stream);
    if (prof_start) hipEventDestroy(prof_start);
    if (prof_stop) hipEventDestroy(prof_stop);
    for (hipEvent_t ev : t_events) hipEventDestroy(ev);
    if (stream) hipStreamDestroy(stream);
}

World* World::create(const Scene& scene, const ZenoConfig& cfg, std::string& err) {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        err = "no HIP device available";
        return nullptr;
    }
    World* w = new World();
    auto fail = [&](const char* what, hipError_t e) -> World* {
        err = std::string(what) + ": " + hipGetErrorString(e);
        delete w;
        return nullptr;
    };
    build_model(scene, w->model);
    const Model& m = w->model;
    w->E = cfg.num_envs;
    w->B = m.num_bodies;
    w->J = m.num_joints;
    w->Jp = std::max<uint32_t>(m.num_joints, 1);
    w->A = m.num_actuators;
    w->Ap = std::max<uint32_t>(m.num_actuators, 1);
    w->obsp = std::max<uint32_t>(m.obs_dim, 1);
    w->N = m.num_constraints;
    w->M = cfg.max_contacts_per_env;
    w->iters = cfg.contact_iterations;
    w->cfg_substeps = cfg.substeps;
    w->adaptive_substeps = cfg.substeps;
    w->seed = cfg.seed;
    w->profiling = cfg.enable_profiling;
    // main.zig:153: 0 (or negative) selects the MJCF timestep.
    w->timestep = cfg.timestep > 0 ? cfg.timestep : m.physics.timestep;
    w->dt = w->timestep / (float)std::max<uint32_t>(cfg.substeps, 1);
    std::memcpy(w->gravity, m.physics.gravity, sizeof w->gravity);
    if (w->E == 0) { err = "num_envs must be > 0"; delete w; return nullptr; }
    if (w->B > 65535 || w->M > 65535 || m.num_geoms > 65535) { err = "scene too large"; delete w; return nullptr; }

    hipError_t e = hipGetDevice(&w->device);
    if (e != hipSuccess) return fail("hipGetDevice", e);

    w->hash = m.num_geoms > kHashMinGeoms;
    if (w->hash && m.num_geoms > kHashMaxGeoms) { err = "scene too large for the spatial hash (over 16384 geoms)"; delete w; return nullptr; }
    EnvLds L = make_env_lds(w->B, w->Jp, w->N, std::max<uint32_t>(w->M, 1), m.num_geoms, 0, false, w->obsp);
    std::vector<float4> invmi(w->B), com(w->B);
    std::vector<uint32_t> flags(w->B);
    for (uint32_t b = 0; b < w->B; ++b) {
        const float* im = &m.inv_mass_inertia[4 * b];
        invmi[b] = make_float4(im[0], im[1], im[2], im[3]);
        com[b] = make_float4(m.bodies[b].com_offset[0], m.bodies[b].com_offset[1], m.bodies[b].com_offset[2], 0.0f);
        flags[b] = ((uint32_t)m.bodies[b].params[1] == 1u ? 1u : 0u) | (im[0] > 1e-8f ? 2u : 0u);
    }
    // Bit 2: the body takes part in a constraint template (a joint solve may move it).
    for (const ConstraintRec& t : m.templates) {
        if (t.indices[0] < w->B) flags[t.indices[0]] |= 4u;
        if (t.indices[1] < w->B) flags[t.indices[1]] |= 4u;
    }
    w->b0_static = w->B > 1 && invmi[0].x < 1e-8f && (flags[0] & 1u) == 0u;
    std::vector<float4> jrec;
    std::vector<JointPhase> jph;
    build_joint_program(m.templates, m.color_ranges, (const float*)invmi.data(), (const float*)com.data(), jrec, jph);
    w->nrec = (uint32_t)(jrec.size() / kJRecQuads);
    w->njph = (uint32_t)jph.size();
    const ModelLayout ML = make_model_layout(w->B, w->J, m.num_geoms, m.num_pairs, w->A, m.num_sensors, w->nrec, w->njph);
    // Placement and launch shape. The step is a chain of dependent solver phases per
    // environment, so throughput follows the number of environments a CU holds at once:
    // each candidate (model records and working sets in LDS with 1, 2, 4 or 8 environments
    // per wave and 1, 4 or 2 waves per workgroup sharing one copy of the model records;
    // model records read from HBM with one working set in LDS; both in HBM) is scored by
    // min(E, environments resident on the GPU), from the HIP occupancy query (LDS and
    // registers). Ties keep the earlier candidate: LDS before HBM, four waves per workgroup
    // before one (one copy of the model records per four waves: less LDS and fewer L2 reads;
    // Ant 4096 79.6 against 80.0 us per step), and among the LDS shapes first the largest
    // environments-per-wave with at least 1024 workgroups and 64 KB of LDS, then the others
    // from 1 up.
    // Each LDS shape also comes split, and ties prefer it: two waves per environment group,
    // the second running the contact pipeline (broad phase to contact levels) while the first
    // solves the joints; same LDS, twice the waves (Ant 4096 74.4 -> 66.2 us per step,
    // Humanoid 16384 266 -> 232 us).
    // ZENO_AMD_PLACEMENT=0/1/2/3, ZENO_AMD_ENVS_PER_WAVE, ZENO_AMD_WAVES and ZENO_AMD_SPLIT=0/1
    // force a placement or a shape (tests of each path; a forced shape implies placement 0).
    const size_t lds_max = max_lds_per_workgroup(w->device);
    int cus = 256;
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, w->device);
    w->cus = cus;
    // Placement 2 keeps the body slot masks in LDS when they fit, else in the HBM working set.
    EnvLds L_small = make_env_lds_small(w->B, w->Jp, std::max<uint32_t>(w->M, 1), m.num_geoms, !w->hash, true);
    if ((size_t)L_small.bytes > lds_max)
        L_small = make_env_lds_small(w->B, w->Jp, std::max<uint32_t>(w->M, 1), m.num_geoms, !w->hash, false);
    const EnvLds L_own = make_env_lds(w->B, w->Jp, w->N, std::max<uint32_t>(w->M, 1), m.num_geoms, 16 * kJRecQuads * w->nrec,
                                      !w->hash, w->obsp);
    // Placement 3: the whole working set in HBM, the hash's staged geoms included.
    const EnvLds L_work = make_env_lds(w->B, w->Jp, w->N, std::max<uint32_t>(w->M, 1), m.num_geoms,
                                       16 * kJRecQuads * w->nrec, !w->hash, w->obsp, true);
    struct Cand { uint32_t pl; int epw; int waves; size_t shmem; bool split; };
    std::vector<Cand> cands;
    int force_pl = -1, force_epw = 0, force_waves = 0, force_split = -1;
    if (const char* env = std::getenv("ZENO_AMD_PLACEMENT")) force_pl = std::min(std::max(std::atoi(env), 0), 3);
    if (const char* env = std::getenv("ZENO_AMD_ENVS_PER_WAVE")) force_epw = std::atoi(env);
    if (const char* env = std::getenv("ZENO_AMD_WAVES")) force_waves = std::atoi(env);
    if (const char* env = std::getenv("ZENO_AMD_SPLIT")) force_split = std::atoi(env) != 0 ? 1 : 0;
    if ((force_epw > 0 || force_waves > 1 || force_split == 1) && force_pl < 0) force_pl = PL_LDS;
    {
        std::vector<int> order;
        for (int cand : {8, 4, 2}) {
            if (w->hash) continue;
            if ((size_t)ML.bytes + (size_t)L.bytes * cand > 64 * 1024) continue;
            if ((w->E + cand - 1) / cand < 1024) continue;
            order.push_back(cand);
            break;
        }
        for (int cand : {1, 2, 4, 8}) {
            if (cand > 1 && w->hash) continue;
            if (std::find(order.begin(), order.end(), cand) == order.end()) order.push_back(cand);
        }
        for (bool split : {true, false}) {
            if (split && w->hash) continue;
            for (int waves : {4, 1, 2}) {
                if (waves > 1 && w->hash) continue;
                for (int cand : order) {
                    const size_t shmem = (size_t)ML.bytes + (size_t)L.bytes * cand * waves;
                    if (shmem <= lds_max) cands.push_back({PL_LDS, cand, waves, shmem, split});
                }
            }
        }
        if ((size_t)L_own.bytes <= lds_max) cands.push_back({PL_MODEL_HBM, 1, 1, (size_t)L_own.bytes, false});
        cands.push_back({PL_ALL_HBM, 1, 1, (size_t)L_small.bytes, false});
    }
    // Placement 3 (no LDS at all) is the fallback for contact lists that no LDS layout
    // holds: it scores well on residency, but its contact pipeline runs out of the caches.
    const std::vector<Cand> fallback{{PL_WORK_HBM, 1, 1, 0, false}};
    const Cand* best = nullptr;
    uint64_t best_score = 0;
    for (int pass = 0; pass < 2 && !best; ++pass) {
      const std::vector<Cand>& list = pass == 0 ? cands : fallback;
      for (const Cand& c : list) {
        if (force_pl >= 0 && (int)c.pl != force_pl) continue;
        if (force_epw > 0 && c.epw != force_epw) continue;
        if (force_waves > 0 && c.waves != force_waves) continue;
        if (force_split >= 0 && c.split != (force_split == 1)) continue;
        const int n = resident_workgroups(c.epw, c.pl, w->hash, c.shmem, c.waves, c.split);
        if (n <= 0) continue;
        const uint64_t score = std::min<uint64_t>(w->E, (uint64_t)n * (uint64_t)c.epw * (uint64_t)c.waves * (uint64_t)cus);
        if (!best || score > best_score) { best = &c; best_score = score; }
      }
    }
    if (!best) {
        err = "no launch shape fits this scene (ZENO_AMD_PLACEMENT / ZENO_AMD_ENVS_PER_WAVE / ZENO_AMD_WAVES / "
              "ZENO_AMD_SPLIT force a shape that cannot launch, or the step kernel cannot run on this device)";
        delete w;
        return nullptr;
    }
    w->placement = best->pl;
    const int epw = best->epw;
    if (best->pl == PL_MODEL_HBM || best->pl == PL_ALL_HBM) L = L_own;
    if (best->pl == PL_WORK_HBM) L = L_work;
    w->lds = L;
    w->lds_small = L_small;
    w->epw = epw;
    w->waves = best->waves;
    w->split = best->split;
    w->base_epw = w->epw;
    w->base_waves = w->waves;
    w->base_split = w->split;
    w->shape_forced = force_pl >= 0 || force_epw > 0 || force_waves > 0 || force_split >= 0;

    if ((e = hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking)) != hipSuccess) return fail("hipStreamCreate", e);
    if ((e = hipStreamCreateWithFlags(&w->view_stream, hipStreamNonBlocking)) != hipSuccess) return fail("hipStreamCreate", e);
    if ((e = hipEventCreateWithFlags(&w->view_evt, hipEventDisableTiming)) != hipSuccess) return fail("hipEventCreate", e);

    // Model blob: every per-scene record the kernel reads, packed per ModelLayout.
    w->ml = ML;
    {
        std::vector<unsigned char> blob(w->ml.bytes, 0);
        auto put = [&](uint32_t off, const void* src, size_t bytes) { if (bytes) std::memcpy(blob.data() + off, src, bytes); };
        put(w->ml.invmi, invmi.data(), 16 * w->B);
        put(w->ml.com, com.data(), 16 * w->B);
        put(w->ml.flags, flags.data(), 4 * w->B);
        put(w->ml.joints, m.joints.data(), sizeof(JointRec) * m.joints.size());
        put(w->ml.geoms, m.geoms.data(), sizeof(GeomRec) * m.geoms.size());
        put(w->ml.pairs, m.pairs.data(), 4 * m.pairs.size());
        put(w->ml.acts, m.actuators.data(), sizeof(ActuatorRec) * m.actuators.size());
        put(w->ml.sensors, m.sensors.data(), sizeof(SensorRec) * m.sensors.size());
        put(w->ml.jrec, jrec.data(), sizeof(float4) * jrec.size());
        put(w->ml.jphase, jph.data(), sizeof(JointPhase) * jph.size());
        std::vector<uint32_t> bjoff, bjl;
        build_body_joint_lists(m.joints, w->B, bjoff, bjl);
        put(w->ml.bjoff, bjoff.data(), 4 * bjoff.size());
        put(w->ml.bjl, bjl.data(), 4 * bjl.size());
        if (w->hash) {
            std::vector<uint32_t> hmeta, hrow;
            w->hrows = build_hash_words(m.geoms, hmeta, hrow);
            put(w->ml.hmeta, hmeta.data(), 4 * hmeta.size());
            put(w->ml.hrow, hrow.data(), 4 * hrow.size());
        }
        if ((e = upload(w, &w->d_model, (const uint4*)blob.data(), w->ml.bytes / 16)) != hipSuccess) return fail("upload", e);
    }
    if (!w->hash && !m.pairs.empty()) {
        std::vector<uint32_t> sweep;
        for (uint32_t g = 0; g < m.num_geoms; ++g) if (m.geoms[g].type_body[0] != GEOM_PLANE) sweep.push_back(g);
        if (!sweep.empty() && sweep.size() <= 64) {
            for (uint32_t pr : m.pairs) {
                if (m.geoms[pr & 0xFFFFu].type_body[0] == GEOM_PLANE || m.geoms[pr >> 16].type_body[0] == GEOM_PLANE) ++w->sweep_planes;
            }
            w->sweep_n = (uint32_t)sweep.size();
            if ((e = upload(w, &w->d_sweep, sweep.data(), sweep.size())) != hipSuccess) return fail("upload", e);
        }
    }
    std::vector<float4> ip(w->B), iq(w->B), iv(w->B), ia(w->B);
    for (uint32_t b = 0; b < w->B; ++b) {
        ip[b] = make_float4(m.init_pos[4 * b], m.init_pos[4 * b + 1], m.init_pos[4 * b + 2], m.init_pos[4 * b + 3]);
        iq[b] = make_float4(m.init_quat[4 * b], m.init_quat[4 * b + 1], m.init_quat[4 * b + 2], m.init_quat[4 * b + 3]);
        iv[b] = make_float4(m.init_vel[4 * b], m.init_vel[4 * b + 1], m.init_vel[4 * b + 2], m.init_vel[4 * b + 3]);
        ia[b] = make_float4(m.init_angvel[4 * b], m.init_angvel[4 * b + 1], m.init_angvel[4 * b + 2], m.init_angvel[4 * b + 3]);
    }
    if ((e = upload(w, &w->d_init_pos, ip.data(), w->B)) != hipSuccess) return fail("upload", e);
    if ((e = upload(w, &w->d_init_quat, iq.data(), w->B)) != hipSuccess) return fail("upload", e);
    if ((e = upload(w, &w->d_init_vel, iv.data(), w->B)) != hipSuccess) return fail("upload", e);
    if ((e = upload(w, &w->d_init_angvel, ia.data(), w->B)) != hipSuccess) return fail("upload", e);
    if (w->profiling) {
        if ((e = dalloc(w, &w->d_phase, kPhaseCount)) != hipSuccess) return fail("hipMalloc", e);
        int khz = 0;
        if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, w->device) == hipSuccess && khz > 0)
            w->wall_clock_hz = 1e3 * (double)khz;
    }

    // State (state.zig:56-117 sizes; zero-filled like fresh Metal buffers).
    const size_t EB = (size_t)w->E * w->B;
    float4** f4s[] = {&w->d_pos, &w->d_quat, &w->d_vel, &w->d_angvel, &w->d_acc};
    for (float4** p : f4s) if ((e = dalloc(w, p, EB)) != hipSuccess) return fail("hipMalloc", e);
    float** fjs[] = {&w->d_jpos, &w->d_jvel, &w->d_jtrq};
    for (float** p : fjs) if ((e = dalloc(w, p, (size_t)w->E * w->Jp)) != hipSuccess) return fail("hipMalloc", e);
    if ((e = dalloc(w, &w->d_obs, (size_t)w->E * w->obsp)) != hipSuccess) return fail("hipMalloc", e);
    if ((e = dalloc(w, &w->d_lam, (size_t)w->E * std::max<uint32_t>(w->N, 1))) != hipSuccess) return fail("hipMalloc", e);
    if ((e = dalloc(w, &w->d_actions, (size_t)w->E * w->Ap)) != hipSuccess) return fail("hipMalloc", e);
    if ((e = dalloc(w, &w->d_con, (size_t)w->E * std::max<uint32_t>(w->M, 1))) != hipSuccess) return fail("hipMalloc", e);
    if ((e = dalloc(w, &w->d_counts, w->E)) != hipSuccess) return fail("hipMalloc", e);
    if ((e = dalloc(w, &w->d_pcounts, w->E)) != hipSuccess) return fail("hipMalloc", e);
    if (w->hash && (e = dalloc(w, &w->d_cell_ids, (size_t)w->E * m.num_geoms)) != hipSuccess) return fail("hipMalloc", e);
    if (w->placement >= PL_ALL_HBM && (e = dalloc(w, &w->d_work, (size_t)w->E * w->lds.bytes)) != hipSuccess) return fail("hipMalloc", e);
    struct Z { void* p; size_t n; } zeros[] = {
        {w->d_pos, EB * 16}, {w->d_quat, EB * 16}, {w->d_vel, EB * 16}, {w->d_angvel, EB * 16}, {w->d_acc, EB * 16},
        {w->d_jpos, (size_t)w->E * w->Jp * 4}, {w->d_jvel, (size_t)w->E * w->Jp * 4}, {w->d_jtrq, (size_t)w->E * w->Jp * 4},
        {w->d_obs, (size_t)w->E * w->obsp * 4}, {w->d_lam, (size_t)w->E * std::max<uint32_t>(w->N, 1) * 4},
        {w->d_actions, (size_t)w->E * w->Ap * 4}, {w->d_con, (size_t)w->E * std::max<uint32_t>(w->M, 1) * 64},
        {w->d_counts, (size_t)w->E * 4}, {w->d_pcounts, (size_t)w->E * 4},
        {w->d_cell_ids, w->d_cell_ids ? (size_t)w->E * m.num_geoms * 4 : 0}};
    for (const Z& z : zeros) if (z.n && (e = hipMemsetAsync(z.p, 0, z.n, w->stream)) != hipSuccess) return fail("hipMemset", e);
    // initializeState (world.zig:663-691): every env starts from the scene pose.
    hipLaunchKernelGGL(reset_envs_kernel, dim3(blocks_for((uint64_t)w->E * (w->B + w->J), 256)), dim3(256), 0, w->stream,
                       w->E, w->B, w->J, w->Jp, (const uint8_t*)nullptr, w->d_init_pos, w->d_init_quat, w->d_init_vel,
                       w->d_init_angvel, w->d_pos, w->d_quat, w->d_vel, w->d_angvel, w->d_jpos, w->d_jvel);
    if ((e = hipGetLastError()) != hipSuccess) return fail("init kernel", e);

    // Host mirrors: pinned, mapped and coherent, so that the step kernel can store the
    // arrays a caller holds straight into them (StepArgs::hv).
    const size_t mb[MIR_COUNT_ALL] = {EB * 16, EB * 16, EB * 16, EB * 16, EB * 16,
                                      (size_t)w->E * w->Jp * 4, (size_t)w->E * w->Jp * 4, (size_t)w->E * w->Jp * 4,
                                      (size_t)w->E * w->obsp * 4, (size_t)w->E * std::max<uint32_t>(w->M, 1) * 64,
                                      (size_t)w->E * 4};
    for (int i = 0; i < MIR_COUNT_ALL; ++i) {
        w->mirror_bytes[i] = mb[i];
        if ((e = hipHostMalloc(&w->h_mirror[i], mb[i], hipHostMallocMapped | hipHostMallocCoherent)) != hipSuccess)
            return fail("hipHostMalloc", e);
        if ((e = hipHostGetDevicePointer(&w->d_view[i], w->h_mirror[i], 0)) != hipSuccess) return fail("hipHostGetDevicePointer", e);
        w->dirty[i] = true;
    }
    w->h_rewards = (float*)std::calloc(w->E, sizeof(float));
    w->h_dones = (uint8_t*)std::calloc(w->E, 1);
    for (int i = 0; i < kStage; ++i) {
        // Coherent (fine-grained) so that the kernel reads what the host wrote before the launch
        // and no stale cached copy of a reused slot.
        if ((e = hipHostMalloc((void**)&w->h_act[i], (size_t)w->E * w->Ap * 4, hipHostMallocMapped | hipHostMallocCoherent)) != hipSuccess)
            return fail("hipHostMalloc", e);
        void* dv = nullptr;
        if ((e = hipHostGetDevicePointer(&dv, w->h_act[i], 0)) != hipSuccess) return fail("hipHostGetDevicePointer", e);
        w->d_act_view[i] = (const float*)dv;
    }
    for (hipEvent_t& ev : w->act_evt)
        if ((e = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess) return fail("hipEventCreate", e);
    if ((e = hipHostMalloc((void**)&w->h_mask_stage, w->E, hipHostMallocDefault)) != hipSuccess) return fail("hipHostMalloc", e);
    if ((e = hipStreamSynchronize(w->stream)) != hipSuccess) return fail("init", e);
    return w;
}

void World::mark_all_dirty() {
    for (int i = 0; i < MIR_COUNT_ALL; ++i) dirty[i] = true;
}

hipError_t World::sync() { return hipStreamSynchronize(stream); }

uint64_t World::state_bytes() const { return device_bytes; }

hipError_t World::launch(const float* d_act, uint32_t substeps, const uint8_t* d_step_mask) {
    StepArgs a{};
    a.E = E; a.B = B; a.J = J; a.Jp = Jp; a.A = A; a.S = model.num_sensors; a.obsp = obsp; a.N = N;
    a.nrec = nrec; a.njph = njph; a.M = M; a.P = model.num_pairs;
    a.G = model.num_geoms; a.Gp = hash ? hash_pad(model.num_geoms) : 0; a.hash = hash ? 1u : 0u;
    a.hrows = hrows ? 1u : 0u;
    a.cell_ids = d_cell_ids;
    a.ext_contacts = ext_contacts ? 1u : 0u;
    a.sort_all = resort ? 1u : 0u;
    a.sweep = d_sweep; a.sweep_n = sweep_n; a.sweep_planes = sweep_planes;
    // Only where it saves a pass: the bodies after body 0 fill whole passes of the lanes.
    a.b_first = (b0_static && (B - 1u) % (64u / (uint32_t)epw) == 0u) ? 1u : 0u;
    resort = false;
    a.placement = placement;
    a.work = d_work;
    a.iters = iters; a.substeps = substeps;
    a.dt = dt;
    a.inv_step = timestep > 0 ? 1.0f / timestep : 0.0f;
    a.gx = gravity[0]; a.gy = gravity[1]; a.gz = gravity[2];
    a.restitution = model.physics.restitution;
    a.baumgarte = model.physics.baumgarte;
    a.slop = model.physics.slop;
    a.model = d_model;
    a.ml = ml;
    a.phase_ticks = profiling ? d_phase : nullptr;
    a.pos = d_pos; a.quat = d_quat; a.vel = d_vel; a.angvel = d_angvel; a.acc = d_acc;
    a.jpos = d_jpos; a.jvel = d_jvel; a.jtrq = d_jtrq; a.obs = d_obs; a.lam = d_lam; a.actions = d_act;
    a.contacts = d_con; a.counts = d_counts; a.pcounts = d_pcounts;
    a.prev_detached = d_prev_detached;
    a.prev_contacts = d_prev_con;
    a.step_mask = d_step_mask;
    a.prev_out = d_prev_con;
    a.prev_detached_out = d_prev_detached;
    a.lds = lds;
    a.lds_small = lds_small;
    // Held views are stored by the kernel itself in eager launches; a captured launch keeps
    // the views of capture time, so graph_launch refreshes them by copies instead.
    const bool direct = !capturing;
    auto view = [&](MirrorId id) { return direct && exposed[id] ? d_view[id] : nullptr; };
    a.hv.pos = (float4*)view(MIR_POS);
    a.hv.quat = (float4*)view(MIR_QUAT);
    a.hv.vel = (float4*)view(MIR_VEL);
    a.hv.angvel = (float4*)view(MIR_ANGVEL);
    a.hv.acc = (float4*)view(MIR_ACC);
    a.hv.jpos = (float*)view(MIR_JPOS);
    a.hv.jvel = (float*)view(MIR_JVEL);
    a.hv.jtrq = (float*)view(MIR_JTRQ);
    a.hv.obs = (float*)view(MIR_OBS);
    a.hv.contacts = (ContactRec*)view(MIR_CON);
    a.hv.counts = (uint32_t*)view(MIR_COUNT);
    hipEvent_t t0 = nullptr, t1 = nullptr;
    // Under capture the launch becomes a graph node; event timing and profiling stay eager-only.
    const bool timed = !capturing && timing > 0 && (t_launch++ % (uint64_t)timing) == 0;
    const bool prof_events = profiling && !capturing;
    if (timed) {
        while (t_events.size() < t_used + 2) {
            // Timing only: no system-scope fence (cache write-back) when the event completes,
            // which would add its own cost to the interval measured.
            hipEvent_t ev;
            ZA_TRY(hipEventCreateWithFlags(&ev, hipEventDisableSystemFence));
            t_events.push_back(ev);
        }
        t0 = t_events[t_used];
        t1 = t_events[t_used + 1];
        t_used += 2;
        ZA_TRY(hipEventRecord(t0, stream));
    }
    if (prof_events) {
        if (!prof_start) { ZA_TRY(hipEventCreate(&prof_start)); ZA_TRY(hipEventCreate(&prof_stop)); }
        ZA_TRY(hipEventRecord(prof_start, stream));
    }
    ZA_TRY(launch_step(a, epw, waves, stream, split));
    if (prof_events) { ZA_TRY(hipEventRecord(prof_stop, stream)); prof_pending = true; }
    if (timed) ZA_TRY(hipEventRecord(t1, stream));
    mark_all_dirty();
    // The held views were current before this launch (every state-changing call leaves them
    // so) and the kernel stores what it changes in them: they are current once the stream
    // reaches this point.
    for (int i = 0; i < MIR_COUNT_ALL; ++i) {
        if (direct && exposed[i]) { dirty[i] = false; views_pending = true; }
    }
    return hipSuccess;
}

// World.step, world.zig:694-746: substeps 0 selects the configured count; dt = timestep /
// substeps; accelerations come from the velocity change over the whole call.
hipError_t World::stage_actions(const float* actions, const float** d_out) {
    const uint64_t k = act_steps;
    const int slot = (int)(k % kStage);
    const int ev = (int)((k / kActGroup) % 2);
    // The steps that last read this group's slots (the group two back) must be done before
    // the host refills them.
    if (k % kActGroup == 0 && act_evt_used[ev]) ZA_TRY(hipEventSynchronize(act_evt[ev]));
    std::memcpy(h_act[slot], actions, (size_t)E * A * sizeof(float));
    *d_out = d_act_view[slot];
    return hipSuccess;
}

hipError_t World::mark_actions_used() {
    const uint64_t k = act_steps++;
    if (k % kActGroup == kActGroup - 1) {
        const int ev = (int)((k / kActGroup) % 2);
        ZA_TRY(hipEventRecord(act_evt[ev], stream));
        act_evt_used[ev] = true;
    }
    return hipSuccess;
}

hipError_t World::step(const float* actions, uint32_t substeps, bool actions_on_device) {
    ZA_TRY(hipSetDevice(device));
    const uint32_t actual = substeps == 0 ? adaptive_substeps : substeps;
    dt = timestep / (float)std::max<uint32_t>(actual, 1);
    const float* d_act = d_actions;
    bool staged = false;
    if (actions_on_device) d_act = actions;
    else if (A > 0) { ZA_TRY(stage_actions(actions, &d_act)); staged = true; }
    ZA_TRY(launch(d_act, actual, nullptr));
    if (staged) ZA_TRY(mark_actions_used());
    return refresh_views();
}

void World::set_extended_contacts(bool on) {
    release_graph();
    ext_contacts = on;
    if (shape_forced || placement != PL_LDS || hash) return;
    epw = base_epw;
    waves = base_waves;
    split = base_split;
    if (!on || M < 64) return;
    // The grouped narrow phase runs in the one-environment-per-wave instances without split
    // groups: the best of those by resident environments (the creation-time score).
    uint64_t best = 0;
    for (int w : {4, 1, 2}) {
        const size_t shmem = (size_t)ml.bytes + (size_t)lds.bytes * (size_t)w;
        const int n = resident_workgroups(1, PL_LDS, false, shmem, w, false);
        if (n <= 0) continue;
        const uint64_t score = std::min<uint64_t>(E, (uint64_t)n * (uint64_t)w * (uint64_t)cus);
        if (score > best) {
            best = score;
            epw = 1;
            waves = w;
            split = false;
        }
    }
}

void World::release_graph() {
    // A replay may still be running: the executable graph is destroyed once it is done.
    if (graph_exec) hipStreamSynchronize(stream);
    if (graph_exec) hipGraphExecDestroy(graph_exec);
    if (graph) hipGraphDestroy(graph);
    graph_exec = nullptr;
    graph = nullptr;
    graph_steps = 0;
}

// `steps` consecutive steps, step k reading its actions at d_actions + k * stride_bytes,
// captured from the world's stream into one HIP graph: a replay is one launch call for the
// whole sequence instead of one per step. Every node is a step-kernel launch (no memset or
// copy nodes). Substeps, dt, gravity, the contact mode and the buffer addresses are fixed at
// capture; the world's setters for them release the graph.
hipError_t World::capture_steps(const float* d_act, uint64_t stride_bytes, uint32_t steps, uint32_t substeps) {
    ZA_TRY(hipSetDevice(device));
    release_graph();
    ZA_TRY(hipStreamSynchronize(stream));
    const uint32_t actual = substeps == 0 ? adaptive_substeps : substeps;
    dt = timestep / (float)std::max<uint32_t>(actual, 1);
    ZA_TRY(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    capturing = true;
    hipError_t e = hipSuccess;
    for (uint32_t k = 0; k < steps && e == hipSuccess; ++k) {
        const float* a = A > 0 ? reinterpret_cast<const float*>(reinterpret_cast<const char*>(d_act) + k * stride_bytes)
                               : d_actions;
        e = launch(a, actual, nullptr);
    }
    capturing = false;
    hipGraph_t g = nullptr;
    const hipError_t ec = hipStreamEndCapture(stream, &g);
    if (e == hipSuccess) e = ec;
    if (e == hipSuccess) e = hipGraphInstantiate(&graph_exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (g) hipGraphDestroy(g);
        graph_exec = nullptr;
        (void)hipGetLastError();
        return e;
    }
    graph = g;
    graph_steps = steps;
    return hipSuccess;
}

hipError_t World::graph_launch() {
    if (!graph_exec) return hipErrorInvalidValue;
    ZA_TRY(hipSetDevice(device));
    ZA_TRY(hipGraphLaunch(graph_exec, stream));
    mark_all_dirty();
    return refresh_views();
}

hipError_t World::ensure_subset_buffers() {
    if (!d_prev_con) {
        release_graph();  // captured launches hold the buffer addresses of capture time
        ZA_TRY(dalloc(this, &d_prev_con, (size_t)E * std::max<uint32_t>(M, 1)));
        ZA_TRY(dalloc(this, &d_prev_detached, E));
        hipLaunchKernelGGL(fill_u8_kernel, dim3(blocks_for(E, 256)), dim3(256), 0, stream, d_prev_detached, E, (uint8_t)0);
        ZA_TRY(hipGetLastError());
    }
    return hipSuccess;
}

hipError_t World::upload_mask(const uint8_t* mask, uint8_t** d_out) {
    if (!mask) { *d_out = nullptr; return hipSuccess; }
    if (!d_mask) ZA_TRY(dalloc(this, &d_mask, E));
    ZA_TRY(hipStreamSynchronize(stream));  // h_mask_stage may still feed an earlier copy
    std::memcpy(h_mask_stage, mask, E);
    ZA_TRY(hipMemcpyAsync(d_mask, h_mask_stage, E, hipMemcpyHostToDevice, stream));
    *d_out = d_mask;
    return hipSuccess;
}

// World.stepSubset, world.zig:833-929: the selected envs advance; the others keep every
// visible buffer while their solver history (lambda, previous contacts) advances.
hipError_t World::step_subset(const float* actions, const uint8_t* mask, uint32_t substeps) {
    ZA_TRY(hipSetDevice(device));
    uint32_t active = 0;
    for (uint32_t e = 0; e < E; ++e) active += mask[e] ? 1u : 0u;
    if (active == 0) return hipSuccess;
    if (active == E) return step(actions, substeps, false);
    ZA_TRY(ensure_subset_buffers());
    const uint32_t actual = substeps == 0 ? adaptive_substeps : substeps;
    dt = timestep / (float)std::max<uint32_t>(actual, 1);
    const float* d_act = d_actions;
    bool staged = false;
    if (A > 0) { ZA_TRY(stage_actions(actions, &d_act)); staged = true; }
    uint8_t* dm = nullptr;
    ZA_TRY(upload_mask(mask, &dm));
    ZA_TRY(launch(d_act, actual, dm));
    if (staged) ZA_TRY(mark_actions_used());
    return refresh_views();
}

// World.reset, world.zig:1296-1314: restore the selected envs, then zero every env's
// contact count (the reference clears all counts whatever the mask).
hipError_t World::reset(const uint8_t* mask) {
    ZA_TRY(hipSetDevice(device));
    uint8_t* dm = nullptr;
    ZA_TRY(upload_mask(mask, &dm));
    hipLaunchKernelGGL(reset_envs_kernel, dim3(blocks_for((uint64_t)E * (B + J), 256)), dim3(256), 0, stream,
                       E, B, J, Jp, (const uint8_t*)dm, d_init_pos, d_init_quat, d_init_vel, d_init_angvel,
                       d_pos, d_quat, d_vel, d_angvel, d_jpos, d_jvel);
    ZA_TRY(hipGetLastError());
    ZA_TRY(fill_u32(stream, d_counts, E, 0));
    mark_all_dirty();
    return refresh_views();
}

// A caller's write through the contact-count pointer the reference hands out (shared memory
// there, main.zig:557-560): the counts become the device's, and the held views follow.
hipError_t World::set_contact_counts(const uint32_t* counts) {
    ZA_TRY(hipSetDevice(device));
    ZA_TRY(hipMemcpyAsync(d_counts, counts, (size_t)E * 4, hipMemcpyHostToDevice, stream));
    ZA_TRY(hipStreamSynchronize(stream));
    resort = true;  // the next step sorts every env's first min(count, M) slots
    mark_all_dirty();
    return refresh_views();
}

hipError_t World::set_state_array(float4* dst, MirrorId mid, const float* src, const uint8_t* mask) {
    ZA_TRY(write_state_array(dst, mid, src, mask));
    return refresh_views();
}

hipError_t World::write_state_array(float4* dst, MirrorId mid, const float* src, const uint8_t* mask) {
    const size_t bytes = (size_t)E * B * 16;
    if (!mask) {
        ZA_TRY(hipStreamSynchronize(stream));
        ZA_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream));
    } else {
        if (!d_stage) ZA_TRY(dalloc(this, &d_stage, (size_t)E * B));
        uint8_t* dm = nullptr;
        ZA_TRY(upload_mask(mask, &dm));
        ZA_TRY(hipMemcpyAsync(d_stage, src, bytes, hipMemcpyHostToDevice, stream));
        hipLaunchKernelGGL(masked_copy_kernel, dim3(blocks_for((uint64_t)E * B, 256)), dim3(256), 0, stream, E, B,
                           (const uint8_t*)dm, (const float4*)d_stage, dst);
        ZA_TRY(hipGetLastError());
    }
    // The caller's buffer is only borrowed for this call.
    ZA_TRY(hipStreamSynchronize(stream));
    dirty[mid] = true;
    return hipSuccess;
}

// main.zig:290-385
hipError_t World::reset_to_state(const float* pos, const float* quat, const float* vel, const float* angvel,
                                 const uint8_t* mask) {
    ZA_TRY(hipSetDevice(device));
    ZA_TRY(write_state_array(d_pos, MIR_POS, pos, mask));
    ZA_TRY(write_state_array(d_quat, MIR_QUAT, quat, mask));
    if (vel) ZA_TRY(write_state_array(d_vel, MIR_VEL, vel, mask));
    if (angvel) ZA_TRY(write_state_array(d_angvel, MIR_ANGVEL, angvel, mask));
    ZA_TRY(fill_u32(stream, d_counts, E, 0));
    dirty[MIR_COUNT] = true;
    return refresh_views();
}

const void* World::device_src(MirrorId id) const {
    switch (id) {
        case MIR_POS: return d_pos;
        case MIR_QUAT: return d_quat;
        case MIR_VEL: return d_vel;
        case MIR_ANGVEL: return d_angvel;
        case MIR_ACC: return d_acc;
        case MIR_JPOS: return d_jpos;
        case MIR_JVEL: return d_jvel;
        case MIR_JTRQ: return d_jtrq;
        case MIR_OBS: return d_obs;
        case MIR_CON: return d_con;
        case MIR_COUNT: return d_counts;
        default: return nullptr;
    }
}

void* World::mirror(MirrorId id, bool expose) {
    if (id < 0 || id >= MIR_COUNT_ALL || hipSetDevice(device) != hipSuccess) return nullptr;
    if (views_pending) {
        if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
        views_pending = false;
    }
    if (dirty[id]) {
        if (hipMemcpyAsync(h_mirror[id], device_src(id), mirror_bytes[id], hipMemcpyDeviceToHost, stream) != hipSuccess)
            return nullptr;
        if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
        dirty[id] = false;
    }
    if (expose) exposed[id] = true;
    return h_mirror[id];
}

// The copies run on view_stream behind an event of the step stream, and the call waits for
// them: a held view must show the state the call produced when the call returns.
hipError_t World::refresh_views() {
    bool any = false;
    for (int i = 0; i < MIR_COUNT_ALL; ++i) any = any || (exposed[i] && dirty[i]);
    if (!any) {
        // Views the step kernel stored itself are current once the stream is done.
        if (views_pending) {
            ZA_TRY(hipStreamSynchronize(stream));
            views_pending = false;
        }
        return hipSuccess;
    }
    views_pending = false;
    ZA_TRY(hipEventRecord(view_evt, stream));
    ZA_TRY(hipStreamWaitEvent(view_stream, view_evt, 0));
    for (int i = 0; i < MIR_COUNT_ALL; ++i) {
        if (!(exposed[i] && dirty[i])) continue;
        ZA_TRY(hipMemcpyAsync(h_mirror[i], device_src((MirrorId)i), mirror_bytes[i], hipMemcpyDeviceToHost, view_stream));
    }
    ZA_TRY(hipStreamSynchronize(view_stream));
    for (int i = 0; i < MIR_COUNT_ALL; ++i) {
        if (exposed[i]) dirty[i] = false;
    }
    return hipSuccess;
}

hipError_t World::get_profiling(ZenoProfilingData* out) {
    if (profiling && prof_pending) {
        ZA_TRY(hipEventSynchronize(prof_stop));
        float ms = 0.0f;
        ZA_TRY(hipEventElapsedTime(&ms, prof_start, prof_stop));
        prof = ZenoProfilingData{};
        prof.total_step_ns = ms * 1.0e6f;
        // Per-phase wall-clock time of workgroup 0 (in-kernel s_memrealtime stamps).
        unsigned long long t[kPhaseCount] = {};
        ZA_TRY(hipMemcpy(t, d_phase, sizeof t, hipMemcpyDeviceToHost));
        const double ns = 1e9 / wall_clock_hz;
        prof.integrate_ns = (float)((double)(t[PH_LOAD] + t[PH_FORCES] + t[PH_POST] + t[PH_STORE]) * ns);
        prof.collision_broad_ns = (float)((double)t[PH_BROAD] * ns);
        prof.collision_narrow_ns = (float)((double)t[PH_NARROW] * ns);
        prof.constraint_solve_ns = (float)((double)(t[PH_JOINTS] + t[PH_CONTACTS]) * ns);
        const uint32_t* counts = (const uint32_t*)mirror(MIR_COUNT, false);
        uint64_t total = 0;
        if (counts) for (uint32_t e = 0; e < E; ++e) total += counts[e];
        prof.num_contacts = (uint32_t)std::min<uint64_t>(total, 0xFFFFFFFFull);
        prof.num_active_constraints = N * E;
        prof_pending = false;
    }
    *out = prof;
    return hipSuccess;
}

hipError_t World::kernel_timing(double* ms, uint64_t* launches) {
    ZA_TRY(hipStreamSynchronize(stream));
    double total = 0.0;
    for (size_t i = 0; i + 1 < t_used; i += 2) {
        float x = 0.0f;
        ZA_TRY(hipEventElapsedTime(&x, t_events[i], t_events[i + 1]));
        total += x;
    }
    *ms = total;
    *launches = t_used / 2;
    t_used = 0;
    return hipSuccess;
}

}  // namespace za
