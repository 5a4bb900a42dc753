// Arguments and LDS layout of the fused step kernel (shared by host and device code).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "layout.h"

namespace za {

// Byte offsets of one environment's working set in LDS. Every section is 16-byte aligned.
struct EnvLds {
    uint32_t pos, quat, vel, angvel, ppos, pquat, frc, trq, vbefore;  // float4[B]
    uint32_t jt, jp, jv;                                               // float[J']
    uint32_t lam;                                                      // float[N]
    uint32_t con;                                                      // ContactRec[M] (physical)
    uint32_t perm;                                                     // u16[M] logical -> physical
    uint32_t skey;                                                     // u32[M] sort keys / levels
    uint32_t pkey, ppen, pimp;                                         // prev: u32[M], float4[M], float4[M]
    uint32_t order;                                                    // u16[M] contact levels
    uint32_t last;                                                     // u16[B]
    uint32_t misc;                                                     // u32[4]: count, pcount, nlev, pad
    uint32_t bytes;                                                    // total, multiple of 16
};

inline uint32_t align16(uint32_t x) { return (x + 15u) & ~15u; }

inline EnvLds make_env_lds(uint32_t B, uint32_t Jp, uint32_t N, uint32_t M) {
    EnvLds L{};
    uint32_t o = 0;
    auto take = [&](uint32_t bytes) { uint32_t r = o; o = align16(o + bytes); return r; };
    L.pos = take(16 * B); L.quat = take(16 * B); L.vel = take(16 * B); L.angvel = take(16 * B);
    L.ppos = take(16 * B); L.pquat = take(16 * B); L.frc = take(16 * B); L.trq = take(16 * B);
    L.vbefore = take(16 * B);
    L.jt = take(4 * Jp); L.jp = take(4 * Jp); L.jv = take(4 * Jp);
    L.lam = take(4 * (N > 0 ? N : 1));
    L.con = take(64 * M);
    L.perm = take(2 * M);
    L.skey = take(4 * M);
    L.pkey = take(4 * M); L.ppen = take(16 * M); L.pimp = take(16 * M);
    L.order = take(2 * M);
    L.last = take(2 * B);
    L.misc = take(16);
    L.bytes = o;
    return L;
}

// Byte offsets of the per-scene model records inside the model blob. The blob is uploaded
// once per world and copied into the front of every workgroup's LDS at kernel start, so
// the solver phases never wait on global memory for model data.
struct ModelLayout {
    uint32_t invmi, com, flags;  // float4[B], float4[B], u32[B] (bit0 kinematic, bit1 inv_m > 1e-8)
    uint32_t joints;             // JointRec[J]
    uint32_t geoms;              // GeomRec[G]
    uint32_t pairs;              // u32[P]
    uint32_t acts;               // ActuatorRec[A]
    uint32_t sensors;            // SensorRec[S]
    uint32_t tmpl;               // ConstraintRec[N]
    uint32_t ranges;             // u32[2 * ncolors]
    uint32_t bytes;              // total, multiple of 16
};

inline ModelLayout make_model_layout(uint32_t B, uint32_t J, uint32_t G, uint32_t P, uint32_t A, uint32_t S,
                                     uint32_t N, uint32_t ncolors) {
    ModelLayout L{};
    uint32_t o = 0;
    auto take = [&](uint32_t bytes) { uint32_t r = o; o = align16(o + bytes); return r; };
    L.invmi = take(16 * B); L.com = take(16 * B); L.flags = take(4 * B);
    L.joints = take(80 * J); L.geoms = take(64 * G); L.pairs = take(4 * P);
    L.acts = take(32 * A); L.sensors = take(32 * S); L.tmpl = take(96 * N); L.ranges = take(8 * ncolors);
    L.bytes = o;
    return L;
}

struct StepArgs {
    // Sizes.
    uint32_t E, B, J, Jp, A, S, obsp, N, ncolors, M, P;
    uint32_t iters, substeps;
    // Scalars (SimParams, world.zig:35-56).
    float dt, inv_step, gx, gy, gz, restitution, baumgarte, slop;
    // Model blob (read-only, one copy per world), laid out by `ml`.
    const uint4* model;
    ModelLayout ml;
    // State (reference layouts, env-major).
    float4* pos; float4* quat; float4* vel; float4* angvel; float4* acc;  // [E*B]
    float* jpos; float* jvel; float* jtrq;                                // [E*J']
    float* obs;                                                           // [E*obs']
    float* lam;                                                           // [E*N]
    const float* actions;                                                 // [E*A]
    ContactRec* contacts;                                                 // [E*M]
    uint32_t* counts; uint32_t* pcounts;                                  // [E]
    // Optional: envs whose previous-contact snapshot lives in prev_contacts (set by
    // step_subset for envs it did not advance); null when unused.
    const uint8_t* prev_detached;   // [E]
    const ContactRec* prev_contacts; // [E*M]
    // Optional per-env mask: envs with mask 0 advance only their solver history (lambda,
    // prev contacts, prev count) and keep every visible buffer. Null = all envs.
    const uint8_t* step_mask;       // [E]
    ContactRec* prev_out;           // [E*M] snapshot target for masked-out envs
    uint8_t* prev_detached_out;     // [E]
    // Optional per-phase wall-clock ticks of workgroup 0 (profiling); null when unused.
    unsigned long long* phase_ticks; // [kPhaseCount]
    EnvLds lds;
};

// Phases timed by the kernel when profiling is enabled.
enum Phase { PH_LOAD, PH_FORCES, PH_BROAD, PH_NARROW, PH_JOINTS, PH_CONTACTS, PH_POST, PH_STORE, kPhaseCount };

// Largest dynamic LDS allocation one workgroup may request on `device`.
size_t max_lds_per_workgroup(int device);

// Launches ceil(E / envs_per_wave) single-wave workgroups. envs_per_wave in {1,2,4,8}.
hipError_t launch_step(const StepArgs& a, int envs_per_wave, hipStream_t stream);

// Largest M supported for a given envs_per_wave (the sort and the contact schedule keep
// M / lanes slots per lane in registers).
inline uint32_t max_contacts_for(int envs_per_wave) { return 8u * (64u / (uint32_t)envs_per_wave); }

}  // namespace za
