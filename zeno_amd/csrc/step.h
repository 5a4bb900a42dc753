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
    uint32_t order, loff;                                              // u16[M], u16[M+1]
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
    L.order = take(2 * M); L.loff = take(2 * (M + 1));
    L.last = take(2 * B);
    L.misc = take(16);
    L.bytes = o;
    return L;
}

struct StepArgs {
    // Sizes.
    uint32_t E, B, J, Jp, A, S, obsp, N, ncolors, M, P;
    uint32_t iters, substeps;
    // Scalars (SimParams, world.zig:35-56).
    float dt, inv_step, gx, gy, gz, restitution, baumgarte, slop;
    // Model (read-only, one copy per world).
    const float4* invmi;         // [B] (inv_m, invI.xyz)
    const float4* com;           // [B] COM offset
    const uint32_t* kinematic;   // [B] body_type == 1
    const JointRec* joints;      // [J]
    const GeomRec* geoms;        // [G]
    const ActuatorRec* acts;     // [A]
    const SensorRec* sensors;    // [S]
    const ConstraintRec* tmpl;   // [N] colour-sorted
    const uint32_t* color_ranges;// [ncolors][2]
    const uint32_t* pairs;       // [P] g | g' << 16
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
    EnvLds lds;
};

// Largest dynamic LDS allocation one workgroup may request on `device`.
size_t max_lds_per_workgroup(int device);

// Launches ceil(E / envs_per_wave) single-wave workgroups. envs_per_wave in {1,2,4,8}.
hipError_t launch_step(const StepArgs& a, int envs_per_wave, hipStream_t stream);

// Largest M supported for a given envs_per_wave (the sort keeps M / lanes records per lane).
inline uint32_t max_contacts_for(int envs_per_wave) { return 8u * (64u / (uint32_t)envs_per_wave); }

}  // namespace za
