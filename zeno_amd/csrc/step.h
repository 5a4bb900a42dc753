// Arguments and LDS layout of the fused step kernel (shared by host and device code).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "layout.h"

namespace za {

// Byte offsets of one environment's working set (in LDS, or in HBM for scenes too large
// for LDS). Every section is 16-byte aligned.
struct EnvLds {
    uint32_t pos, quat, vel, angvel, ppos, pquat, frc, trq, vbefore;  // float4[B]
    uint32_t jt, jp, jv;                                               // float[J']
    uint32_t lam;                                                      // float[N]
    uint32_t con;                                                      // ContactRec[M] (physical)
    uint32_t perm;                                                     // u16[M] logical -> physical
    uint32_t skey;                                                     // u32[M] sort keys (float4[J'] in stage C)
    uint32_t ppen, pimp;                                               // prev snapshot: float4[M] x2
    uint32_t order;                                                    // u16[M] level of each valid slot
    // Contact schedule, aliased onto arrays that are dead by then: vlist and lst (u16[M]
    // each: valid slots, valid slots by level) share skey; loff (u16[M + 2], level ranges
    // in lst) and the level computation's per-slot dynamic bodies and predecessors
    // (u32[M] each, at byte 8M and 12M) share ppen.
    uint32_t vlist, lst, loff;
    // Spatial-hash broad phase (scenes above kHashMinGeoms geoms), on skey as well: hkey
    // u32[hash_keys(G)] (cell << 14 | geom, sorted), then, staged, hpos float4[G] (world
    // centre and radius) and hmeta u32[G] (the model's compact geom word) of each geom.
    uint32_t hkey, hpos;
    uint32_t bmask;  // contact levels: u64[B][ceil(M/64)] slot masks per body
    // Joint solve records with compliance / dt^2 filled in: a per-environment copy used
    // when the model blob is read in place from HBM.
    uint32_t jrec;
    // Candidate-pair broad phase with the model records in HBM: each geom's local centre and
    // radius (float4[G]) and body | type << 16 (u32[G]), staged once per launch.
    uint32_t gst, gmeta;
    uint32_t obs;                                                      // float[obs']: the observation row
    uint32_t misc;                                                     // u32[4]: count, pcount, nlev, pad
    uint32_t bytes;                                                    // total, multiple of 16
};

inline uint32_t align16(uint32_t x) { return (x + 15u) & ~15u; }

// Spatial-hash sort length: G rounded up to a power of two.
inline uint32_t hash_pad(uint32_t G) { uint32_t p = 1; while (p < G) p <<= 1; return p; }
// Contact lists longer than kRankSortMax slots per lane are sorted by a bitonic network over
// the slots' keys (on skey) and logical positions (on order), both padded to a power of two.
constexpr uint32_t kRankSortMax = 8;
inline uint32_t sort_pad(uint32_t M) { return hash_pad(M); }
// Spatial-hash scratch (on the sort-key region): the sort keys, then 16-B aligned hpos
// float4[G] (world centre, radius) and hmeta u32[G] (the model's compact geom word: body,
// plane flag, filter class) of every geom, staged once per substep for the queries. Up to
// 1024 keys are sorted in registers and only the G real keys are stored; longer lists are
// sorted in LDS, padded to a power of two.
constexpr uint32_t kHashClasses = 32;  // filter classes the model's rows describe
inline uint32_t hash_keys(uint32_t G) { return hash_pad(G) <= 1024u ? G : hash_pad(G); }
inline uint32_t hash_hpos_off(uint32_t G) { return align16(4 * hash_keys(G)); }
// staged: with hpos / hmeta (the layout for working sets in HBM, where reading the model
// records and body poses in the queries would go to global memory).
inline uint32_t hash_bytes_for(uint32_t G, bool staged) {
    if (G <= kHashMinGeoms) return 0;
    return staged ? hash_hpos_off(G) + 20 * G : 4 * hash_keys(G);
}

// G = geom count (hash arrays only when G > kHashMinGeoms); jrec_bytes = size of the joint
// solve records when they are copied per environment (HBM working set), else 0;
// hash_staged: the spatial hash's staged geom centres and metadata (hpos / hmeta) are part of
// the layout (a working set whose contact arrays live in HBM as well, placement 3).
inline EnvLds make_env_lds(uint32_t B, uint32_t Jp, uint32_t N, uint32_t M, uint32_t G = 0, uint32_t jrec_bytes = 0,
                           bool stage_geoms = false, uint32_t obsp = 1, bool hash_staged = false) {
    EnvLds L{};
    uint32_t o = 0;
    auto take = [&](uint32_t bytes) { uint32_t r = o; o = align16(o + bytes); return r; };
    const uint32_t hash_bytes = hash_bytes_for(G, hash_staged);
    L.pos = take(16 * B); L.quat = take(16 * B); L.vel = take(16 * B); L.angvel = take(16 * B);
    L.ppos = take(16 * B); L.pquat = take(16 * B); L.frc = take(16 * B); L.trq = take(16 * B);
    L.vbefore = take(16 * B);
    L.jt = take(4 * Jp); L.jp = take(4 * Jp); L.jv = take(4 * Jp);
    L.lam = take(4 * (N > 0 ? N : 1));
    L.con = take(64 * M);
    L.perm = take(2 * M);
    L.skey = take(std::max(std::max(4 * sort_pad(M), 16 * Jp), hash_bytes));  // also stage-C joint contributions, hash
    L.ppen = take(16 * M); L.pimp = take(16 * M);
    L.order = take(2 * sort_pad(M));
    L.vlist = L.skey; L.lst = L.skey + 2 * M;
    L.loff = L.ppen;  // 16 * M >= 2 * (M + 2) for M >= 1
    L.hkey = L.skey;
    // The queries stage nothing when the working set is in LDS; in HBM (placement 3) they
    // stage each geom's centre and compact word after the sorted keys.
    L.hpos = L.skey + (hash_staged && G > kHashMinGeoms ? hash_hpos_off(G) : 0);
    // Per-body bit masks of the valid contact slots touching the body (u64[B][ceil(M/64)]),
    // on the force and torque arrays (dead from integration to the next substep) when they fit.
    const uint32_t mask_words = (M + 63) / 64;
    L.bmask = 8 * mask_words <= 32 ? L.frc : 0u;
    L.jrec = take(jrec_bytes);
    if (8 * mask_words > 32) L.bmask = take(8 * mask_words * B);
    if (stage_geoms) { L.gst = take(16 * G); L.gmeta = take(4 * G); }
    L.obs = take(4 * obsp);
    L.misc = take(16);
    L.bytes = o;
    return L;
}

// With the working sets in HBM (placement 2) the arrays that the contact pipeline and the
// spatial hash touch most (contact records, permutation, sort keys and everything aliased on
// them, the snapshot, levels, body slot masks) still live in LDS, in this compact layout of
// their own; only their offsets in the returned EnvLds are meaningful. With masks_in_lds
// false the body slot masks stay in the HBM working set (bmask = kInHbm): scenes with many
// bodies and long contact lists, whose masks alone would not fit.
// With the spatial hash the previous-contact snapshot shares the sort-key region too, above
// the sort keys, level lists and body masks: the kernel takes it after the broad phase (the
// hash's arrays are dead by then), so the region serves both and the layout stays small
// enough for two environments per SIMD.
constexpr uint32_t kInHbm = 0xFFFFFFFFu;
inline EnvLds make_env_lds_small(uint32_t B, uint32_t Jp, uint32_t M, uint32_t G = 0, bool stage_geoms = false,
                                 bool masks_in_lds = true) {
    EnvLds L{};
    uint32_t o = 0;
    auto take = [&](uint32_t bytes) { uint32_t r = o; o = align16(o + bytes); return r; };
    const bool hash = G > kHashMinGeoms;
    const uint32_t hash_bytes = hash_bytes_for(G, true);
    L.con = take(64 * M);
    L.perm = take(2 * M);
    const uint32_t mask_bytes = masks_in_lds ? 8 * ((M + 63) / 64) * B : 0u;
    // bmask follows vlist and lst on the sort-key region: the levels run after the sort and
    // the broad phase are done with it.
    const uint32_t lists = align16(std::max(std::max(4 * M + mask_bytes, 4 * sort_pad(M)), 16 * Jp));
    L.skey = take(std::max(hash ? lists + 32 * M : lists, hash_bytes));
    if (hash) {
        L.ppen = L.skey + lists; L.pimp = L.ppen + 16 * M;
    } else {
        L.ppen = take(16 * M); L.pimp = take(16 * M);
    }
    L.order = take(2 * sort_pad(M));
    L.vlist = L.skey; L.lst = L.skey + 2 * M;
    L.loff = L.ppen;
    L.hkey = L.skey;
    L.hpos = L.skey + (hash ? hash_hpos_off(G) : 0);
    L.bmask = masks_in_lds ? L.skey + 4 * M : kInHbm;
    if (stage_geoms) { L.gst = take(16 * G); L.gmeta = take(4 * G); }
    L.misc = take(16);
    L.bytes = o;
    return L;
}

// Joint-solve program. The colour-sorted constraint templates are re-packed on the host
// into solve records whose fields are exactly what one constraint type reads, with the
// static body data (inverse mass and inertia, centre of mass) already gathered, and into
// phases: runs of one constraint type inside one colour. Constraints of a colour share no
// body, so running a colour as several same-type phases gives the same result as any
// order inside the colour, and every phase takes one branch for the whole wave.
// Templates that the solver skips (types without a solver, or two static bodies) are
// dropped here.
constexpr float kTwoPiF = 6.28318548f;  // 2 * fp32(pi), the largest |2 atan2(y, x)|
constexpr uint32_t kJRecQuads = 8;  // float4 per solve record
constexpr uint32_t kJHalfQuads = 4;  // float4 per lane-pair half record
struct JointPhase { uint32_t type, start, count, pad; };

// Record layout (float4 quads). q0 = (ia, ib, template index, flags) [u32]; flags: bit0
// inv_m_a > 0, bit1 inv_m_b > 0, bits 8-15 the constraint type.
// Lane-pair types (POSITIONAL, ANGULAR, ANGULAR_LIMIT) hold two halves, quads 0-3 for the
// lane of body a and quads 4-7 for the lane of body b, each laid out as
//   h0 = q0,  h1 = inverse mass and inertia of the lane's body,
//   h2 = (vector, compliance): POSITIONAL the lane's anchor, ANGULAR the lane's axis,
//        ANGULAR_LIMIT the limit axis; .w is replaced by compliance / dt^2 at kernel start,
//   h3 = POSITIONAL the lane's centre of mass, ANGULAR_LIMIT (lower, upper), else 0,
// so each lane reads only its own half and needs no selects between the two bodies.
// Single-lane types (run by body a's lane) use quads 0-6:
//   q1 / q2 = inverse mass and inertia of body a / b, q3.w = compliance (-> / dt^2),
//   WELD:       q3.xyz anchor_a, q4.xyz anchor_b, q5 target quaternion
//   LIN. LIMIT: q3.xyz axis, q4.xyz anchor_b, q5.xy (lower, upper)
//   SLIDER:     q3.xyz anchor_a, q4.xyz anchor_b, q5.xyz axis, q6 target quaternion
inline bool joint_type_solved(uint32_t t) {
    return t == C_POSITIONAL || t == C_ANGULAR || t == C_ANGULAR_LIMIT || t == C_LINEAR_LIMIT || t == C_WELD ||
           t == C_SLIDER;
}
__host__ __device__ inline bool joint_type_paired(uint32_t t) { return t == C_POSITIONAL || t == C_ANGULAR || t == C_ANGULAR_LIMIT; }

inline void build_joint_program(const std::vector<ConstraintRec>& tmpl, const std::vector<uint32_t>& ranges,
                                const float* invmi /* [B][4] */, const float* com /* [B][4] */,
                                std::vector<float4>& recs, std::vector<JointPhase>& phases) {
    recs.clear();
    phases.clear();
    const uint32_t ncol = (uint32_t)(ranges.size() / 2);
    static const uint32_t order[] = {C_POSITIONAL, C_WELD, C_ANGULAR, C_ANGULAR_LIMIT, C_LINEAR_LIMIT, C_SLIDER};
    auto u = [](uint32_t x) { float f; std::memcpy(&f, &x, 4); return f; };
    for (uint32_t c = 0; c < ncol; ++c) {
        const uint32_t off = ranges[2 * c], cnt = ranges[2 * c + 1];
        for (uint32_t type : order) {
            JointPhase ph{type, (uint32_t)(recs.size() / kJRecQuads), 0u, 0u};
            for (uint32_t k = off; k < off + cnt; ++k) {
                const ConstraintRec& t = tmpl[k];
                if ((t.indices[3] & 0xFFu) != type) continue;
                const uint32_t ia = t.indices[0], ib = t.indices[1];
                const float* ma = invmi + 4 * ia;
                const float* mb = invmi + 4 * ib;
                if (ma[0] + mb[0] < 1e-8f) continue;  // all_shaders.metal:924: nothing to move
                // An angular limit whose bounds lie beyond +-2 pi can never act: its angle
                // 2 atan2(...) (:1206) is within +-6.28318548 for every input (atan2 returns at
                // most fp32(pi) = 3.14159274 in magnitude), so neither angle < lower nor
                // angle > upper holds (NaN compares false as well), the violation stays 0 and
                // the solve writes nothing (:1216). Such bounds are MJCF ranges in degrees, which
                // the reference's parser keeps as given (ant.xml's hips: -30..30).
                if (type == C_ANGULAR_LIMIT && t.limits[0] <= -kTwoPiF && t.limits[1] >= kTwoPiF) continue;
                float4 q[kJRecQuads];
                for (auto& x : q) x = make_float4(0, 0, 0, 0);
                const uint32_t flags = (ma[0] > 0 ? 1u : 0u) | (mb[0] > 0 ? 2u : 0u) | (type << 8);
                const float4 head = make_float4(u(ia), u(ib), u(k), u(flags));
                const float4 mia = make_float4(ma[0], ma[1], ma[2], ma[3]);
                const float4 mib = make_float4(mb[0], mb[1], mb[2], mb[3]);
                const float* A = t.anchor_a;
                const float* Bv = t.anchor_b;
                const float comp = A[3];
                if (joint_type_paired(type)) {
                    q[0] = head; q[1] = mia;
                    q[4] = head; q[5] = mib;
                    q[2] = make_float4(A[0], A[1], A[2], comp);
                    switch (type) {
                        case C_POSITIONAL:
                            q[6] = make_float4(Bv[0], Bv[1], Bv[2], comp);
                            q[3] = make_float4(com[4 * ia], com[4 * ia + 1], com[4 * ia + 2], 0);
                            q[7] = make_float4(com[4 * ib], com[4 * ib + 1], com[4 * ib + 2], 0);
                            break;
                        case C_ANGULAR:
                            q[6] = make_float4(Bv[0], Bv[1], Bv[2], comp);
                            break;
                        case C_ANGULAR_LIMIT:
                            q[6] = q[2];
                            q[3] = q[7] = make_float4(t.limits[0], t.limits[1], 0, 0);
                            break;
                    }
                } else {
                    q[0] = head; q[1] = mia; q[2] = mib;
                    q[3] = make_float4(A[0], A[1], A[2], comp);
                    switch (type) {
                        case C_WELD:
                            q[4] = make_float4(Bv[0], Bv[1], Bv[2], 0);
                            q[5] = make_float4(t.axis_target[0], t.axis_target[1], t.axis_target[2], t.axis_target[3]);
                            break;
                        case C_LINEAR_LIMIT:
                            q[4] = make_float4(Bv[0], Bv[1], Bv[2], 0);
                            q[5] = make_float4(t.limits[0], t.limits[1], 0, 0);
                            break;
                        case C_SLIDER:
                            q[4] = make_float4(Bv[0], Bv[1], Bv[2], 0);
                            q[5] = make_float4(t.axis_target[0], t.axis_target[1], t.axis_target[2], 0);
                            q[6] = make_float4(t.limits[0], t.limits[1], t.limits[2], t.limits[3]);
                            break;
                    }
                }
                recs.insert(recs.end(), q, q + kJRecQuads);
                ++ph.count;
            }
            if (ph.count) phases.push_back(ph);
        }
    }
}

// Joints acting on each body for apply_joint_forces (all_shaders.metal:122-190), in
// ascending joint order: entry = joint index | bit 30 (body is the joint's parent, the
// contribution is negated) | bit 31 (prismatic: force, else torque). Body 0 gets none.
// The spatial hash's compact geom words and filter rows (ModelLayout.hmeta / hrow): a dense
// id per body that owns a geom (at most kHashMaxGeoms of them, so 14 bits), the plane flag,
// and a class per distinct (contype, conaffinity) pair in order of first appearance. The
// queries compare the ids for "different bodies" and test the filter of :493-522,
// (contype_a & conaffinity_b) || (contype_b & conaffinity_a), as bit c of row k for classes
// k and c. Returns false when there are more than kHashClasses classes: the rows are then
// unused and the queries read the masks from the geom records.
inline bool build_hash_words(const std::vector<GeomRec>& geoms, std::vector<uint32_t>& meta, std::vector<uint32_t>& rows) {
    std::vector<uint32_t> body_id, ct, ca;
    meta.assign(geoms.size(), 0u);
    rows.assign(kHashClasses, 0u);
    uint32_t ids = 0;
    bool fits = true;
    for (size_t g = 0; g < geoms.size(); ++g) {
        const GeomRec& gr = geoms[g];
        const uint32_t body = gr.type_body[1];
        if (body >= body_id.size()) body_id.resize((size_t)body + 1, 0xFFFFFFFFu);
        if (body_id[body] == 0xFFFFFFFFu) body_id[body] = ids++;
        uint32_t cls = 0;
        if (fits) {
            while (cls < ct.size() && !(ct[cls] == gr.type_body[3] && ca[cls] == gr.type_body[2])) ++cls;
            if (cls == ct.size()) {
                if (cls == kHashClasses) fits = false;
                else { ct.push_back(gr.type_body[3]); ca.push_back(gr.type_body[2]); }
            }
        }
        meta[g] = (body_id[body] & 0x3FFFu) | (gr.type_body[0] == GEOM_PLANE ? 1u << 14 : 0u) | ((fits ? cls : 0u) << 15);
    }
    if (!fits) {
        for (uint32_t& w : meta) w &= 0x7FFFu;
        return false;
    }
    for (size_t k = 0; k < ct.size(); ++k)
        for (size_t c = 0; c < ct.size(); ++c)
            if ((ct[k] & ca[c]) != 0u || (ct[c] & ca[k]) != 0u) rows[k] |= 1u << c;
    return true;
}

inline void build_body_joint_lists(const std::vector<JointRec>& joints, uint32_t B, std::vector<uint32_t>& off,
                                   std::vector<uint32_t>& ent) {
    off.assign(B + 1, 0);
    ent.clear();
    for (uint32_t b = 0; b < B; ++b) {
        off[b] = (uint32_t)ent.size();
        if (b == 0) continue;
        for (uint32_t j = 0; j < joints.size(); ++j) {
            const uint32_t ja = (uint32_t)joints[j].params[1], jb = (uint32_t)joints[j].params[2];
            if (ja != b && jb != b) continue;
            const bool prism = (uint32_t)joints[j].params[0] == JOINT_PRISMATIC;
            ent.push_back(j | (ja == b ? (1u << 30) : 0u) | (prism ? (1u << 31) : 0u));
        }
    }
    off[B] = (uint32_t)ent.size();
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
    uint32_t jrec;               // float4[kJRecQuads * R] joint solve records
    uint32_t jphase;             // JointPhase[nph]
    uint32_t bjoff, bjl;         // u32[B + 1] offsets into u32[2J]: joints acting on each body
    // Spatial hash (G > kHashMinGeoms) only: hmeta u32[G], each geom's compact word for the
    // queries (bits 0-13 a dense id of its body, bit 14 plane, bits 15-19 its filter class),
    // and hrow u32[32], the classes' filter rows (bit c of row k: a geom of class k and one
    // of class c pass the contype / conaffinity test), valid when StepArgs.hrows is set.
    uint32_t hmeta, hrow;
    uint32_t bytes;              // total, multiple of 16
};

inline ModelLayout make_model_layout(uint32_t B, uint32_t J, uint32_t G, uint32_t P, uint32_t A, uint32_t S,
                                     uint32_t nrec, uint32_t nph) {
    ModelLayout L{};
    uint32_t o = 0;
    auto take = [&](uint32_t bytes) { uint32_t r = o; o = align16(o + bytes); return r; };
    L.invmi = take(16 * B); L.com = take(16 * B); L.flags = take(4 * B);
    L.joints = take(80 * J); L.geoms = take(64 * G); L.pairs = take(4 * P);
    L.acts = take(32 * A); L.sensors = take(32 * S);
    L.jrec = take(16 * kJRecQuads * nrec); L.jphase = take(16 * nph);
    L.bjoff = take(4 * (B + 1)); L.bjl = take(4 * 2 * J);
    const bool hash = G > kHashMinGeoms;
    L.hmeta = take(hash ? 4 * G : 0); L.hrow = take(hash ? 4 * kHashClasses : 0);
    L.bytes = o;
    return L;
}

struct StepArgs {
    // Sizes. G = geoms; Gp = G rounded up to a power of two (hash mode).
    uint32_t E, B, J, Jp, A, S, obsp, N, nrec, njph, M, P, G, Gp;
    uint32_t hash;  // 1: spatial-hash broad phase (G > kHashMinGeoms), 0: candidate pair list
    // 1: at most kHashClasses distinct (contype, conaffinity) pairs, so the hash queries test
    // the filter by the model's class rows; 0: they read both geoms' masks from the records.
    uint32_t hrows;
    uint32_t ext_contacts;  // 1: pairs the reference's narrow phase leaves invalid use detectCollision
    // 1: sort the contact list in the first substep even if no append took a slot below M (the
    // host changed the counts, exposing slots whose order the last sort did not cover).
    uint32_t sort_all;
    // Count-only broad phase of a full list (one environment per wave): the non-plane geoms
    // (sweep_n <= 64, else 0 and the sweep is off) and the number of listed pairs with a plane.
    const uint32_t* sweep;
    uint32_t sweep_n, sweep_planes;
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
    // Device addresses of the host mirrors a caller holds (mapped pinned memory), else null:
    // the write-back stores each of these arrays there as well as to HBM, so a held view is
    // current when the stream completes, without a separate copy.
    struct HostViews {
        float4 *pos, *quat, *vel, *angvel, *acc;
        float *jpos, *jvel, *jtrq, *obs;
        ContactRec* contacts;
        uint32_t* counts;
    } hv;
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
    uint32_t* cell_ids;             // [E*G] hash mode: each geom's cell in the last substep
    uint32_t placement;             // Placement of the model records and working sets
    unsigned char* work;            // PL_ALL_HBM, PL_WORK_HBM: lds.bytes per environment; else null
    EnvLds lds;
    EnvLds lds_small;               // PL_ALL_HBM: the arrays kept in LDS (make_env_lds_small)
    // 1: body 0 is static (inverse mass < 1e-8) and not kinematic, and the bodies after it fill
    // whole passes of an environment's lanes. Its forces are zero, its previous pose is its
    // pose, and it is neither integrated nor given a velocity update, so the per-body stages
    // of the unsplit shapes take bodies 1.. across the lanes and set body 0's entries aside.
    uint32_t b_first;
};

// Where the step kernel keeps the model records and each environment's working set.
// PL_LDS: both in LDS (several environments per workgroup). PL_MODEL_HBM: the model blob
// is read in place from HBM (through the caches) and the working set is in LDS.
// PL_ALL_HBM: both in HBM, except the contact pipeline's arrays (make_env_lds_small), which
// stay in LDS. PL_WORK_HBM: everything in HBM, for contact lists too long for LDS
// (max_contacts_per_env beyond ~1,400: 64-B records, snapshot and sort keys are ~104 B per
// slot); the kernel then uses no LDS. The world scores the shapes that fit and keeps the best.
enum Placement : uint32_t { PL_LDS = 0, PL_MODEL_HBM = 1, PL_ALL_HBM = 2, PL_WORK_HBM = 3 };

// Phases timed by the kernel when profiling is enabled.
enum Phase { PH_LOAD, PH_FORCES, PH_BROAD, PH_NARROW, PH_JOINTS, PH_CONTACTS, PH_POST, PH_STORE, kPhaseCount };

// Largest dynamic LDS allocation one workgroup may request on `device`.
size_t max_lds_per_workgroup(int device);

// Step-kernel workgroups one CU holds at once for a launch shape (LDS and register
// limits, from the HIP occupancy query); 0 when the shape cannot launch.
// split: two waves per environment group (step_kernel's SPLIT instances); waves counts the
// groups of a workgroup either way.
int resident_workgroups(int envs_per_wave, uint32_t placement, bool hash, size_t shmem, int waves = 1, bool split = false);

// Launches ceil(E / (envs_per_wave * waves)) workgroups of `waves` environment groups, one
// wave per group (two with split). envs_per_wave in {1,2,4,8} and waves in 1..4; both 1 and
// split off unless a.placement is PL_LDS and the hash is off.
hipError_t launch_step(const StepArgs& a, int envs_per_wave, int waves, hipStream_t stream, bool split = false);


}  // namespace za
