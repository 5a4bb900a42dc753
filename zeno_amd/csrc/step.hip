// Fused physics step for CDNA4 (gfx950).
//
// One wave steps EPW environments; each environment owns G = 64 / EPW lanes and an LDS
// working set (bodies, joint state, lambdas, the contact list and the previous-contact
// snapshot). A workgroup holds up to four such groups sharing one LDS copy of the model
// records, and in the split shapes each group has a second wave that runs the contact
// pipeline while the first solves the joints (see step_kernel). A launch runs every substep
// of one zeno_world_step call, so HBM is read once and written once per call while all
// solver iterations stay in LDS.
//
// Stage order and arithmetic follow World.stepOnce (src/world/world.zig:934-1293) and the
// MSL kernels of src/shaders/all_shaders.metal, cited per stage. Where the reference runs
// unordered atomics or races, this kernel produces the deterministic schedule:
//   S1 broad-phase appends in (g, g') order: wave ballot + popcount prefix per env;
//   S2 per-body joint-force sums in ascending joint order, body_a before body_b;
//   S3 joint constraints per colour (bodies in one colour are disjoint);
//   S4 contact slots Gauss-Seidel in slot order: slots are levelled so that a slot runs
//      after every earlier slot sharing a body it writes, then levels run in order.
// The stable contact sort (all_shaders.metal:711-745) is a rank sort over a logical->physical
// permutation, so 64-byte records never move in LDS; the permutation is applied when the
// list is written back.
#include <hip/hip_runtime.h>

#include "dmath.h"
#include "narrow_ext.h"
#include "step.h"

namespace za {
namespace {

constexpr int kWave = 64;
constexpr int kMaxWaves = 4;  // waves per workgroup (model records in LDS: one copy shared by all)
constexpr int kMaxRecsPerLane = (int)kRankSortMax;

__device__ __forceinline__ uint32_t pair_key(uint32_t a, uint32_t b) {
    uint32_t lo = a < b ? a : b, hi = a < b ? b : a;
    return (lo << 16) | hi;
}

struct Lds {
    float4 *pos, *quat, *vel, *angvel, *ppos, *pquat, *frc, *trq, *vb;
    float *jt, *jp, *jv, *lam;
    ContactRec* con;
    uint16_t* perm;
    uint32_t* skey;
    float4 *ppen, *pimp;  // prev snapshot: position_pen; impulses.xyz with the pair key in .w
    float4* jw;  // per-joint force/torque contributions (stage C), aliased on skey
    uint16_t *order, *vlist, *lst, *loff;
    uint32_t* hkey;          // spatial hash, aliased on skey
    float4* hpos;            // spatial hash: geom world centre + radius (then u32 meta[G])
    uint32_t *vbod, *prv;    // contact levels: per-slot dynamic bodies and predecessors (on ppen)
    unsigned long long* bmask;  // contact levels: per-body slot masks
    float4* jrec;            // per-environment solve records (model records in HBM)
    float4* gst;             // staged geom local centre + radius (model records in HBM, no hash)
    uint32_t* gmeta;         // staged geom body | type << 16
    float* obs;              // the observation row (stage L), written back with the state
    uint32_t* misc;
};

__device__ __forceinline__ Lds bind_lds(unsigned char* base, const EnvLds& L) {
    Lds s;
    s.pos = (float4*)(base + L.pos); s.quat = (float4*)(base + L.quat);
    s.vel = (float4*)(base + L.vel); s.angvel = (float4*)(base + L.angvel);
    s.ppos = (float4*)(base + L.ppos); s.pquat = (float4*)(base + L.pquat);
    s.frc = (float4*)(base + L.frc); s.trq = (float4*)(base + L.trq);
    s.vb = (float4*)(base + L.vbefore);
    s.jt = (float*)(base + L.jt); s.jp = (float*)(base + L.jp); s.jv = (float*)(base + L.jv);
    s.lam = (float*)(base + L.lam);
    s.con = (ContactRec*)(base + L.con);
    s.perm = (uint16_t*)(base + L.perm);
    s.skey = (uint32_t*)(base + L.skey);
    s.jw = (float4*)(base + L.skey);
    s.ppen = (float4*)(base + L.ppen); s.pimp = (float4*)(base + L.pimp);
    s.order = (uint16_t*)(base + L.order);
    s.vlist = (uint16_t*)(base + L.vlist);
    s.lst = (uint16_t*)(base + L.lst);
    s.loff = (uint16_t*)(base + L.loff);
    s.hkey = (uint32_t*)(base + L.hkey);
    s.hpos = (float4*)(base + L.hpos);
    s.vbod = (uint32_t*)(base + L.ppen + 0u);  // placed by bind_levels
    s.prv = s.vbod;
    s.bmask = (unsigned long long*)(base + L.bmask);
    s.jrec = (float4*)(base + L.jrec);
    s.gst = (float4*)(base + L.gst);
    s.gmeta = (uint32_t*)(base + L.gmeta);
    s.obs = (float*)(base + L.obs);
    s.misc = (uint32_t*)(base + L.misc);
    return s;
}

// Rebinds the arrays of make_env_lds_small to base (working sets in HBM, placement 2).
__device__ __forceinline__ void bind_small(Lds& s, unsigned char* base, const EnvLds& L) {
    s.con = (ContactRec*)(base + L.con);
    s.perm = (uint16_t*)(base + L.perm);
    s.skey = (uint32_t*)(base + L.skey);
    s.jw = (float4*)(base + L.skey);
    s.ppen = (float4*)(base + L.ppen); s.pimp = (float4*)(base + L.pimp);
    s.order = (uint16_t*)(base + L.order);
    s.vlist = (uint16_t*)(base + L.vlist);
    s.lst = (uint16_t*)(base + L.lst);
    s.loff = (uint16_t*)(base + L.loff);
    s.hkey = (uint32_t*)(base + L.hkey);
    s.hpos = (float4*)(base + L.hpos);
    if (L.bmask != kInHbm) s.bmask = (unsigned long long*)(base + L.bmask);  // else: in the HBM working set
    s.gst = (float4*)(base + L.gst);
    s.gmeta = (uint32_t*)(base + L.gmeta);
    s.misc = (uint32_t*)(base + L.misc);
}

// The level computation's per-slot arrays (u32[M] each) at bytes 8M and 12M of the snapshot
// position array, which is dead once matching is done.
__device__ __forceinline__ void bind_levels(Lds& s, uint32_t M) {
    s.vbod = (uint32_t*)((unsigned char*)s.ppen + 8u * M);
    s.prv = (uint32_t*)((unsigned char*)s.ppen + 12u * M);
}

// Model records staged in LDS (see ModelLayout).
struct Mdl {
    const float4* invmi;
    const float4* com;
    const uint32_t* flags;
    const JointRec* joints;
    const GeomRec* geoms;
    const uint32_t* pairs;
    const ActuatorRec* acts;
    const SensorRec* sensors;
    const float4* jrec;
    const JointPhase* jph;
    const uint32_t *bjoff, *bjl;
    const uint32_t *hmeta, *hrow;
};

__device__ __forceinline__ Mdl bind_model(const unsigned char* base, const ModelLayout& L) {
    Mdl m;
    m.invmi = (const float4*)(base + L.invmi);
    m.com = (const float4*)(base + L.com);
    m.flags = (const uint32_t*)(base + L.flags);
    m.joints = (const JointRec*)(base + L.joints);
    m.geoms = (const GeomRec*)(base + L.geoms);
    m.pairs = (const uint32_t*)(base + L.pairs);
    m.acts = (const ActuatorRec*)(base + L.acts);
    m.sensors = (const SensorRec*)(base + L.sensors);
    m.jrec = (const float4*)(base + L.jrec);
    m.jph = (const JointPhase*)(base + L.jphase);
    m.bjoff = (const uint32_t*)(base + L.bjoff);
    m.bjl = (const uint32_t*)(base + L.bjl);
    m.hmeta = (const uint32_t*)(base + L.hmeta);
    m.hrow = (const uint32_t*)(base + L.hrow);
    return m;
}

__device__ __forceinline__ void set_xyz(float4* p, f3 v) { p->x = v.x; p->y = v.y; p->z = v.z; }

// ---------------------------------------------------------------------------------------
// solve_joints, all_shaders.metal:909-1399: one constraint per lane, read from its solve
// record (see build_joint_program), against LDS body state. One function per type.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t fbits(float x) { return __float_as_uint(x); }

// Single-wave workgroups: LDS operations of one wave complete in program order, so a
// compiler-level ordering point is all that is needed between dependent phases. A
// working set in HBM takes workgroup-scope fences (stores complete before later loads).
template <bool HBM>
__device__ __forceinline__ void wave_sync() {
    if (HBM) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Lane pairs. The positional, hinge and angular-limit solves run on two adjacent lanes:
// the even lane owns body a and the odd lane body b. Each lane evaluates the terms of its
// own body (anchor rotation, generalized inverse mass term, position and orientation
// update) and takes the partner's terms through a DPP swap, so one instruction stream
// covers both bodies. Shared quantities (the constraint error, its direction, the
// multiplier) are evaluated identically on both lanes, operands in the reference's order;
// where the reference subtracts body b's update (x - d) the odd lane adds (-1 * d), which
// is the same IEEE result. A sign applied to a product is applied to one of its factors
// instead ((-1 * x) * y and x * (-1 * y) round identically), never to a sum, whose zero signs
// it could change.
template <int PERM>
__device__ __forceinline__ float qperm(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), PERM, 0xF, 0xF, false));
}
// quad_perm(1, 0, 3, 2): the partner lane's value.
__device__ __forceinline__ float pair_swap(float v) { return qperm<0xB1>(v); }
// quad_perm(0, 0, 2, 2) and (1, 1, 3, 3): the even (body a) and odd (body b) lane's value on
// both lanes of the pair.
__device__ __forceinline__ f3 pair_a(f3 v) { return {qperm<0xA0>(v.x), qperm<0xA0>(v.y), qperm<0xA0>(v.z)}; }
__device__ __forceinline__ f3 pair_b(f3 v) { return {qperm<0xF5>(v.x), qperm<0xF5>(v.y), qperm<0xF5>(v.z)}; }
__device__ __forceinline__ q4 pair_a(q4 v) { return {qperm<0xA0>(v.x), qperm<0xA0>(v.y), qperm<0xA0>(v.z), qperm<0xA0>(v.w)}; }
__device__ __forceinline__ q4 pair_b(q4 v) { return {qperm<0xF5>(v.x), qperm<0xF5>(v.y), qperm<0xF5>(v.z), qperm<0xF5>(v.w)}; }
// qdelta with its factor 0.5 carrying the lane's sign: sg * (0.5 * x) == (sg * 0.5) * x.
__device__ __forceinline__ q4 qdelta_signed(f3 d, q4 q, float sg) { return qscale(qmul(mk4(d.x, d.y, d.z, 0.0f), q), 0.5f * sg); }

// The lane's half of a lane-pair solve record (build_joint_program): header, the lane's
// body's inverse mass and inertia, its vector (anchor or axis) with compliance / dt^2 in .w,
// and its centre of mass or the angular limits.
struct JHalf { float4 h0, mi, v1, v2; };
__device__ __forceinline__ JHalf load_half(const float4* p) { return JHalf{p[0], p[1], p[2], p[3]}; }
// The state a lane-pair solve reads for the lane's body: position, orientation and the
// constraint's multiplier (every record's header holds a valid multiplier index).
struct JState { float4 P, Q; float lam; };
__device__ __forceinline__ JState load_jstate(const JHalf& h, const Lds& s, bool odd) {
    const uint32_t me = odd ? fbits(h.h0.y) : fbits(h.h0.x);
    return JState{s.pos[me], s.quat[me], s.lam[fbits(h.h0.z)]};
}

// Late selects. The positional and hinge solves evaluate their update unconditionally and
// apply the reference's conditions (C > 1e-6, w > 1e-8, inverse mass > 0) only to the values
// they store: a compare that feeds a branch or a select right away waits about 30 cycles for
// its lane mask, while one whose mask is needed only at the stores overlaps the rest of the
// solve. A store that the reference skips writes back the value the lane read, so the memory
// is unchanged (the constraints of one phase touch disjoint bodies; a static body that several
// constraints share only ever gets its own value written back). The square roots compared
// against those thresholds use sqrt_gate, which is the correctly rounded root wherever the
// comparison can pass.

// :934-1037 positional (point-to-point), lane pair. r - qrot(com, q) is evaluated for every
// centre of mass: for com = +0 and a finite q the rotated offset is exactly +0 and r - (+0) == r.
__device__ __forceinline__ void solve_positional2(const JHalf& h, const JState& st, const Lds& s, bool odd) {
    const uint32_t ia = fbits(h.h0.x), ib = fbits(h.h0.y), ci = fbits(h.h0.z);
    const uint32_t me = odd ? ib : ia;
    const float alpha_tilde = h.v1.w;
    const float inv_mass = h.mi.x;
    const f3 iI = mk3(h.mi.y, h.mi.z, h.mi.w);
    const float sg = odd ? -1.0f : 1.0f;
    const f3 P = xyz(st.P);
    const q4 Q = toq(st.Q);
    const float lambda_prev = st.lam;
    const f3 rr = qrot(xyz(h.v1), Q);                      // r_a or r_b
    const f3 u = add(P, rr);                               // pos + r
    const f3 diff = sub(pair_a(u), pair_b(u));             // (pos_a + r_a) - (pos_b + r_b)
    const float C = len_gate(diff);
    const f3 n = divs(diff, C);
    const f3 rn = cross(rr, n);
    const float t = inv_mass + dot(mul(rn, iI), rn);
    const float w = t + pair_swap(t);                      // (w_a) + (w_b), addition commutes
    const float d_lambda = (-C - alpha_tilde * lambda_prev) / (w + alpha_tilde);
    const f3 impulse = sscale(d_lambda, n);
    const f3 rc = sub(rr, qrot(xyz(h.v2), Q));
    const f3 Pn = add(P, scale(impulse, sg * inv_mass));
    const q4 Qn = qnormalize_sel(qadd(Q, qdelta_signed(mul(cross(rc, impulse), iI), Q, sg)));
    const bool act = C > 1e-6f, moved = act && inv_mass > 0;
    s.lam[ci] = act ? lambda_prev + d_lambda : lambda_prev;  // both lanes store the same value
    set_xyz(&s.pos[me], moved ? Pn : P);
    s.quat[me] = tof4(moved ? Qn : Q);
}

// :1131-1186 hinge axis alignment, lane pair.
__device__ __forceinline__ void solve_angular2(const JHalf& h, const JState& st, const Lds& s, bool odd) {
    const uint32_t me = odd ? fbits(h.h0.y) : fbits(h.h0.x);
    const float alpha_tilde = h.v1.w;
    const float inv_mass = h.mi.x;
    const f3 iI = mk3(h.mi.y, h.mi.z, h.mi.w);
    const q4 Q = toq(st.Q);
    const f3 axw = qrot(xyz(h.v1), Q);
    const f3 cr = cross(pair_a(axw), pair_b(axw));
    const float sin_angle = len_gate(cr);
    const f3 n = divs(cr, sin_angle);
    const float ang_C = z_asinf(clampf(sin_angle, -1.0f, 1.0f));
    const float t = dot(mul(n, iI), n);
    const float w = t + pair_swap(t);
    const float d_lambda = -ang_C / (w + alpha_tilde);
    const float dl = odd ? -d_lambda : d_lambda;
    const q4 Qn = qnormalize_sel(qadd(Q, qdelta(mul(sscale(dl, n), iI), Q)));
    const bool moved = sin_angle > 1e-6f && w > 1e-8f && inv_mass > 0;
    s.quat[me] = tof4(moved ? Qn : Q);
}

// :1189-1238 angular limit, lane pair.
__device__ __forceinline__ void solve_angular_limit2(const JHalf& h, const JState& st, const Lds& s, bool odd) {
    const uint32_t me = odd ? fbits(h.h0.y) : fbits(h.h0.x);
    const float alpha_tilde = h.v1.w;
    const float inv_mass = h.mi.x;
    const f3 iI = mk3(h.mi.y, h.mi.z, h.mi.w);
    const float sg = odd ? -1.0f : 1.0f;
    const f3 axis_local = xyz(h.v1);
    const float lower = h.v2.x, upper = h.v2.y;
    const q4 Q = toq(st.Q);
    const q4 qa = pair_a(Q), qb = pair_b(Q);
    const q4 q_rel = qmul(qconj(qa), qb);
    const float angle = 2.0f * z_atan2f(dot(xyz(q_rel), axis_local), q_rel.w);
    float violation = 0.0f;
    if (angle < lower) violation = lower - angle;
    else if (angle > upper) violation = upper - angle;
    if (__builtin_fabsf(violation) > 1e-6f) {
        const f3 aw = qrot(axis_local, qa);
        const float t = dot(mul(aw, iI), aw);
        const float w = t + pair_swap(t);
        // Inside the violation branch (the common case is no violation, which skips the
        // update): the update is evaluated before its conditions, as above.
        const float d_lambda = violation / (w + alpha_tilde);
        const f3 ang_impulse = sscale(d_lambda, aw);
        const q4 Qn = qnormalize_sel(qadd(Q, qdelta_signed(mul(ang_impulse, iI), Q, sg)));
        if (w > 1e-8f && inv_mass > 0) s.quat[me] = tof4(Qn);
    }
}

// :1039-1129 weld (corrects body b only), one lane.
__device__ __forceinline__ void solve_weld(const float4* r, const Lds& s) {
    const float4 q0 = r[0], mb = r[2], a3 = r[3], b4 = r[4], tg = r[5];
    const uint32_t ia = fbits(q0.x), ib = fbits(q0.y);
    const float inv_mass_b = mb.x;
    const f3 iI_b = mk3(mb.y, mb.z, mb.w);
    const float alpha_tilde = a3.w;
    const f3 pos_a = xyz(s.pos[ia]), pos_b = xyz(s.pos[ib]);
    const q4 quat_a = toq(s.quat[ia]), quat_b = toq(s.quat[ib]);
    f3 r_a = qrot(xyz(a3), quat_a);
    f3 r_b = qrot(xyz(b4), quat_b);
    f3 diff = sub(add(pos_a, r_a), add(pos_b, r_b));
    float C = len(diff);
    q4 qb = quat_b;
    if (C > 1e-6f) {
        f3 n = divs(diff, C);
        f3 rn_b = cross(r_b, n);
        float w_b = inv_mass_b + dot(mul(rn_b, iI_b), rn_b);
        if (w_b > 1e-8f) {
            float d_lambda = (-C) / (w_b + alpha_tilde);
            f3 impulse = sscale(d_lambda, n);
            set_xyz(&s.pos[ib], sub(pos_b, scale(impulse, inv_mass_b)));
            qb = qnormalize(qsub(quat_b, qdelta(mul(cross(r_b, impulse), iI_b), quat_b)));
            s.quat[ib] = tof4(qb);
        }
    }
    const q4 target = toq(tg);
    const q4 qa = quat_a;
    q4 q_err = qmul(qmul(qconj(qa), qb), qconj(target));
    if (q_err.w < 0) q_err = qneg(q_err);
    f3 e = xyz(q_err);
    float sh = len(e);
    if (sh > 1e-6f) {
        f3 axis_rel = divs(e, sh);
        float angle = 2.0f * z_atan2f(sh, q_err.w);
        f3 aw = qrot(axis_rel, qa);
        float w_b = dot(mul(aw, iI_b), aw);
        if (w_b > 1e-8f) {
            float d_lambda_ang = angle / (w_b + alpha_tilde);
            f3 ang_impulse = sscale(d_lambda_ang, aw);
            if (inv_mass_b > 0) s.quat[ib] = tof4(qnormalize(qsub(qb, qdelta(mul(ang_impulse, iI_b), qb))));
        }
    }
}

// :1241-1293 linear limit, one lane.
__device__ __forceinline__ void solve_linear_limit(const float4* r, const Lds& s) {
    const float4 q0 = r[0], ma = r[1], mb = r[2], a3 = r[3], b4 = r[4], lim = r[5];
    const uint32_t ia = fbits(q0.x), ib = fbits(q0.y);
    const float inv_mass_a = ma.x, inv_mass_b = mb.x;
    const f3 iI_a = mk3(ma.y, ma.z, ma.w), iI_b = mk3(mb.y, mb.z, mb.w);
    const float alpha_tilde = a3.w;
    const f3 axis_local = xyz(a3);
    const float lower = lim.x, upper = lim.y;
    const f3 pos_a = xyz(s.pos[ia]), pos_b = xyz(s.pos[ib]);
    const q4 qa = toq(s.quat[ia]), qb = toq(s.quat[ib]);
    f3 r_a = qrot(mk3(0.0f, 0.0f, 0.0f), qa);
    f3 r_b = qrot(xyz(b4), qb);
    f3 aw = qrot(axis_local, qa);
    float dist = dot(sub(add(pos_b, r_b), add(pos_a, r_a)), aw);
    float violation = 0.0f;
    if (dist < lower) violation = lower - dist;
    else if (dist > upper) violation = upper - dist;
    if (__builtin_fabsf(violation) > 1e-6f) {
        f3 n = violation > 0 ? aw : neg(aw);
        float abs_v = __builtin_fabsf(violation);
        f3 rn_a = cross(r_a, n), rn_b = cross(r_b, n);
        float w = (inv_mass_a + dot(mul(rn_a, iI_a), rn_a)) + (inv_mass_b + dot(mul(rn_b, iI_b), rn_b));
        if (w > 1e-8f) {
            float d_lambda = abs_v / (w + alpha_tilde);
            f3 impulse = sscale(d_lambda, n);
            if (inv_mass_a > 0) set_xyz(&s.pos[ia], sub(pos_a, scale(impulse, inv_mass_a)));
            if (inv_mass_b > 0) set_xyz(&s.pos[ib], add(pos_b, scale(impulse, inv_mass_b)));
        }
    }
}

// :1296-1399 slider, one lane.
__device__ __forceinline__ void solve_slider(const float4* r, const Lds& s) {
    const float4 q0 = r[0], ma = r[1], mb = r[2], a3 = r[3], b4 = r[4], ax = r[5], tg = r[6];
    const uint32_t ia = fbits(q0.x), ib = fbits(q0.y);
    const float inv_mass_a = ma.x, inv_mass_b = mb.x;
    const f3 iI_a = mk3(ma.y, ma.z, ma.w), iI_b = mk3(mb.y, mb.z, mb.w);
    const float alpha_tilde = a3.w;
    const f3 pos_a = xyz(s.pos[ia]), pos_b = xyz(s.pos[ib]);
    const q4 quat_a = toq(s.quat[ia]), quat_b = toq(s.quat[ib]);
    f3 r_a = qrot(xyz(a3), quat_a);
    f3 r_b = qrot(xyz(b4), quat_b);
    f3 diff = sub(add(pos_a, r_a), add(pos_b, r_b));
    f3 aw = qrot(xyz(ax), quat_a);
    float along = dot(diff, aw);
    f3 perp = sub(diff, sscale(along, aw));
    float perp_len = len(perp);
    q4 qa = quat_a, qb = quat_b;
    if (perp_len > 1e-6f) {
        f3 n = divs(perp, perp_len);
        f3 rn_a = cross(r_a, n), rn_b = cross(r_b, n);
        float w = (inv_mass_a + dot(mul(rn_a, iI_a), rn_a)) + (inv_mass_b + dot(mul(rn_b, iI_b), rn_b));
        float d_lambda = (-perp_len) / (w + alpha_tilde);
        f3 impulse = sscale(d_lambda, n);
        if (inv_mass_a > 0) {
            set_xyz(&s.pos[ia], add(pos_a, scale(impulse, inv_mass_a)));
            qa = qnormalize(qadd(quat_a, qdelta(mul(cross(r_a, impulse), iI_a), quat_a)));
        }
        if (inv_mass_b > 0) {
            set_xyz(&s.pos[ib], sub(pos_b, scale(impulse, inv_mass_b)));
            qb = qnormalize(qsub(quat_b, qdelta(mul(cross(r_b, impulse), iI_b), quat_b)));
        }
    }
    const q4 target = toq(tg);
    q4 q_err = qmul(qmul(qconj(qa), qb), qconj(target));
    if (q_err.w < 0) q_err = qneg(q_err);
    f3 e = xyz(q_err);
    float sh = len(e);
    if (sh > 1e-6f) {
        f3 axis_err = divs(e, sh);
        float angle_err = 2.0f * z_atan2f(sh, q_err.w);
        f3 aw2 = qrot(axis_err, qa);
        float w = dot(mul(aw2, iI_a), aw2) + dot(mul(aw2, iI_b), aw2);
        if (w > 1e-8f) {
            float d_lambda_ang = angle_err / (w + alpha_tilde);
            f3 ang_impulse = sscale(d_lambda_ang, aw2);
            if (inv_mass_a > 0) qa = qnormalize(qadd(qa, qdelta(mul(ang_impulse, iI_a), qa)));
            if (inv_mass_b > 0) qb = qnormalize(qsub(qb, qdelta(mul(ang_impulse, iI_b), qb)));
        }
    }
    if (inv_mass_a > 0) s.quat[ia] = tof4(qa);
    if (inv_mass_b > 0) s.quat[ib] = tof4(qb);
}

// Inclusive max-scan of v over segments of G lanes (sl = lane within the segment): DPP row
// shifts when a segment lies inside one 16-lane row, LDS-backed shuffles otherwise.
template <int G>
__device__ __forceinline__ uint32_t seg_max_scan(uint32_t v, uint32_t sl) {
    if constexpr (G <= 16) {
        auto step = [&](uint32_t t, uint32_t d) { if (sl >= d) v = t > v ? t : v; };
        if constexpr (G > 1) step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false), 1);  // row_shr:1
        if constexpr (G > 2) step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false), 2);  // row_shr:2
        if constexpr (G > 4) step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false), 4);  // row_shr:4
        if constexpr (G > 8) step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false), 8);  // row_shr:8
    } else {
        for (uint32_t d = 1; d < (uint32_t)G; d <<= 1) {
            const uint32_t t = __shfl_up(v, d, G);
            if (sl >= d) v = t > v ? t : v;
        }
    }
    return v;
}

// ---------------------------------------------------------------------------------------
// solve_contacts, all_shaders.metal:1644-1793.
// ---------------------------------------------------------------------------------------
// solve_contacts on a lane pair: the even lane owns body a, the odd lane body b (see the
// joint lane pairs). Operands keep the reference's order; body b's updates, which the
// reference subtracts, are added with a factor of -1.
// The parts of a contact slot the solve reads that do not change during the solve
// iterations (only impulses.x does, written by the slot's own solve), so they can be read
// ahead of the slot's turn.
struct CRec {
    float4 pp, nf, aux;  // position_pen, normal_friction, (bias, share a, share b, inverse mass sum)
    uint32_t ia, ib, phys;
    float rest;          // impulses.w
};

__device__ __forceinline__ CRec load_crec(const Lds& s, uint32_t phys) {
    const ContactRec* cr = &s.con[phys];
    CRec c;
    c.pp = *(const float4*)cr->position_pen;
    c.nf = *(const float4*)cr->normal_friction;
    c.aux = s.pimp[phys];
    c.ia = cr->indices[0];
    c.ib = cr->indices[1];
    c.phys = phys;
    c.rest = cr->impulses[3];
    return c;
}

__device__ __forceinline__ void solve_contact_rec(const Mdl& md, const Lds& s, const CRec& c, bool odd) {
    ContactRec* cr = &s.con[c.phys];
    const float4 pp = c.pp;
    const float4 nf = c.nf;
    const float4 aux = c.aux;
    const uint32_t me = odd ? c.ib : c.ia;
    const float4 imi = md.invmi[me];
    const float inv_mass = imi.x;
    const f3 iI = mk3(imi.y, imi.z, imi.w);
    const float inv_mass_sum = aux.w;
    if (inv_mass_sum < 1e-8f) return;
    const f3 normal = mk3(nf.x, nf.y, nf.z);
    const float friction = nf.w;
    const f3 cp = mk3(pp.x, pp.y, pp.z);
    const float4 P0 = s.pos[me], V0 = s.vel[me], W0 = s.angvel[me];
    // impulses.x (the slot's normal impulse from the previous iteration, written only by
    // this solve) is read with the body state, so that read lands in the same round trip.
    float jn_prev = cr->impulses[0];
    const float sg = odd ? -1.0f : 1.0f;
    const f3 r = sub(cp, xyz(P0));
    const f3 vpt = add(xyz(V0), cross(xyz(W0), r));
    asm volatile("" : "+v"(jn_prev));
    const f3 rel_vel = sub(pair_a(vpt), pair_b(vpt));
    const float vel_normal = dot(rel_vel, normal);
    const f3 vel_tangent = sub(rel_vel, sscale(vel_normal, normal));
    const float tangent_speed = len_gate(vel_tangent);  // used only when > 1e-6
    const f3 rn = cross(r, normal);
    const float tn = inv_mass + dot(mul(rn, iI), rn);
    const float w_normal = tn + pair_swap(tn);
    if (w_normal < 1e-8f) return;
    const float bias = aux.x;
    const float restitution = c.rest;
    const float vel_restitution = vel_normal < -0.5f ? restitution * vel_normal : 0.0f;
    float j_n = (-(vel_normal + vel_restitution) + bias) / w_normal;
    j_n = fmaxf(j_n, 0.0f);
    const f3 impulse_n = sscale(j_n, normal);
    f3 v = xyz(V0), w = xyz(W0);
    const f3 siI = sscale(sg, iI);
    if (inv_mass > 1e-8f) {
        v = add(v, scale(impulse_n, sg * inv_mass));
        w = add(w, mul(cross(r, impulse_n), siI));
        set_xyz(&s.pos[me], add(xyz(P0), sscale(sg * (odd ? aux.z : aux.y), normal)));
    }
    const float j_n_acc = jn_prev + j_n;
    if (tangent_speed > 1e-6f && j_n_acc > 1e-6f) {
        const f3 tangent = divs(vel_tangent, tangent_speed);
        const f3 rt = cross(r, tangent);
        const float tt = inv_mass + dot(mul(rt, iI), rt);
        const float w_tangent = tt + pair_swap(tt);
        if (w_tangent > 1e-8f) {
            const float j_t = fminf(tangent_speed / w_tangent, friction * j_n_acc);
            const f3 impulse_t = sscale(j_t, tangent);
            if (inv_mass > 1e-8f) {
                v = add(v, scale(impulse_t, -sg * inv_mass));
                w = add(w, mul(cross(r, impulse_t), neg(siI)));
            }
        }
    }
    if (inv_mass > 1e-8f) {
        set_xyz(&s.vel[me], v);
        set_xyz(&s.angvel[me], w);
    }
    cr->impulses[0] = j_n;  // both lanes store the same value
}

__device__ __forceinline__ void solve_contact2(const Mdl& md, const Lds& s, uint32_t phys, bool odd) {
    solve_contact_rec(md, s, load_crec(s, phys), odd);
}

// ---------------------------------------------------------------------------------------
// narrow_phase, all_shaders.metal:751-894, one slot.
// ---------------------------------------------------------------------------------------
// AHEAD (model records in HBM): both geom records are read whole at the start, so their reads
// are in flight together instead of some waiting behind the type tests.
template <bool AHEAD>
__device__ __forceinline__ void narrow_slot(const StepArgs& a, const Mdl& md, const Lds& s, ContactRec* c) {
    const uint32_t body_a = c->indices[0], body_b = c->indices[1];
    GeomRec la, lb;
    if constexpr (AHEAD) {
        la = md.geoms[c->indices[2]];
        lb = md.geoms[c->indices[3]];
    }
    const GeomRec& ga = AHEAD ? la : md.geoms[c->indices[2]];
    const GeomRec& gb = AHEAD ? lb : md.geoms[c->indices[3]];
    const f3 pos_a = add(xyz(s.pos[body_a]), mk3(ga.pos_size0[0], ga.pos_size0[1], ga.pos_size0[2]));
    const f3 pos_b = add(xyz(s.pos[body_b]), mk3(gb.pos_size0[0], gb.pos_size0[1], gb.pos_size0[2]));
    const uint32_t type_a = ga.type_body[0], type_b = gb.type_body[0];
    f3 normal = mk3(0, 0, 0), cp = mk3(0, 0, 0);
    float pen = 0.0f;
    bool hit = false;
    if (type_a == GEOM_SPHERE && type_b == GEOM_SPHERE) {
        float ra = ga.pos_size0[3], rb = gb.pos_size0[3];
        f3 diff = sub(pos_b, pos_a);
        float dist = len(diff);
        float min_dist = ra + rb;
        if (dist < min_dist && dist > 1e-6f) {
            normal = divs(diff, dist);
            pen = min_dist - dist;
            cp = add(pos_a, scale(normal, ra - pen * 0.5f));
            hit = true;
        }
    } else if ((type_a == GEOM_SPHERE && type_b == GEOM_PLANE) || (type_a == GEOM_PLANE && type_b == GEOM_SPHERE)) {
        const f3 plane_normal = mk3(0, 0, 1);
        f3 sphere_pos = type_a == GEOM_SPHERE ? pos_a : pos_b;
        float radius = type_a == GEOM_SPHERE ? ga.pos_size0[3] : gb.pos_size0[3];
        f3 plane_pos = type_a == GEOM_SPHERE ? pos_b : pos_a;
        float signed_dist = dot(sub(sphere_pos, plane_pos), plane_normal);
        if (signed_dist < radius) {
            normal = plane_normal;
            pen = radius - signed_dist;
            cp = sub(sphere_pos, scale(plane_normal, signed_dist + pen * 0.5f));
            hit = true;
            if (type_a == GEOM_PLANE) normal = neg(normal);
        }
    } else if ((type_a == GEOM_CAPSULE && type_b == GEOM_PLANE) || (type_a == GEOM_PLANE && type_b == GEOM_CAPSULE)) {
        const f3 plane_normal = mk3(0, 0, 1);
        const GeomRec& gc = type_a == GEOM_CAPSULE ? ga : gb;
        f3 cap_pos = type_a == GEOM_CAPSULE ? pos_a : pos_b;
        float r = gc.pos_size0[3], hl = gc.params[0];
        f3 axis = qrot(mk3(0, 0, 1), mk4(gc.quat[0], gc.quat[1], gc.quat[2], gc.quat[3]));
        f3 p1 = sub(cap_pos, scale(axis, hl));
        f3 p2 = add(cap_pos, scale(axis, hl));
        float d1 = p1.z - r, d2 = p2.z - r;
        if (d1 < 0 || d2 < 0) {
            f3 deepest = d1 < d2 ? p1 : p2;
            float dist = fminf(d1, d2);
            normal = type_a == GEOM_CAPSULE ? plane_normal : neg(plane_normal);
            pen = -dist;
            cp = deepest;
            cp.z = 0;
            hit = true;
        }
    } else if (a.ext_contacts) {
        // Extended-contact mode (opt-in; the reference's step has none): the pairs its
        // narrow_phase kernel leaves invalid go through narrow_phase.detectCollision
        // (narrow_phase.zig:28-123) on the bodies' poses, and a contact becomes a slot
        // like any other (point, penetration, normal, friction, restitution). The contact
        // solve pushes body a along +normal, so the slot's normal points from b to a:
        // detectCollision gives that for every mixed pair and the opposite for
        // capsule-capsule and box-box, whose normal is negated here.
        const np::Side sa{type_a, mk3(ga.pos_size0[3], ga.params[0], ga.params[1]),
                          mk3(ga.pos_size0[0], ga.pos_size0[1], ga.pos_size0[2]), xyz(s.pos[body_a]), toq(s.quat[body_a])};
        const np::Side sb{type_b, mk3(gb.pos_size0[3], gb.params[0], gb.params[1]),
                          mk3(gb.pos_size0[0], gb.pos_size0[1], gb.pos_size0[2]), xyz(s.pos[body_b]), toq(s.quat[body_b])};
        const np::Result r = np::detect(sa, sb);
        if (r.valid) {
            normal = type_a == type_b ? neg(r.normal) : r.normal;
            pen = r.pen;
            cp = r.point;
            hit = true;
        }
    }
    if (hit) {
        float mu = __builtin_sqrtf(ga.params[2] * gb.params[2]);
        *(float4*)c->position_pen = make_float4(cp.x, cp.y, cp.z, pen);
        *(float4*)c->normal_friction = make_float4(normal.x, normal.y, normal.z, mu);
        *(float4*)c->impulses = make_float4(0.0f, 0.0f, 0.0f, a.restitution);
    } else {
        c->position_pen[3] = -1.0f;
    }
}

// One joint solve of the given type on the lane pair: h is the lane's half record and st its
// body's state (lane-pair types), r the whole record in LDS (single-lane types, run by body
// a's lane, which read the state themselves).
__device__ __forceinline__ void solve_joint(uint32_t type, const JHalf& h, const JState& st, const float4* r, const Lds& s,
                                            bool odd) {
    switch (type) {
        case C_POSITIONAL: solve_positional2(h, st, s, odd); break;
        case C_ANGULAR: solve_angular2(h, st, s, odd); break;
        case C_ANGULAR_LIMIT: solve_angular_limit2(h, st, s, odd); break;
        case C_WELD: if (!odd) solve_weld(r, s); break;
        case C_LINEAR_LIMIT: if (!odd) solve_linear_limit(r, s); break;
        case C_SLIDER: if (!odd) solve_slider(r, s); break;
        default: break;
    }
}

// ---------------------------------------------------------------------------------------
// Spatial-hash broad phase, all_shaders.metal:556-703 (scenes above 512 geoms,
// world.zig:534). The reference's dense per-env grid (64^3 counters and offsets, a serial
// 262,144-cell scan per env) becomes a sorted list: every geom's key cell << 14 | geom is
// sorted in the env's working set, and a geom's 3x3x3 neighbourhood is nine rows of three
// consecutive cell ids, each found by one binary search and read forward. Appends follow the sequential order
// of the reference's loops: geom ascending, then dz, dy, dx, then geoms of a cell in
// ascending order (the reference's atomic appends make any interleaving possible).
// ---------------------------------------------------------------------------------------
// Cell coordinate (:574-575): floor, GPU float->int conversion (NaN -> 0), clamp to [0, 63].
__device__ __forceinline__ uint32_t hash_axis(float p) {
    const float f = __builtin_floorf(p * 1.0f);
    return !(f >= 0.0f) ? 0u : (f >= 63.0f ? 63u : (uint32_t)f);
}

// Bitonic sort of n <= 1024 keys held in registers, one wave: lane l holds elements
// 16 l .. 16 l + 15 (positions from n on read as 0xFFFFFFFF and sort last, so the first n
// sorted elements are the n keys sorted). Passes whose partners are less than 16 apart
// compare registers of one lane; the others pair lane l with lane l ^ (distance / 16), each
// lane keeping the smaller or the larger of its two values. A sorting network's output is the
// sorted sequence whatever its steps, so the keys come out as any sort leaves them.
__device__ __forceinline__ void sort_keys_1024(uint32_t* key, uint32_t n, uint32_t lane) {
    uint32_t v[16];
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) v[r] = 16u * lane + r < n ? key[16u * lane + r] : 0xFFFFFFFFu;
#pragma unroll
    for (uint32_t k = 2; k <= 1024; k <<= 1) {
#pragma unroll
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            if (j >= 16) {
                const int d = (int)(j >> 4);
                const bool lower = (lane & (uint32_t)d) == 0u;
                const bool asc = ((16u * lane) & k) == 0u;
                const bool take_min = lower == asc;
#pragma unroll
                for (uint32_t r = 0; r < 16; ++r) {
                    const uint32_t p = (uint32_t)__shfl_xor((int)v[r], d);
                    v[r] = take_min ? (v[r] < p ? v[r] : p) : (v[r] < p ? p : v[r]);
                }
            } else {
#pragma unroll
                for (uint32_t r = 0; r < 16; ++r) {
                    if ((r & j) != 0u) continue;
                    const uint32_t r2 = r | j;
                    const bool asc = k < 16 ? (r & k) == 0u : ((16u * lane) & k) == 0u;
                    const uint32_t lo = v[r] < v[r2] ? v[r] : v[r2], hi = v[r] < v[r2] ? v[r2] : v[r];
                    v[r] = asc ? lo : hi;
                    v[r2] = asc ? hi : lo;
                }
            }
        }
    }
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) {
        if (16u * lane + r < n) key[16u * lane + r] = v[r];
    }
}

// Pairs (g, other > g) of one geom (:632-700). Returns their number; with emit set, writes
// pair k to logical slot `slot + k` while that is below M.
// STAGED: the geom data come from hpos / hmeta (working sets in HBM); otherwise from the
// model records and the body poses directly (both in LDS, or the model records in cache).
template <bool STAGED>
__device__ __forceinline__ float4 hash_geom_pos(const Mdl& md, const Lds& s, uint32_t g) {
    if (STAGED) return s.hpos[g];
    const GeomRec& gr = md.geoms[g];
    return tof4(add(xyz(s.pos[gr.type_body[1]]), mk3(gr.pos_size0[0], gr.pos_size0[1], gr.pos_size0[2])), gr.pos_size0[3]);
}
template <bool STAGED>
__device__ __forceinline__ uint32_t hash_geom_meta(const Mdl& md, const uint32_t* hmeta, uint32_t g) {
    if (STAGED) return hmeta[g];
    return md.hmeta[g];
}
// Fields of a geom's compact word (ModelLayout.hmeta).
__device__ __forceinline__ uint32_t hw_body(uint32_t w) { return w & 0x3FFFu; }
__device__ __forceinline__ bool hw_plane(uint32_t w) { return ((w >> 14) & 1u) != 0u; }
__device__ __forceinline__ uint32_t hw_class(uint32_t w) { return (w >> 15) & 31u; }
// A geom's side of the contype / conaffinity test (:493-522): its class row, or, when the
// classes do not fit the rows, (contype, conaffinity) from its record.
__device__ __forceinline__ uint2 hash_filter_of(const StepArgs& a, const Mdl& md, uint32_t g, uint32_t w) {
    if (a.hrows) return make_uint2(md.hrow[hw_class(w)], 0u);
    const GeomRec& gr = md.geoms[g];
    return make_uint2(gr.type_body[3], gr.type_body[2]);
}
// (contype_a & conaffinity_b) || (contype_b & conaffinity_a) for the geom of filter words fa
// and geom o of word w.
__device__ __forceinline__ bool hash_filter_pass(const StepArgs& a, const Mdl& md, uint2 fa, uint32_t o, uint32_t w) {
    if (a.hrows) return ((fa.x >> hw_class(w)) & 1u) != 0u;
    const GeomRec& gr = md.geoms[o];
    return ((fa.x & gr.type_body[2]) | (gr.type_body[3] & fa.y)) != 0u;
}

template <bool STAGED>
__device__ __forceinline__ uint32_t hash_pairs_of(const StepArgs& a, const Mdl& md, const Lds& s, const uint32_t* hmeta, uint32_t g, bool emit,
                                  uint32_t slot) {
    const float4 pa4 = hash_geom_pos<STAGED>(md, s, g);
    const uint32_t wa = hash_geom_meta<STAGED>(md, hmeta, g);
    const uint2 fa = hash_filter_of(a, md, g, wa);
    const f3 pa = xyz(pa4);
    const float ra = pa4.w;
    // The geom's cell, from the same centre the staging hashed.
    const uint32_t id = hash_axis(pa.x) + hash_axis(pa.y) * 64u + hash_axis(pa.z) * 4096u;
    const int cx = (int)(id & 63u), cy = (int)((id >> 6) & 63u), cz = (int)(id >> 12);
    const uint32_t xlo = cx > 0 ? (uint32_t)cx - 1u : 0u, xhi = cx < 63 ? (uint32_t)cx + 1u : 63u;
    // The nine rows' first positions (first key whose cell is >= the row's first cell), by
    // binary searches run side by side: each step reads the nine midpoints unconditionally,
    // so the reads are in flight together. Rows outside the grid keep lo = G (no keys).
    uint32_t lo[9], hi[9], tg[9];
#pragma unroll
    for (int r = 0; r < 9; ++r) {
        const int ny = cy + r % 3 - 1, nz = cz + r / 3 - 1;
        const bool in = ny >= 0 && ny <= 63 && nz >= 0 && nz <= 63;
        tg[r] = in ? (uint32_t)ny * 64u + (uint32_t)nz * 4096u + xlo : 0u;
        lo[r] = in ? 0u : a.G;
        hi[r] = a.G;
    }
    for (uint32_t span = a.G; span > 0u; span >>= 1) {
        uint32_t kv[9];
#pragma unroll
        for (int r = 0; r < 9; ++r) {
            const uint32_t mid = (lo[r] + hi[r]) >> 1;
            kv[r] = s.hkey[mid < a.G ? mid : a.G - 1u];
        }
#pragma unroll
        for (int r = 0; r < 9; ++r) {
            const uint32_t mid = (lo[r] + hi[r]) >> 1;
            const bool act = lo[r] < hi[r];
            const bool below = (kv[r] >> 14) < tg[r];
            lo[r] = act && below ? mid + 1u : lo[r];
            hi[r] = act && !below ? mid : hi[r];
        }
    }
    uint32_t hits = 0;
    for (int dz = -1; dz <= 1; ++dz) {
        const int nz = cz + dz;
        if (nz < 0 || nz > 63) continue;
        for (int dy = -1; dy <= 1; ++dy) {
            const int ny = cy + dy;
            if (ny < 0 || ny > 63) continue;
            const uint32_t row = (uint32_t)ny * 64u + (uint32_t)nz * 4096u;
            const uint32_t last = (row + xhi) << 14 | 0x3FFFu;  // largest key of the row's cells
            const int r = (dz + 1) * 3 + (dy + 1);
            const uint32_t first = r == 0 ? lo[0] : r == 1 ? lo[1] : r == 2 ? lo[2] : r == 3 ? lo[3] : r == 4 ? lo[4]
                                 : r == 5 ? lo[5] : r == 6 ? lo[6] : r == 7 ? lo[7] : lo[8];
            for (uint32_t k = first; k < a.G; ++k) {
                const uint32_t key = s.hkey[k];
                if (key > last) break;
                const uint32_t o = key & 0x3FFFu;
                if (o <= g) continue;
                const uint32_t wb = hash_geom_meta<STAGED>(md, hmeta, o);
                if (hw_body(wa) == hw_body(wb)) continue;
                if (!hash_filter_pass(a, md, fa, o, wb)) continue;
                if (!(hw_plane(wa) || hw_plane(wb))) {
                    const float4 pb4 = hash_geom_pos<STAGED>(md, s, o);
                    const f3 diff = sub(xyz(pb4), pa);
                    const float min_dist = ra + pb4.w + 0.1f;
                    if (dot(diff, diff) >= min_dist * min_dist) continue;
                }
                if (emit && slot + hits < a.M) {
                    uint32_t* idx = s.con[s.perm[slot + hits]].indices;
                    idx[0] = md.geoms[g].type_body[1]; idx[1] = md.geoms[o].type_body[1]; idx[2] = g; idx[3] = o;
                }
                ++hits;
            }
        }
    }
    return hits;
}

// Count-only hash queries (one environment per wave, a full contact list): the number of
// pairs the queries above would append, without their order. Each unordered pair of geoms in
// adjacent cells is met once, from the earlier of the two in the sorted key list: there the
// other is in the same cell or in one of the 13 adjacent cells of larger id (dx + 64 dy +
// 4096 dz > 0), i.e. in five runs of the list: the rest of the cell and the cell at x + 1,
// the row y + 1 at z, and the rows y - 1, y, y + 1 at z + 1 (x - 1 .. x + 1 each). The pair
// tests are those of hash_pairs_of; each is symmetric in its two geoms (the difference's
// sign does not change its square, nor the radii's order their sum), so the earlier geom
// may take either role. The runs' nine ends are found by interleaved binary searches; then
// each lane walks its own candidates, or, when one lane holds more than twice the mean, the
// wave's candidates are dealt out four per lane at a time, each lane finding its candidate's
// run by a search over the lanes' prefix sums, so a crowded cell does not hold the wave up.
template <bool STAGED>
__device__ __forceinline__ uint32_t hash_count_forward(const StepArgs& a, const Mdl& md, const Lds& s, const uint32_t* hmeta, int lane) {
    constexpr int R = 5;
    const uint32_t NG = a.G;
    uint32_t hits = 0;
    for (uint32_t base = 0; base < NG; base += kWave) {
        const uint32_t i = base + (uint32_t)lane;
        const bool mine = i < NG;
        uint32_t ga = 0, rs[R], rl[R];
        uint32_t tgt[2 * R] = {};
        uint32_t key_i = mine ? s.hkey[i] : 0u;
        ga = key_i & 0x3FFFu;
        const uint32_t c = key_i >> 14;
        const uint32_t x = c & 63u, y = (c >> 6) & 63u, z = c >> 12;
        const uint32_t xlo = x > 0u ? x - 1u : 0u, xhi1 = (x < 63u ? x + 1u : 63u) + 1u;
        // Targets (first cell of a run, first cell past it); an empty run has equal targets.
        tgt[0] = 0u; tgt[1] = x < 63u ? c + 2u : c + 1u;
        if (y < 63u) { const uint32_t row = (y + 1u) * 64u + z * 4096u; tgt[2] = row + xlo; tgt[3] = row + xhi1; }
#pragma unroll
        for (uint32_t k = 0; k < 3; ++k) {
            const uint32_t yy = y + k;  // y - 1 + k, offset by one
            if (z < 63u && yy >= 1u && yy <= 64u) {
                const uint32_t row = (yy - 1u) * 64u + (z + 1u) * 4096u;
                tgt[4 + 2 * k] = row + xlo; tgt[5 + 2 * k] = row + xhi1;
            }
        }
        // Interleaved lower bounds over [i + 1, NG): the first position whose cell >= target.
        uint32_t lo[2 * R], hi[2 * R];
#pragma unroll
        for (int k = 0; k < 2 * R; ++k) { lo[k] = mine ? i + 1u : NG; hi[k] = NG; }
        // Each step reads the nine midpoints unconditionally (a finished search reads a valid
        // place and keeps its bounds), so the nine reads are in flight together.
        for (uint32_t span = NG; span > 0u; span >>= 1) {
            uint32_t kv[2 * R];
#pragma unroll
            for (int k = 1; k < 2 * R; ++k) {
                const uint32_t mid = (lo[k] + hi[k]) >> 1;
                kv[k] = s.hkey[mid < NG ? mid : NG - 1u];
            }
#pragma unroll
            for (int k = 1; k < 2 * R; ++k) {
                const uint32_t mid = (lo[k] + hi[k]) >> 1;
                const bool act = lo[k] < hi[k];
                const bool below = (kv[k] >> 14) < tgt[k];
                lo[k] = act && below ? mid + 1u : lo[k];
                hi[k] = act && !below ? mid : hi[k];
            }
        }
        // Run 0 starts right after i; the others between their two bounds.
        rs[0] = mine ? i + 1u : NG;
        rl[0] = lo[1] - rs[0];
#pragma unroll
        for (int k = 1; k < R; ++k) { rs[k] = lo[2 * k]; rl[k] = lo[2 * k + 1] - lo[2 * k]; }
        uint32_t n = 0;
#pragma unroll
        for (int k = 0; k < R; ++k) n += rl[k];
        // Inclusive prefix over the wave's lanes; T candidates this round.
        uint32_t inc = n;
        for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t t = (uint32_t)__shfl_up((int)inc, d);
            if (lane >= d) inc += t;
        }
        const uint32_t T = (uint32_t)__shfl((int)inc, kWave - 1);
        const float4 pa4 = mine ? hash_geom_pos<STAGED>(md, s, ga) : make_float4(0, 0, 0, 0);
        const uint32_t wa = mine ? hash_geom_meta<STAGED>(md, hmeta, ga) : 0u;
        const uint2 fa = mine ? hash_filter_of(a, md, ga, wa) : make_uint2(0u, 0u);
        // Balanced rounds (no lane with more than twice the mean's chunks) walk each lane's own
        // runs; others deal the candidates out.
        uint32_t nmax = n;
        for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t t = (uint32_t)__shfl_xor((int)nmax, d);
            nmax = t > nmax ? t : nmax;
        }
        if (nmax <= 2u * ((T + kWave - 1u) / kWave)) {
            // Four of the lane's candidates per trip: their positions first, then their reads
            // side by side, then the tests of hash_pairs_of (different bodies, contype /
            // conaffinity, and the distance unless a plane takes part; the distance is evaluated
            // whatever the other conditions give and combined with them after).
            constexpr int U = 4;
            uint32_t k = 0, left = rl[0], pos = rs[0];
            for (uint32_t q = 0; q < nmax; q += U) {
                uint32_t p[U];
                bool ok[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    ok[u] = q + (uint32_t)u < n;
                    p[u] = 0u;
                    if (ok[u]) {
                        while (left == 0u) {
                            ++k;
                            left = k == 1 ? rl[1] : k == 2 ? rl[2] : k == 3 ? rl[3] : rl[4];
                            pos = k == 1 ? rs[1] : k == 2 ? rs[2] : k == 3 ? rs[3] : rs[4];
                        }
                        p[u] = pos;
                        ++pos;
                        --left;
                    }
                }
                uint32_t o[U];
#pragma unroll
                for (int u = 0; u < U; ++u) o[u] = s.hkey[p[u]] & 0x3FFFu;
                uint32_t wb[U];
                float4 pb[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    wb[u] = hash_geom_meta<STAGED>(md, hmeta, o[u]);
                    pb[u] = hash_geom_pos<STAGED>(md, s, o[u]);
                }
                bool fp[U];
#pragma unroll
                for (int u = 0; u < U; ++u) fp[u] = hash_filter_pass(a, md, fa, o[u], wb[u]);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const bool pass = hw_body(wb[u]) != hw_body(wa) && fp[u];
                    const f3 diff = sub(xyz(pb[u]), xyz(pa4));
                    const float min_dist = pa4.w + pb[u].w + 0.1f;
                    const bool near = !(dot(diff, diff) >= min_dist * min_dist);
                    const bool plane = hw_plane(wa) || hw_plane(wb[u]);
                    hits += (ok[u] && pass && (plane || near)) ? 1u : 0u;
                }
            }
            continue;
        }
        // Four candidates per lane and trip (t, t + 64, t + 128, t + 192), each stage of the
        // four side by side: the owners (the first lane whose inclusive prefix exceeds t), the
        // candidates' places in their owners' runs, the owners' geoms, the reads, the tests.
        constexpr int D = 4;
        for (uint32_t t0 = 0; t0 < T; t0 += (uint32_t)D * kWave) {
            uint32_t tt[D], lo[D], hi[D];
#pragma unroll
            for (int u = 0; u < D; ++u) { tt[u] = t0 + (uint32_t)u * kWave + (uint32_t)lane; lo[u] = 0u; hi[u] = kWave - 1; }
            for (int step = 0; step < 6; ++step) {
#pragma unroll
                for (int u = 0; u < D; ++u) {
                    const uint32_t mid = (lo[u] + hi[u]) >> 1;
                    const uint32_t v = (uint32_t)__shfl((int)inc, (int)mid);
                    if (v > tt[u]) hi[u] = mid; else lo[u] = mid + 1u;
                }
            }
            uint32_t p[D];
            bool ok[D];
            float4 pa[D];
            uint32_t wo[D];
            uint2 fo[D];
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int ow = (int)lo[u];
                uint32_t c = tt[u] - ((uint32_t)__shfl((int)inc, ow) - (uint32_t)__shfl((int)n, ow));
                uint32_t pos = 0;
                bool found = false;
#pragma unroll
                for (int k = 0; k < R; ++k) {
                    const uint32_t len = (uint32_t)__shfl((int)rl[k], ow);
                    const uint32_t st = (uint32_t)__shfl((int)rs[k], ow);
                    if (!found && c < len) { pos = st + c; found = true; }
                    if (!found) c -= len;
                }
                p[u] = pos;
                ok[u] = tt[u] < T && found;
                if (STAGED) {  // the owner's geom from the staged arrays
                    const uint32_t go = (uint32_t)__shfl((int)ga, ow);
                    pa[u] = hash_geom_pos<STAGED>(md, s, go);
                    wo[u] = hash_geom_meta<STAGED>(md, hmeta, go);
                } else {
                    pa[u] = make_float4(__shfl(pa4.x, ow), __shfl(pa4.y, ow), __shfl(pa4.z, ow), __shfl(pa4.w, ow));
                    wo[u] = (uint32_t)__shfl((int)wa, ow);
                }
                fo[u] = make_uint2((uint32_t)__shfl((int)fa.x, ow), (uint32_t)__shfl((int)fa.y, ow));
            }
            uint32_t o[D];
#pragma unroll
            for (int u = 0; u < D; ++u) o[u] = s.hkey[p[u]] & 0x3FFFu;
            uint32_t wb[D];
            float4 pb[D];
#pragma unroll
            for (int u = 0; u < D; ++u) {
                wb[u] = hash_geom_meta<STAGED>(md, hmeta, o[u]);
                pb[u] = hash_geom_pos<STAGED>(md, s, o[u]);
            }
            bool fp[D];
#pragma unroll
            for (int u = 0; u < D; ++u) fp[u] = hash_filter_pass(a, md, fo[u], o[u], wb[u]);
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const bool pass = hw_body(wb[u]) != hw_body(wo[u]) && fp[u];
                const f3 diff = sub(xyz(pb[u]), xyz(pa[u]));
                const float min_dist = pa[u].w + pb[u].w + 0.1f;
                const bool near = !(dot(diff, diff) >= min_dist * min_dist);
                const bool plane = hw_plane(wo[u]) || hw_plane(wb[u]);
                hits += (ok[u] && pass && (plane || near)) ? 1u : 0u;
            }
        }
    }
    for (int d = 1; d < kWave; d <<= 1) hits += (uint32_t)__shfl_xor((int)hits, d);
    return hits;
}

// PL: where the model records and the working sets live (Placement): PL_LDS, both in LDS
// (EPW environments per wave, and up to kMaxWaves independent waves per workgroup sharing one
// copy of the model records); PL_MODEL_HBM, the model blob read in place from HBM and one
// working set in LDS; PL_ALL_HBM, both in HBM (the working set in a.work) but the contact
// pipeline's arrays in LDS; PL_WORK_HBM, all of it in HBM (no LDS), for contact lists longer
// than LDS holds.
// HASH: the spatial-hash broad phase (scenes above kHashMinGeoms geoms) instead of the
// candidate pair list. Both non-LDS placements and the hash run one environment per
// workgroup. GROUP: the narrow phase visits the slots grouped by geom-type pair (the
// extended-contact mode, one environment per workgroup); a separate instance, so that the
// other shapes' register allocation is not touched by it.
// The waves of a workgroup meet at one barrier, after the model records are in LDS; from
// there each wave steps its own environments and synchronises with itself only.
// SPLIT: two waves per group of EPW environments, on the same SIMD (wave w and wave w + NG of
// a workgroup of 2 NG waves). The solver wave runs stages A-D, the joint and contact solves
// and the post-solve stages; the helper wave runs the snapshot, the broad phase, the sort, the
// narrow phase, the cache matching and the contact levels while the solver runs the joints
// (these read the poses after integration and write nothing the joint solve reads), and
// writes the contact list back while the solver finishes. The solver leaves the poses after
// integration in the force and torque arrays (dead until the next substep) for the helper, as
// the joint solve moves the bodies meanwhile. Three workgroup barriers per substep order the
// two: after integration, before the contact solve and after it.
// Two waves per SIMD at most 256 registers: the one-environment shapes hide their memory
// latency with a second resident wave, and more than 256 registers would leave one.
template <int EPW, int PL, bool HASH, bool GROUP, bool SPLIT = false>
__global__ __launch_bounds__(SPLIT ? 2 * kMaxWaves * kWave : (PL == PL_LDS && !HASH ? kMaxWaves * kWave : kWave))
__attribute__((amdgpu_waves_per_eu(2)))
void step_kernel(StepArgs a) {
    constexpr int G = kWave / EPW;
    constexpr bool HBM = PL >= PL_ALL_HBM;  // working set in HBM
    // Placement 2 with the spatial hash keeps the previous-contact snapshot on the hash's
    // arrays (make_env_lds_small): it is taken after the broad phase.
    constexpr bool LATE_SNAP = HASH && PL == PL_ALL_HBM;
    static_assert(PL == PL_LDS || EPW == 1, "model records in HBM run one environment per workgroup");
    static_assert(!HASH || EPW == 1, "the spatial hash runs one environment per workgroup");
    static_assert(!GROUP || EPW == 1, "type-grouped narrow phase: one environment per workgroup");
    static_assert(!SPLIT || (PL == PL_LDS && !HASH && !GROUP), "split groups: working sets and model in LDS");
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = (int)(threadIdx.x & (kWave - 1));    // lane
    constexpr bool MULTI = PL == PL_LDS && !HASH;          // several waves per workgroup possible
    const uint32_t wv = MULTI ? threadIdx.x / kWave : 0u;  // wave in this workgroup
    const uint32_t W = MULTI ? blockDim.x / kWave : 1u;    // waves in this workgroup
    const uint32_t NG = SPLIT ? W / 2u : W;                 // environment groups in this workgroup
    const bool helper = SPLIT && wv >= NG;                  // split: the group's second wave
    const bool do_solve = !helper, do_prep = !SPLIT || helper;
    const uint32_t grp = SPLIT ? wv % NG : wv;              // this wave's group in the workgroup
    const uint32_t wave_id = blockIdx.x * NG + grp;         // environment group
    const int le = tid / G;
    const int sl = tid % G;
    const uint32_t env = wave_id * EPW + le;
    const bool live = env < a.E;
    unsigned char* const env_base = HBM ? a.work + (size_t)wave_id * a.lds.bytes
                                        : smem + (PL == PL_LDS ? a.ml.bytes : 0u) + grp * EPW * a.lds.bytes;
    Lds s = bind_lds(env_base + le * a.lds.bytes, a.lds);
    // The HBM working set's own snapshot arrays, unused by placement 2 but for a substep whose
    // appends may wrap the count past 2^32 (LATE_SNAP below).
    float4* const hppen = s.ppen;
    float4* const hpimp = s.pimp;
    if (PL == PL_ALL_HBM) bind_small(s, smem, a.lds_small);  // PL_WORK_HBM: all of it in a.work
    bind_levels(s, a.M);
    Mdl md = bind_model(PL == PL_LDS ? smem : (const unsigned char*)a.model, a.ml);
    if (PL != PL_LDS) md.jrec = s.jrec;
    const uint32_t B = a.B, M = a.M, N = a.N, Jp = a.Jp;
    const bool stepped = live && (a.step_mask == nullptr || a.step_mask[env] != 0);
    // Working sets in HBM: an advanced environment's pose and velocity arrays are its slices
    // of the state arrays themselves (the same layout), so they are neither copied in nor
    // written back. An environment that is not advanced keeps its visible state and works on
    // copies in the working set, as the other placements do.
    const bool alias = HBM && stepped;
    // Aliased and with no host view held, the last substep's velocity update writes each
    // dynamic body's acceleration itself (the write-back then covers the static bodies only).
    const bool j_acc = alias && !a.hv.pos && !a.hv.quat && !a.hv.vel && !a.hv.angvel && !a.hv.acc;
    if (alias) {
        const size_t eb0 = (size_t)env * a.B;
        s.pos = a.pos + eb0; s.quat = a.quat + eb0; s.vel = a.vel + eb0; s.angvel = a.angvel + eb0;
    }

    // Phase timer: workgroup 0, lane 0 accumulates wall-clock ticks per phase.
    const bool timer = a.phase_ticks != nullptr && blockIdx.x == 0 && threadIdx.x == 0;
    unsigned long long t_last = timer ? (unsigned long long)wall_clock64() : 0ull;
    unsigned long long t_acc[kPhaseCount] = {};
    auto tick = [&](int ph) {
        if (timer) {
            unsigned long long t = (unsigned long long)wall_clock64();
            t_acc[ph] += t - t_last;
            t_last = t;
        }
    };

    // ---- Model records (one blob per scene) and the env's working set -> LDS -----------
    // The environment's HBM reads are issued first and held in registers (up to kPreBodies
    // bodies, kPreSlots contact slots and two lambdas and joint torques per lane, which covers
    // every shape but the largest scenes), then the model records are copied (the same blob
    // for every workgroup: L2 hits), and only then is anything written to LDS, so the reads
    // of the different arrays overlap instead of waiting for one another. Entries beyond the
    // prefetch counts are copied by the loops after.
    // A contact slot's four quads, read ahead into registers.
    struct Slot4 { float4 q0, q1, q2, q3; };
    auto read_slot = [](const ContactRec* r) {
        const float4* v = (const float4*)r;
        return Slot4{v[0], v[1], v[2], v[3]};
    };
    auto write_slot = [](ContactRec* r, const Slot4& x) {
        float4* v = (float4*)r;
        v[0] = x.q0; v[1] = x.q1; v[2] = x.q2; v[3] = x.q3;
    };
    constexpr uint32_t kPreSlots = 4;  // slots per lane read ahead: 4 G, 64 at four envs per wave
    uint32_t count = 0, pcount = 0;
    bool detached = false;
    // The lane's first action (read by stage A of every substep) is loaded with the state.
    const float act0 = (live && do_solve && (uint32_t)sl < a.A) ? a.actions[(size_t)env * a.A + sl] : 0.0f;
    const size_t eb = (size_t)env * B;
    const ContactRec* gc = a.contacts + (size_t)env * M;
    const uint32_t b0 = sl, j0 = sl;
    // One environment per workgroup with the model records in HBM: a second body per lane is
    // read ahead as well, so scenes of up to 2 G bodies (the pile's 65) load in one round trip.
    constexpr bool PRE2 = EPW == 1 && PL == PL_MODEL_HBM && !HASH;
    // Split groups keep every body on the lanes (their solver chain gains nothing from it).
    const uint32_t bf = SPLIT ? 0u : a.b_first;
    float4 p_pos = make_float4(0, 0, 0, 0), p_quat = p_pos, p_vel = p_pos, p_ang = p_pos;
    float4 q_pos = p_pos, q_quat = p_pos, q_vel = p_pos, q_ang = p_pos;
    float p_jt = 0.0f, p_lam = 0.0f;
    Slot4 c0{}, c1{}, c2{}, c3{};
    if (live && do_solve) {
        if (b0 < B && !alias) {
            p_pos = a.pos[eb + b0];
            p_quat = a.quat[eb + b0];
            p_vel = a.vel[eb + b0];
            p_ang = a.angvel[eb + b0];
        }
        if (PRE2 && b0 + G < B) {
            q_pos = a.pos[eb + b0 + G];
            q_quat = a.quat[eb + b0 + G];
            q_vel = a.vel[eb + b0 + G];
            q_ang = a.angvel[eb + b0 + G];
        }
        if (j0 < Jp) p_jt = a.jtrq[(size_t)env * Jp + j0];
        if (j0 < N) p_lam = a.lam[(size_t)env * N + j0];
    }
    // The contact list and counts, read ahead into registers (one wave per group). A split
    // group's helper reads them after the first barrier of the first substep instead, straight
    // into LDS: the contact records are most of the bytes, and the helper needs them only after
    // integration, while the solver's body reads then meet no contact traffic.
    auto load_contacts = [&]() {
        if (sl < M) c0 = read_slot(&gc[sl]);
        if (sl + G < M) c1 = read_slot(&gc[sl + G]);
        if (sl + 2 * G < M) c2 = read_slot(&gc[sl + 2 * G]);
        if (sl + 3 * G < M) c3 = read_slot(&gc[sl + 3 * G]);
        count = a.counts[env];
        pcount = a.pcounts[env];
        detached = a.prev_detached != nullptr && a.prev_detached[env] != 0;
    };
    if (!SPLIT && live) load_contacts();
    // With the model records in HBM, the working-set reads follow the copy of the solve
    // records and the geom staging without a barrier in between, so their HBM latencies
    // overlap.
    // A split workgroup's solver waves copy the model records alone: a wave's loads return in
    // order, so a helper's share of the copy would land only after its contact records.
    const uint32_t copy_threads = SPLIT ? NG * kWave : blockDim.x;
    if (PL == PL_LDS && threadIdx.x < copy_threads) {
        const uint32_t nq = a.ml.bytes / 16u;
        uint4* const dst = (uint4*)smem;
        const uint32_t nt = copy_threads;
        for (uint32_t i0 = threadIdx.x; i0 < nq; i0 += 4u * nt) {
            const uint32_t i1 = i0 + nt, i2 = i0 + 2u * nt, i3 = i0 + 3u * nt;
            const uint4 q0 = a.model[i0];
            const uint4 q1 = i1 < nq ? a.model[i1] : q0;
            const uint4 q2 = i2 < nq ? a.model[i2] : q0;
            const uint4 q3 = i3 < nq ? a.model[i3] : q0;
            dst[i0] = q0;
            if (i1 < nq) dst[i1] = q1;
            if (i2 < nq) dst[i2] = q2;
            if (i3 < nq) dst[i3] = q3;
        }
    } else if (PL != PL_LDS) {
        const uint4* src = a.model + a.ml.jrec / 16u;
        for (uint32_t i = tid; i < a.nrec * kJRecQuads; i += kWave) ((uint4*)s.jrec)[i] = src[i];
        if (!HASH) {
            // Two geoms per lane and trip, both read before either is written.
            for (uint32_t g = tid; g < a.G; g += 2u * kWave) {
                const uint32_t g2 = g + kWave;
                const float4 ps = *(const float4*)md.geoms[g].pos_size0;
                const uint4 tb = *(const uint4*)md.geoms[g].type_body;
                float4 ps2 = ps;
                uint4 tb2 = tb;
                if (g2 < a.G) { ps2 = *(const float4*)md.geoms[g2].pos_size0; tb2 = *(const uint4*)md.geoms[g2].type_body; }
                s.gst[g] = ps;
                s.gmeta[g] = tb.y | (tb.x << 16);
                if (g2 < a.G) { s.gst[g2] = ps2; s.gmeta[g2] = tb2.y | (tb2.x << 16); }
            }
        }
    }

    // alpha~ = compliance / dt^2 (all_shaders.metal:928), the same value for every solve of
    // this launch: computed once per record, after the records have landed.
    auto fill_alpha = [&](uint32_t first, uint32_t stride) {
        for (uint32_t i = first; i < a.nrec; i += stride) {
            float4* q = (float4*)md.jrec + i * kJRecQuads;
            if (joint_type_paired((fbits(q[0].w) >> 8) & 0xFFu)) {
                q[2].w = q[2].w / (a.dt * a.dt);
                q[6].w = q[6].w / (a.dt * a.dt);
            } else {
                q[3].w = q[3].w / (a.dt * a.dt);
            }
        }
    };
    if (PL == PL_LDS) {
        __syncthreads();
        if (threadIdx.x < copy_threads) fill_alpha(threadIdx.x, copy_threads);  // the workgroup's one copy of the records
    }

    if (live && do_solve) {
        if (b0 < B && !alias) {  // aliased: the velocity at call start is taken by stage B of substep 0
            s.pos[b0] = p_pos;
            s.quat[b0] = p_quat;
            s.vel[b0] = p_vel;
            s.vb[b0] = p_vel;
            s.angvel[b0] = p_ang;
        }
        if (PRE2 && b0 + G < B) {
            s.pos[b0 + G] = q_pos;
            s.quat[b0 + G] = q_quat;
            s.vel[b0 + G] = q_vel;
            s.vb[b0 + G] = q_vel;
            s.angvel[b0 + G] = q_ang;
        }
        for (uint32_t b = sl + (PRE2 ? 2u : 1u) * G; b < B && !alias; b += G) {
            s.pos[b] = a.pos[eb + b];
            s.quat[b] = a.quat[eb + b];
            float4 v = a.vel[eb + b];
            s.vel[b] = v;
            s.vb[b] = v;
            s.angvel[b] = a.angvel[eb + b];
        }
        if (j0 < Jp) s.jt[j0] = p_jt;
        if (j0 < N) s.lam[j0] = p_lam;
        for (uint32_t j = sl + G; j < Jp; j += G) s.jt[j] = a.jtrq[(size_t)env * Jp + j];
        for (uint32_t i = sl + G; i < N; i += G) s.lam[i] = a.lam[(size_t)env * N + i];
    }
    // The contact list -> LDS (from the registers read ahead above).
    auto write_contacts = [&]() {
        if (sl < M) { write_slot(&s.con[sl], c0); s.perm[sl] = (uint16_t)sl; }
        if (sl + G < M) { write_slot(&s.con[sl + G], c1); s.perm[sl + G] = (uint16_t)(sl + G); }
        if (sl + 2 * G < M) { write_slot(&s.con[sl + 2 * G], c2); s.perm[sl + 2 * G] = (uint16_t)(sl + 2 * G); }
        if (sl + 3 * G < M) { write_slot(&s.con[sl + 3 * G], c3); s.perm[sl + 3 * G] = (uint16_t)(sl + 3 * G); }
#pragma unroll 4
        for (uint32_t k = sl + kPreSlots * G; k < M; k += G) {
            write_slot(&s.con[k], read_slot(&gc[k]));
            s.perm[k] = (uint16_t)k;
        }
    };
    if (!SPLIT && live) write_contacts();
    __syncthreads();  // below, each wave syncs with itself (split groups: three barriers per substep)
    if (PL != PL_LDS) fill_alpha(tid, kWave);
    tick(PH_LOAD);

    for (uint32_t step = 0; step < a.substeps; ++step) {
        // ---- Previous-contact snapshot (cache_contacts of the last substep) -----------
        // A split group's helper takes it after the first barrier of the substep (with the
        // contact list's LDS copy in the first substep), so the solver never waits for it.
        // Taken after the broad phase (LATE_SNAP), its slots at or past the count the broad
        // phase started from (`kept`) may hold appends: a list whose count the host lowered or
        // reset before this call. The first substep reads those from the call's list in HBM,
        // as loaded (the permutation is still the identity); in later substeps the snapshot's
        // slots all lie below that count, where no append lands unless the count wraps past
        // 2^32: a substep that may wrap takes the snapshot first, into the HBM working set,
        // and copies it into place after the broad phase.
        auto snapshot = [&](uint32_t kept, float4* dpen, float4* dimp) {
            const uint32_t pn = pcount < M ? pcount : M;
            const bool from_det = step == 0 && detached;
            for (uint32_t k = sl; k < pn; k += G) {
                const bool from_list = LATE_SNAP && k >= kept;
                const ContactRec* r = from_det ? &a.prev_contacts[(size_t)env * M + k] : from_list ? &gc[k] : &s.con[s.perm[k]];
                dpen[k] = *(const float4*)r->position_pen;
                dimp[k] = make_float4(r->impulses[0], r->impulses[1], r->impulses[2],
                                      __uint_as_float(pair_key(r->indices[0], r->indices[1])));
            }
        };
        const bool snap_first = LATE_SNAP && (uint64_t)count + (uint64_t)a.G * (uint64_t)(a.G - 1u) / 2u > 0xFFFFFFFFull;
        if (!SPLIT && (!LATE_SNAP || snap_first) && live) snapshot(M, snap_first ? hppen : s.ppen, snap_first ? hpimp : s.pimp);
        // Stage B (below), one text for the two places it runs from.
        const bool take_vb = alias && step == 0;  // aliased: the velocity at call start
        auto stage_b = [&]() {
            if (bf != 0u && sl == 0) {
                s.frc[0] = make_float4(0, 0, 0, 0);
                s.trq[0] = make_float4(0, 0, 0, 0);
                s.ppos[0] = s.pos[0];
                s.pquat[0] = s.quat[0];
                if (take_vb) s.vb[0] = s.vel[0];
            }
            for (uint32_t b = bf + sl; b < B; b += G) {
                // The body's model records are read before any branch, so the reads are in
                // flight together (the model may be in HBM).
                const float4 imi = md.invmi[b], com = md.com[b];
                const uint32_t fl = md.flags[b];
                float4 P = s.pos[b], Q = s.quat[b];
                if (take_vb) s.vb[b] = s.vel[b];
                if (imi.x < 1e-8f) {
                    s.frc[b] = make_float4(0, 0, 0, 0);
                    s.trq[b] = make_float4(0, 0, 0, 0);
                } else {
                    float mass = 1.0f / imi.x;
                    f3 force = mk3(a.gx * mass, a.gy * mass, a.gz * mass);
                    s.frc[b] = tof4(force, 0.0f);
                    f3 cw = qrot(xyz(com), toq(Q));
                    s.trq[b] = tof4(cross(cw, force), 0.0f);
                }
                if (fl & 1u) {
                    P = tof4(add(xyz(P), scale(xyz(s.vel[b]), a.dt)), 0.0f);
                    const q4 q = toq(Q);
                    f3 h = scale(scale(xyz(s.angvel[b]), a.dt), 0.5f);
                    Q = tof4(qnormalize(qadd(q, qmul(mk4(h.x, h.y, h.z, 0.0f), q))));
                    s.pos[b] = P;
                    s.quat[b] = Q;
                }
                s.ppos[b] = P;
                s.pquat[b] = Q;
            }
        };
        // ---- A + B: warm_start_constraints, apply_actions (:1408-1426, :196-229), then per
        // body compute_forces and update_kinematic in dispatch order (:345-388, :304-339,
        // world.zig:962-990: the torque reads the quaternion before a kinematic body's
        // update) and save_prev_state (:1900-1913). Each lane touches only its own entries.
        if (live && do_solve) {
            for (uint32_t i = sl; i < N; i += G) s.lam[i] = 0.8f * s.lam[i];
            for (uint32_t k = sl; k < a.A; k += G) {
                const ActuatorRec& act = md.acts[k];
                const float av = k == (uint32_t)sl ? act0 : a.actions[(size_t)env * a.A + k];
                float ctrl = clampf(av, act.params[1], act.params[2]);
                float torque = clampf(ctrl * act.params[3], act.params2[0], act.params2[1]);
                s.jt[(uint32_t)act.params[0]] = torque;
            }
            if (!HBM) stage_b();
        }
        // Working sets in HBM, one environment per wave: when no joint contributes a force
        // (every |tau| < 1e-6, so stage C adds nothing), each body's forces feed its own
        // integration at once, in registers (the same operations as B then D), and the force,
        // torque and contribution arrays are neither written nor read.
        // A full list that this substep cannot wrap takes no append (see the count-only broad
        // phase), so the bodies its slots name are known before the broad phase runs. A dynamic,
        // non-kinematic body that no constraint template and no slot names is moved by nothing
        // between integration and the velocity update: with the working sets in HBM, the fused
        // integration finishes it (the update's velocities from the same operands, and the
        // last substep's accelerations), and the velocity update skips it (the lane keeps one
        // bit per body of its loop), so its previous pose is neither written nor read.
        const uint64_t max_appends = HASH ? (uint64_t)a.G * (uint64_t)(a.G - 1u) / 2u : (uint64_t)a.P;
        const uint32_t named_cap = PL == PL_ALL_HBM ? a.lds_small.ppen - a.lds_small.skey : a.lds.ppen - a.lds.skey;
        const bool frozen = HBM && live && count >= M && (uint64_t)count + max_appends <= 0xFFFFFFFFull &&
                            B <= bf + 32u * (uint32_t)G && B <= named_cap;
        uint32_t early_bits = 0;  // bit k: this lane's k-th body of the per-body loops finished early
        // One byte per body on the sort-key region (dead until the broad phase); the slots' lanes
        // store 1 for both of their bodies (equal stores, no atomics). The region is in LDS but
        // for placement 3, so a wave-level fence orders it there.
        uint8_t* const named = (uint8_t*)s.skey;
        auto mark_named = [&]() {
            const uint32_t words = (B + 3u) / 4u;
            for (uint32_t w = sl; w < words; w += G) ((uint32_t*)named)[w] = 0u;
            wave_sync<PL == PL_WORK_HBM>();
            for (uint32_t k = sl; k < M; k += G) {
                const uint32_t* idx = s.con[s.perm[k]].indices;
                named[idx[0]] = 1u;
                named[idx[1]] = 1u;
            }
            wave_sync<PL == PL_WORK_HBM>();
        };
        auto finished_early = [&](uint32_t b, float4 imi) {
            return frozen && !(imi.x < 1e-8f) && (md.flags[b] & 5u) == 0u && named[b] == 0u;
        };
        auto joint_forces_absent = [&]() {
            wave_sync<HBM>();  // the torques apply_actions wrote
            bool contrib = false;
            if (live && do_solve) {
                for (uint32_t j = sl; j < a.J; j += G) contrib = contrib || !(__builtin_fabsf(s.jt[j]) < 1e-6f);
            }
            return __ballot(contrib) == 0ull;
        };
        const bool fuse = HBM ? joint_forces_absent() : false;
        if constexpr (HBM) {
        if (frozen && fuse && do_solve) mark_named();
        if (live && do_solve && fuse) {
            const float inv_dt = 1.0f / a.dt;
            if (bf != 0u && sl == 0) {
                s.ppos[0] = s.pos[0];
                s.pquat[0] = s.quat[0];
                if (take_vb) s.vb[0] = s.vel[0];
            }
            uint32_t kb = 0;
            for (uint32_t b = bf + sl; b < B; b += G, ++kb) {
                const float4 imi = md.invmi[b];
                float4 P = s.pos[b], Q = s.quat[b];
                const float4 V = s.vel[b];
                if (take_vb) s.vb[b] = V;
                const bool dyn = !(imi.x < 1e-8f);
                f3 force = mk3(0.0f, 0.0f, 0.0f), torque = force;
                if (dyn) {
                    float mass = 1.0f / imi.x;
                    force = mk3(a.gx * mass, a.gy * mass, a.gz * mass);
                    f3 cw = qrot(xyz(md.com[b]), toq(Q));
                    torque = cross(cw, force);
                }
                if (md.flags[b] & 1u) {
                    P = tof4(add(xyz(P), scale(xyz(V), a.dt)), 0.0f);
                    const q4 q = toq(Q);
                    f3 h = scale(scale(xyz(s.angvel[b]), a.dt), 0.5f);
                    Q = tof4(qnormalize(qadd(q, qmul(mk4(h.x, h.y, h.z, 0.0f), q))));
                    s.pos[b] = P;
                    s.quat[b] = Q;
                }
                const bool early = finished_early(b, imi);
                if (!early) {
                    s.ppos[b] = P;
                    s.pquat[b] = Q;
                }
                if (!dyn) continue;
                f3 vel = add(xyz(V), scale(scale(force, imi.x), a.dt));
                vel = scale(vel, 0.999f);
                f3 pos = add(xyz(P), scale(vel, a.dt));
                s.pos[b] = tof4(pos, 0.0f);
                f3 om = add(xyz(s.angvel[b]), scale(mul(mk3(imi.y, imi.z, imi.w), torque), a.dt));
                om = scale(om, 0.999f);
                q4 q = toq(Q);
                f3 h = scale(scale(om, a.dt), 0.5f);
                q = qadd(q, qmul(mk4(h.x, h.y, h.z, 0.0f), q));
                q = qnormalize(q);
                s.quat[b] = tof4(q);
                if (!early) {
                    s.vel[b] = tof4(vel, 0.0f);
                    s.angvel[b] = tof4(om, 0.0f);
                    continue;
                }
                // The velocity update's values (pose now minus previous pose), from registers.
                early_bits |= 1u << kb;
                const float4 v = tof4(scale(sub(pos, xyz(P)), inv_dt), 0.0f);
                s.vel[b] = v;
                q4 dq = qmul(toq(tof4(q)), qconj(toq(Q)));
                if (dq.w < 0) dq = qneg(dq);
                s.angvel[b] = tof4(scale(sscale(2.0f, xyz(dq)), inv_dt), 0.0f);
                if (j_acc && step + 1 == a.substeps) {
                    const float4 v0 = take_vb ? V : s.vb[b];
                    a.acc[(size_t)env * B + b] = make_float4((v.x - v0.x) * a.inv_step, (v.y - v0.y) * a.inv_step, (v.z - v0.z) * a.inv_step, 0.0f);
                }
            }
        }
        if (live && do_solve && !fuse) stage_b();
        }
        wave_sync<HBM>();
        // ---- C: apply_joint_forces (S2, :122-190) -------------------------------------
        // Each joint's world-frame contribution axis_world * tau is formed by one lane into
        // jw (skipped when |tau| < 1e-6, flag w = 0); then each body sums the contributions
        // of its joints in ascending joint order (build_body_joint_lists), and integrates.
        if (live && do_solve && !fuse) {
            for (uint32_t j = sl; j < a.J; j += G) {
                const JointRec& jr = md.joints[j];
                const float tau = s.jt[j];
                float4 c = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (!(__builtin_fabsf(tau) < 1e-6f)) {
                    const uint32_t ja = (uint32_t)jr.params[1];
                    c = tof4(scale(qrot(mk3(jr.axis[0], jr.axis[1], jr.axis[2]), toq(s.quat[ja])), tau), 1.0f);
                }
                s.jw[j] = c;
            }
        }
        wave_sync<HBM>();
        // ---- D: integrate (:394-462), on the lane that formed the body's forces -----------
        if (live && do_solve && !fuse) {
            for (uint32_t b = bf + sl; b < B; b += G) {
                const float4 imi = md.invmi[b];
                const uint32_t e0 = md.bjoff[b], e1 = md.bjoff[b + 1];
                if (imi.x < 1e-8f) {
                    if (SPLIT) { s.frc[b] = s.pos[b]; s.trq[b] = s.quat[b]; }  // the helper's pose copy
                    continue;
                }
                float4 f = s.frc[b], t = s.trq[b];
                // The body's list entries and contributions are read four at a time (one LDS
                // round trip each), then summed in list order.
                for (uint32_t e = e0; e < e1; e += 4) {
                    uint32_t ent[4];
                    float4 c[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) ent[i] = e + i < e1 ? md.bjl[e + i] : 0u;
#pragma unroll
                    for (int i = 0; i < 4; ++i) c[i] = e + i < e1 ? s.jw[ent[i] & 0x3FFFFFFFu] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (c[i].w == 0.0f) continue;  // no contribution (or past the list's end)
                        const f3 d = (ent[i] & (1u << 30)) ? neg(xyz(c[i])) : xyz(c[i]);
                        if (ent[i] & (1u << 31)) { f.x = f.x + d.x; f.y = f.y + d.y; f.z = f.z + d.z; }
                        else { t.x = t.x + d.x; t.y = t.y + d.y; t.z = t.z + d.z; }
                    }
                }
                f3 vel = add(xyz(s.vel[b]), scale(scale(xyz(f), imi.x), a.dt));
                vel = scale(vel, 0.999f);
                f3 pos = add(xyz(s.pos[b]), scale(vel, a.dt));
                s.vel[b] = tof4(vel, 0.0f);
                s.pos[b] = tof4(pos, 0.0f);
                f3 om = add(xyz(s.angvel[b]), scale(mul(mk3(imi.y, imi.z, imi.w), xyz(t)), a.dt));
                om = scale(om, 0.999f);
                q4 q = toq(s.quat[b]);
                f3 h = scale(scale(om, a.dt), 0.5f);
                q = qadd(q, qmul(mk4(h.x, h.y, h.z, 0.0f), q));
                q = qnormalize(q);
                s.angvel[b] = tof4(om, 0.0f);
                s.quat[b] = tof4(q);
                if (SPLIT) { s.frc[b] = tof4(pos, 0.0f); s.trq[b] = tof4(q); }  // the helper's pose copy
            }
        }
        wave_sync<HBM>();
        tick(PH_FORCES);
        if (SPLIT) {
            __syncthreads();  // split barrier 1: poses after integration are in place
            if (live && helper) {
                if (step == 0) {
                    count = a.counts[env];
                    pcount = a.pcounts[env];
                    detached = a.prev_detached != nullptr && a.prev_detached[env] != 0;
#pragma unroll 4
                    for (uint32_t k = sl; k < M; k += G) {
                        write_slot(&s.con[k], read_slot(&gc[k]));
                        s.perm[k] = (uint16_t)k;
                    }
                }
                snapshot(M, s.ppen, s.pimp);
            }
        }
        // ---- E: broad_phase (S1), :468-533, or the spatial hash, :556-703 -------------
        // Broad phase to contact levels: the helper's part of a split group, on the poses
        // after integration (the force and torque arrays hold them; the level masks overwrite
        // them after the narrow phase).
        if (do_prep) {
        Lds sp = s;
        if (SPLIT) { sp.pos = s.frc; sp.quat = s.trq; }
        Lds& s = sp;
        const uint32_t count_before = count;
        if (HASH) {
            uint32_t* const hmeta = (uint32_t*)(s.hpos + a.G);
            // Cells (broad_phase_count_cells, :556-584), sort keys and each geom's staged
            // centre, radius and compact word. Up to 1024 keys are sorted in registers, which
            // pad the list themselves, so only the G real keys are stored; a longer list is
            // padded to Gp in LDS (padding keys sort last).
            const uint32_t nkeys = a.Gp <= 1024u ? a.G : a.Gp;
            if (live) {
                for (uint32_t g = sl; g < nkeys; g += G) {
                    uint32_t key = 0xFFFFFFFFu;
                    if (g < a.G) {
                        const GeomRec& gr = md.geoms[g];
                        const f3 p = add(xyz(s.pos[gr.type_body[1]]), mk3(gr.pos_size0[0], gr.pos_size0[1], gr.pos_size0[2]));
                        const uint32_t id = hash_axis(p.x) + hash_axis(p.y) * 64u + hash_axis(p.z) * 4096u;
                        if (HBM) {
                            s.hpos[g] = tof4(p, gr.pos_size0[3]);
                            hmeta[g] = md.hmeta[g];
                        }
                        a.cell_ids[(size_t)env * a.G + g] = id;
                        key = (id << 14) | g;
                    }
                    s.hkey[g] = key;
                }
            }
            wave_sync<HBM>();
            // Bitonic sort of the keys: up to 1024 in registers (sixteen per lane), more in
            // LDS, one compare-exchange pair per lane and pass.
            if (a.Gp <= 1024u) {
                if (live) sort_keys_1024(s.hkey, a.G, (uint32_t)sl);
                wave_sync<HBM>();
            } else
            for (uint32_t k = 2; k <= a.Gp; k <<= 1) {
                for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                    if (live) {
                        for (uint32_t t = sl; t < a.Gp / 2; t += G) {
                            const uint32_t i = ((t & ~(j - 1u)) << 1) | (t & (j - 1u));
                            const uint32_t l = i | j;
                            const uint32_t x = s.hkey[i], y = s.hkey[l];
                            if ((x > y) == ((i & k) == 0)) { s.hkey[i] = y; s.hkey[l] = x; }
                        }
                    }
                    wave_sync<HBM>();
                }
            }
            // Queries (broad_phase_detect, :632-700): count each geom's pairs, place them
            // with a prefix sum over the env's lanes, then write them. A full list whose
            // count cannot wrap past 2^32 this substep (at most G (G - 1) / 2 pairs) takes
            // no append, so only the number of pairs is needed.
            const uint64_t max_pairs = (uint64_t)a.G * (uint64_t)(a.G - 1u) / 2u;
            if (live && count >= M && (uint64_t)count + max_pairs <= 0xFFFFFFFFull) {
                count += hash_count_forward<HBM>(a, md, s, hmeta, sl);
            } else
            for (uint32_t base = 0; base < a.G; base += G) {
                const uint32_t g = base + sl;
                const bool mine = live && g < a.G;
                const uint32_t h = mine ? hash_pairs_of<HBM>(a, md, s, hmeta, g, false, 0) : 0u;
                uint32_t inc = h;
                for (uint32_t d = 1; d < (uint32_t)G; d <<= 1) {
                    const uint32_t t = __shfl_up(inc, d, G);
                    if ((uint32_t)sl >= d) inc += t;
                }
                const uint32_t total = __shfl(inc, G - 1, G);
                // The geom's pairs take slots start .. start + h - 1 in u32 arithmetic: some land
                // below M if the first does, or if they wrap the count past 2^32 (then from 0).
                const uint32_t start = count + (inc - h);
                if (mine && h > 0 && (start < M || (uint64_t)start + h > 0xFFFFFFFFull))
                    hash_pairs_of<HBM>(a, md, s, hmeta, g, true, start);
                count += total;
            }
            if (LATE_SNAP) {  // the hash's arrays are dead: the snapshot takes their place
                wave_sync<HBM>();
                if (live && snap_first) {
                    for (uint32_t k = sl; k < (pcount < M ? pcount : M); k += G) { s.ppen[k] = hppen[k]; s.pimp[k] = hpimp[k]; }
                } else if (live) {
                    snapshot(count_before, s.ppen, s.pimp);
                }
            }
        } else if (EPW == 1 && live && a.sweep_n != 0u && count >= M && count <= 0xFFFFFFFFu - a.P) {
            // Count-only sweep. The list is full (count >= M) and this substep cannot wrap
            // the count past 2^32 (at most P appends), so no append lands below M: the broad
            // phase only advances the count by the listed pairs that pass (:468-533). Pairs
            // with a plane always pass (no distance test), so their number is a model constant
            // (sweep_planes). The other geoms, at most 64 (sweep), sit one per lane; after k
            // one-lane rotations of the wave each lane holds the geom k lanes along, so
            // k = 1..32 meets every unordered pair once (k = 32 from the lower half only). Each
            // pair takes the list's filters (different bodies, contype / conaffinity; the list
            // holds exactly the pairs passing them, model.cpp) and the same distance test: the
            // difference's sign does not change its square, nor the radii's order their sum.
            const bool mine = (uint32_t)sl < a.sweep_n;
            f3 c = mk3(0.0f, 0.0f, 0.0f);
            float r = 0.0f;
            uint32_t body = 0, grp = 0, msk = 0;  // an empty lane passes no mask test
            if (mine) {
                const GeomRec& gr = md.geoms[a.sweep[sl]];
                c = add(xyz(s.pos[gr.type_body[1]]), mk3(gr.pos_size0[0], gr.pos_size0[1], gr.pos_size0[2]));
                r = gr.pos_size0[3];
                body = gr.type_body[1]; grp = gr.type_body[3]; msk = gr.type_body[2];
            }
            auto rol = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x134, 0xF, 0xF, false); };  // wave_rol:1
            auto rolf = [&](float v) { return __int_as_float((int)rol((uint32_t)__float_as_int(v))); };
            float px = c.x, py = c.y, pz = c.z, pr = r;
            uint32_t pb = body, pg = grp, pm = msk, hits = 0;
#pragma unroll 4
            for (uint32_t k = 1; k <= 32u; ++k) {
                px = rolf(px); py = rolf(py); pz = rolf(pz); pr = rolf(pr);
                pb = rol(pb); pg = rol(pg); pm = rol(pm);
                const f3 diff = sub(mk3(px, py, pz), c);
                const float min_dist = r + pr + 0.1f;
                const bool near = !(dot(diff, diff) >= min_dist * min_dist);  // NaN distances pass, as in :521
                const bool listed = body != pb && ((grp & pm) != 0u || (pg & msk) != 0u);
                const bool once = k < 32u || (uint32_t)sl < 32u;
                hits += (near && listed && once) ? 1u : 0u;
            }
            for (uint32_t d = 1; d < 64u; d <<= 1) hits += (uint32_t)__shfl_xor((int)hits, (int)d);
            count += a.sweep_planes + hits;
        } else {
            const uint64_t group_mask = (G == 64) ? ~0ull : (((1ull << (G % 64)) - 1ull) << (le * G));
            const uint64_t below = (sl == 0) ? 0ull : ((~0ull) >> (64 - sl)) << (le * G);
            // With the model records in HBM the geoms come from their LDS copy (s.gst /
            // s.gmeta) and the loop is software-pipelined over chunks of G pairs: while chunk
            // k is tested, the pair list of chunk k + 2 (HBM) and the staged geoms of chunk
            // k + 1 (LDS) are loaded, so a chunk starts with only body positions to read.
            constexpr bool GSTAGE = PL != PL_LDS;
            auto pair_at = [&](uint32_t p) -> uint32_t { return (live && p < a.P) ? md.pairs[p] : 0u; };
            uint32_t pr1 = 0, pr2 = 0, m1a = 0, m1b = 0;
            float4 c1a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c1b = c1a;
            if (GSTAGE && a.P > 0) {
                pr1 = pair_at(sl);
                pr2 = pair_at(sl + G);
                m1a = s.gmeta[pr1 & 0xFFFFu]; m1b = s.gmeta[pr1 >> 16];
                c1a = s.gst[pr1 & 0xFFFFu]; c1b = s.gst[pr1 >> 16];
            }
            for (uint32_t base = 0; base < a.P; base += G) {
                const uint32_t p = base + sl;
                uint32_t pr = 0, m0a = 0, m0b = 0;
                float4 c0a = c1a, c0b = c1b;
                if (GSTAGE) {
                    pr = pr1; m0a = m1a; m0b = m1b;
                    pr1 = pr2;
                    pr2 = pair_at(p + 2 * G);
                    m1a = s.gmeta[pr1 & 0xFFFFu]; m1b = s.gmeta[pr1 >> 16];
                    c1a = s.gst[pr1 & 0xFFFFu]; c1b = s.gst[pr1 >> 16];
                }
                bool hit = false;
                uint32_t g = 0, h = 0, ba = 0, bb = 0;
                if (live && p < a.P) {
                    float4 ca, cb;
                    uint32_t ta, tb;
                    if (GSTAGE) {
                        g = pr & 0xFFFFu;
                        h = pr >> 16;
                        ca = c0a;
                        cb = c0b;
                        ba = m0a & 0xFFFFu; ta = m0a >> 16;
                        bb = m0b & 0xFFFFu; tb = m0b >> 16;
                    } else {
                        pr = md.pairs[p];
                        g = pr & 0xFFFFu;
                        h = pr >> 16;
                        const GeomRec& ga = md.geoms[g];
                        const GeomRec& gb = md.geoms[h];
                        ba = ga.type_body[1]; ta = ga.type_body[0];
                        bb = gb.type_body[1]; tb = gb.type_body[0];
                        ca = *(const float4*)ga.pos_size0;
                        cb = *(const float4*)gb.pos_size0;
                    }
                    if (ta == GEOM_PLANE || tb == GEOM_PLANE) {
                        hit = true;
                    } else {
                        f3 pa = add(xyz(s.pos[ba]), mk3(ca.x, ca.y, ca.z));
                        f3 pb = add(xyz(s.pos[bb]), mk3(cb.x, cb.y, cb.z));
                        f3 diff = sub(pb, pa);
                        float min_dist = ca.w + cb.w + 0.1f;
                        hit = !(dot(diff, diff) >= min_dist * min_dist);  // NaN distances pass, as in :521
                    }
                }
                const uint64_t ballot = __ballot(hit);
                const uint32_t rank = (uint32_t)__popcll(ballot & below);
                const uint32_t total = (uint32_t)__popcll(ballot & group_mask);
                if (hit) {
                    const uint32_t slot = count + rank;
                    if (slot < M) {
                        uint32_t* idx = s.con[s.perm[slot]].indices;
                        idx[0] = ba; idx[1] = bb; idx[2] = g; idx[3] = h;
                    }
                }
                count += total;
            }
        }
        wave_sync<HBM>();
        // ---- E.5: sort_contacts (:711-745), stable rank sort over the permutation ------
        // Up to kMaxRecsPerLane slots per lane: each slot's rank (keys below it, plus equal
        // keys at lower slots) is counted in registers. Longer lists: a bitonic network over
        // (key, logical slot) pairs, keys on s.skey and slots on s.order padded to a power of
        // two; the slot breaks ties between equal keys, so the order is the stable one.
        {
            const uint32_t n = count < M ? count : M;
            // The reference sorts the first min(count, M) slots every substep; a list the last
            // sort left in order changes only when this step's appends (slots count_before ..
            // count - 1, in u32 arithmetic) took a slot below M: from below M, or by wrapping
            // past 2^32 (the count is never cleared), after which the appends restart at slot 0.
            // A count the host has set since the last step may expose slots that sort never
            // covered, so the first substep after it sorts unconditionally.
            const bool wrote = (a.sort_all != 0u && step == 0) ||
                               (count != count_before && (count_before < M || count < count_before));
            const bool need = live && wrote && n > 1;
            const bool big = __ballot(need && n > (uint32_t)(kMaxRecsPerLane * G)) != 0ull;
            if (!big) {
                if (need) {
                    for (uint32_t k = sl; k < n; k += G) {
                        const uint32_t* idx = s.con[s.perm[k]].indices;
                        s.skey[k] = pair_key(idx[0], idx[1]);
                    }
                }
                wave_sync<HBM>();
                uint16_t keep[kMaxRecsPerLane];
                uint32_t dst[kMaxRecsPerLane];
                if (need) {
#pragma unroll
                    for (int r = 0; r < kMaxRecsPerLane; ++r) {
                        const uint32_t k = sl + r * G;
                        if (k < n) {
                            const uint32_t key = s.skey[k];
                            uint32_t rank = 0;
                            for (uint32_t j = 0; j < n; ++j) {
                                const uint32_t kj = s.skey[j];
                                rank += (kj < key || (kj == key && j < k)) ? 1u : 0u;
                            }
                            keep[r] = s.perm[k];
                            dst[r] = rank;
                        }
                    }
                }
                wave_sync<HBM>();
                if (need) {
#pragma unroll
                    for (int r = 0; r < kMaxRecsPerLane; ++r) {
                        const uint32_t k = sl + r * G;
                        if (k < n) s.perm[dst[r]] = keep[r];
                    }
                }
            } else {
                // One environment per wave here (the long lists need EPW 1 or 2 to fit LDS);
                // the network runs to the wave's largest padded length.
                uint32_t np = 1;
                while (np < n) np <<= 1;
                uint32_t wave_np = need ? np : 1u;
                for (uint32_t d = 1; d < 64u; d <<= 1) {
                    const uint32_t t = __shfl_xor(wave_np, d);
                    wave_np = t > wave_np ? t : wave_np;
                }
                if (need) {
                    for (uint32_t k = sl; k < np; k += G) {
                        uint32_t key = 0xFFFFFFFFu;
                        if (k < n) {
                            const uint32_t* idx = s.con[s.perm[k]].indices;
                            key = pair_key(idx[0], idx[1]);
                        }
                        s.skey[k] = key;
                        s.order[k] = (uint16_t)k;
                    }
                }
                wave_sync<HBM>();
                for (uint32_t kk = 2; kk <= wave_np; kk <<= 1) {
                    for (uint32_t j = kk >> 1; j > 0; j >>= 1) {
                        if (need && kk <= np) {
                            for (uint32_t t = sl; t < np / 2; t += G) {
                                const uint32_t i = ((t & ~(j - 1u)) << 1) | (t & (j - 1u));
                                const uint32_t l = i | j;
                                const uint32_t xa = s.skey[i], xb = s.skey[l];
                                const uint32_t ia = s.order[i], ib = s.order[l];
                                const bool gt = xa > xb || (xa == xb && ia > ib);
                                if (gt == ((i & kk) == 0)) {
                                    s.skey[i] = xb; s.skey[l] = xa;
                                    s.order[i] = (uint16_t)ib; s.order[l] = (uint16_t)ia;
                                }
                            }
                        }
                        wave_sync<HBM>();
                    }
                }
                // order[k] = logical slot now at position k -> its physical slot, then perm.
                if (need) {
                    for (uint32_t k = sl; k < n; k += G) s.order[k] = s.perm[s.order[k]];
                }
                wave_sync<HBM>();
                if (need) {
                    for (uint32_t k = sl; k < n; k += G) s.perm[k] = s.order[k];
                }
            }
        }
        wave_sync<HBM>();
        tick(PH_BROAD);
        // ---- F: narrow_phase (:751-894) -----------------------------------------------
        const uint32_t n_live = count < M ? count : M;
        if (GROUP && a.ext_contacts && M >= 64) {
            // Extended mode: each slot's pair type picks one of detectCollision's branches,
            // and a wave runs every branch that its lanes need. The slots are visited grouped
            // by (type a, type b): a counting sort over the 64 ordered type pairs into s.order
            // (dead until the levels), with the class counters on s.skey (dead after the
            // sort). Each slot's result depends on that slot alone, so the visiting order
            // changes no result.
            uint32_t* ccount = s.skey;
            auto geom_type = [&](uint32_t g) -> uint32_t {
                if (PL != PL_LDS && !HASH) return s.gmeta[g] >> 16;
                return md.geoms[g].type_body[0];
            };
            auto slot_class = [&](uint32_t phys) -> uint32_t {
                const uint32_t* idx = s.con[phys].indices;
                return (geom_type(idx[2]) & 7u) * 8u + (geom_type(idx[3]) & 7u);
            };
            constexpr uint32_t kPer = 64u / G;  // classes per lane
            for (uint32_t i = 0; i < kPer; ++i) ccount[sl * kPer + i] = 0u;
            wave_sync<HBM>();
            if (live) {
                for (uint32_t k = sl; k < n_live; k += G) atomicAdd(&ccount[slot_class(s.perm[k])], 1u);
            }
            wave_sync<HBM>();
            // Exclusive scan of the env's 64 counters: each lane sums its kPer classes, the
            // env's G lanes scan those sums, and each lane writes its classes' offsets.
            uint32_t sum = 0;
            for (uint32_t i = 0; i < kPer; ++i) sum += ccount[sl * kPer + i];
            uint32_t incl = sum;
            for (int d = 1; d < G; d <<= 1) {
                const uint32_t t = __shfl_up(incl, d, G);
                if (sl >= d) incl += t;
            }
            uint32_t run = incl - sum;
            for (uint32_t i = 0; i < kPer; ++i) {
                const uint32_t c = ccount[sl * kPer + i];
                ccount[sl * kPer + i] = run;
                run += c;
            }
            wave_sync<HBM>();
            if (live) {
                for (uint32_t k = sl; k < n_live; k += G) {
                    const uint32_t phys = s.perm[k];
                    s.order[atomicAdd(&ccount[slot_class(phys)], 1u)] = (uint16_t)phys;
                }
            }
            wave_sync<HBM>();
            if (live) {
                for (uint32_t k = sl; k < n_live; k += G) narrow_slot<PL != PL_LDS>(a, md, s, &s.con[s.order[k]]);
            }
        } else if (live) {
            for (uint32_t k = sl; k < n_live; k += G) narrow_slot<PL != PL_LDS>(a, md, s, &s.con[s.perm[k]]);
        }
        wave_sync<HBM>();
        // ---- G: match_cached_contacts (:1483-1544) ------------------------------------
        // The snapshot is key-sorted (it is a sorted list from the last substep), so the
        // entries with this slot's body pair form one run; the match is the run's first
        // entry at the smallest squared distance below 0.04 (the reference's first strict
        // minimum in index order). Each snapshot entry's run start comes from a segmented
        // max-scan over the sorted keys (on the sort-key region, free from here to the
        // levels). Once the list has stopped growing, snapshot entry k holds the same pair as
        // slot k and the slot's run starts at entry k's; otherwise the run's first entry is
        // found by binary search. The run is read four entries per LDS round trip.
        const uint32_t pn = pcount < M ? pcount : M;
        auto key_at = [&](uint32_t i) { return __float_as_uint(s.pimp[i].w); };
        uint32_t* const rstart = s.skey;
        if (live) {
            uint32_t carry = 0;
            for (uint32_t base = 0; base < pn; base += G) {
                const uint32_t i = base + sl;
                uint32_t v = 0;
                if (i < pn && i > 0 && key_at(i - 1) != key_at(i)) v = i;
                v = seg_max_scan<G>(v, sl);
                v = carry > v ? carry : v;
                if (i < pn) rstart[i] = v;
                carry = __shfl(v, G - 1, G);
            }
        }
        wave_sync<HBM>();
        if (live) {
            for (uint32_t k = sl; k < n_live; k += G) {
                ContactRec* c = &s.con[s.perm[k]];
                if (c->position_pen[3] < 0) continue;
                const uint32_t key = pair_key(c->indices[0], c->indices[1]);
                uint32_t lo;
                if (k < pn && key_at(k) == key) {
                    lo = rstart[k];
                } else {
                    uint32_t hi = pn;
                    lo = 0;
                    while (lo < hi) {
                        uint32_t mid = (lo + hi) >> 1;
                        if (key_at(mid) < key) lo = mid + 1; else hi = mid;
                    }
                }
                const f3 p = mk3(c->position_pen[0], c->position_pen[1], c->position_pen[2]);
                float best = 0.04f;
                int best_i = -1;
                // The run ends at the first entry with another key (the list is sorted).
                bool more = true;
                auto visit = [&](uint32_t j, uint32_t kj, float4 q) {
                    if (!(more && j < pn && kj == key)) { more = false; return; }
                    if (q.w < 0) return;
                    const f3 d = sub(mk3(q.x, q.y, q.z), p);
                    const float dsq = dot(d, d);
                    if (dsq < best) { best = dsq; best_i = (int)j; }
                };
                for (uint32_t i = lo; more && i < pn; i += 4) {
                    const uint32_t j1 = i + 1 < pn ? i + 1 : i, j2 = i + 2 < pn ? i + 2 : i, j3 = i + 3 < pn ? i + 3 : i;
                    const uint32_t k0 = key_at(i), k1 = key_at(j1), k2 = key_at(j2), k3 = key_at(j3);
                    const float4 q0 = s.ppen[i], q1 = s.ppen[j1], q2 = s.ppen[j2], q3 = s.ppen[j3];
                    visit(i, k0, q0);
                    visit(i + 1, k1, q1);
                    visit(i + 2, k2, q2);
                    visit(i + 3, k3, q3);
                }
                if (best_i >= 0) {
                    const float4 im = s.pimp[best_i];
                    c->impulses[0] = im.x * 0.8f;
                    c->impulses[1] = im.y * 0.8f;
                    c->impulses[2] = im.z * 0.8f;
                }
            }
        }
        // ---- Contact levels for S4 -----------------------------------------------------
        // level(slot) = 1 + max level of earlier valid slots sharing a body that the solve
        // writes (inv_m > 1e-8). Running levels in order reproduces the sequential slot
        // order exactly, and the slots of one level share no such body, so they may run in
        // any order. Valid slots (solve_contacts skips only pen < 0, :1667) are compacted in
        // slot order with a ballot, and each dynamic body gets a bit mask of the compacted
        // slots touching it. When no slot of the environment writes two bodies (contacts
        // with static geometry), a slot's level is its rank among the slots of its body: 1 +
        // the number of lower bits in that body's mask. Otherwise a slot's level is 1 + the
        // larger level of its predecessors on its two bodies (the highest lower bit of each
        // body's mask), and levels follow by relaxation, one pass per level. Each level's
        // slots are then placed by a counting sort into s.lst, level l owning
        // [s.loff[l - 1], s.loff[l]).
        wave_sync<HBM>();  // matching has read the snapshot, which the level arrays reuse
        uint32_t nv = 0;
        const uint32_t mw = (M + 63u) >> 6;                                        // mask words per body
        uint32_t* const vbod = s.vbod;  // u32[M] dynamic bodies
        uint32_t* const prv = s.prv;    // u32[M] predecessors, then the level counters
        const uint64_t group_mask = (G == 64) ? ~0ull : (((1ull << (G % 64)) - 1ull) << (le * G));
        const uint64_t below = (sl == 0) ? 0ull : ((~0ull) >> (64 - sl)) << (le * G);
        if (live) {
            for (uint32_t i = sl; i < B * mw; i += G) s.bmask[i] = 0ull;
        }
        wave_sync<HBM>();
        bool two_bodies = false;  // some valid slot of this lane writes both of its bodies
        if (live) {
            for (uint32_t base = 0; base < n_live; base += G) {
                const uint32_t k = base + sl;
                bool valid = false;
                uint32_t phys = 0;
                if (k < n_live) {
                    phys = s.perm[k];
                    valid = !(s.con[phys].position_pen[3] < 0);
                }
                const uint64_t ballot = __ballot(valid);
                if (valid) {
                    const uint32_t at = nv + (uint32_t)__popcll(ballot & below);
                    const ContactRec* c = &s.con[phys];
                    const uint32_t ia = c->indices[0], ib = c->indices[1];
                    const uint32_t A = (md.flags[ia] & 2u) ? ia : 0xFFFFu, Bd = (md.flags[ib] & 2u) ? ib : 0xFFFFu;
                    s.vlist[at] = (uint16_t)phys;
                    vbod[at] = A | (Bd << 16);
                    const unsigned long long bit = 1ull << (at & 63u);
                    if (A != 0xFFFFu) atomicOr(&s.bmask[A * mw + (at >> 6)], bit);
                    if (Bd != 0xFFFFu) atomicOr(&s.bmask[Bd * mw + (at >> 6)], bit);
                    two_bodies = two_bodies || (A != 0xFFFFu && Bd != 0xFFFFu);
                }
                nv += (uint32_t)__popcll(ballot & group_mask);
            }
        }
        const bool relax = (__ballot(two_bodies) & group_mask) != 0ull;  // per environment
        wave_sync<HBM>();
        if (live && !relax) {
            for (uint32_t i = sl; i < nv; i += G) {
                const uint32_t bo = vbod[i];
                const uint32_t body = (bo & 0xFFFFu) != 0xFFFFu ? (bo & 0xFFFFu) : (bo >> 16);
                uint32_t lv = 1;
                if (body != 0xFFFFu) {
                    const unsigned long long* m = &s.bmask[body * mw];
                    for (uint32_t w = 0; w < (i >> 6); ++w) lv += (uint32_t)__popcll(m[w]);
                    lv += (uint32_t)__popcll(m[i >> 6] & ((1ull << (i & 63u)) - 1ull));
                }
                s.order[i] = (uint16_t)lv;
            }
        }
        // Predecessor on a body: the highest set bit below slot i in the body's mask.
        auto pred = [&](uint32_t body, uint32_t i) -> uint32_t {
            if (body == 0xFFFFu) return 0xFFFFu;
            for (int w = (int)(i >> 6); w >= 0; --w) {
                unsigned long long m = s.bmask[body * mw + (uint32_t)w];
                if ((uint32_t)w == (i >> 6)) m &= (1ull << (i & 63u)) - 1ull;
                if (m) return (uint32_t)w * 64u + 63u - (uint32_t)__clzll(m);
            }
            return 0xFFFFu;
        };
        if (__ballot(live && relax) != 0ull) {
            if (live && relax) {
                for (uint32_t i = sl; i < nv; i += G) {
                    const uint32_t bo = vbod[i];
                    prv[i] = pred(bo & 0xFFFFu, i) | (pred(bo >> 16, i) << 16);
                    s.order[i] = 1;
                }
            }
            wave_sync<HBM>();
            for (;;) {
                bool changed = false;
                if (live && relax) {
                    for (uint32_t i = sl; i < nv; i += G) {
                        const uint32_t pr = prv[i], pa = pr & 0xFFFFu, pb = pr >> 16;
                        const uint32_t la = pa != 0xFFFFu ? s.order[pa] : 0u;
                        const uint32_t lb = pb != 0xFFFFu ? s.order[pb] : 0u;
                        const uint32_t lv = (la > lb ? la : lb) + 1u;
                        if (lv != s.order[i]) { s.order[i] = (uint16_t)lv; changed = true; }
                    }
                }
                wave_sync<HBM>();
                if (__ballot(changed) == 0ull) break;
            }
        }
        wave_sync<HBM>();
        {
            uint32_t nlev = 0;
            if (live) {
                for (uint32_t i = sl; i < nv; i += G) nlev = s.order[i] > nlev ? s.order[i] : nlev;
            }
            for (uint32_t d = 1; d < (uint32_t)G; d <<= 1) {
                const uint32_t t = __shfl_xor(nlev, d, G);
                nlev = t > nlev ? t : nlev;
            }
            uint32_t wave_nlev = nlev;  // the scan below runs to the largest count of the wave
            for (uint32_t d = G; d < 64u; d <<= 1) {
                const uint32_t t = __shfl_xor(wave_nlev, d);
                wave_nlev = t > wave_nlev ? t : wave_nlev;
            }
            // Counting sort by level: per-level counts, their running sum (s.loff), then each
            // slot takes the next place of its level.
            uint32_t* const cnt = prv;  // u32[nlev]: entry l - 1 for level l (prv is dead now)
            if (live) {
                for (uint32_t l = sl; l < nlev; l += G) cnt[l] = 0u;
            }
            wave_sync<HBM>();
            if (live) {
                for (uint32_t i = sl; i < nv; i += G) atomicAdd(&cnt[s.order[i] - 1u], 1u);
            }
            wave_sync<HBM>();
            uint32_t run = 0;
            for (uint32_t l0 = 1; l0 <= wave_nlev; l0 += G) {
                const uint32_t l = l0 + sl;
                const bool mine = live && l <= nlev;
                const uint32_t v = mine ? cnt[l - 1u] : 0u;
                uint32_t incl = v;
                for (uint32_t d = 1; d < (uint32_t)G; d <<= 1) {
                    const uint32_t t = __shfl_up(incl, d, G);
                    if ((uint32_t)sl >= d) incl += t;
                }
                if (mine) {
                    s.loff[l] = (uint16_t)(run + incl);
                    cnt[l - 1u] = run + incl - v;  // the level's first place
                }
                run += __shfl(incl, G - 1, G);
            }
            if (live && sl == 0) {
                s.loff[0] = 0;
                s.misc[2] = nlev;
            }
            wave_sync<HBM>();
            if (live) {
                for (uint32_t i = sl; i < nv; i += G) s.lst[atomicAdd(&cnt[s.order[i] - 1u], 1u)] = s.vlist[i];
            }
        }
        // Per-slot constants of the contact solve (the same in every iteration): the bias
        // velocity, the two position-correction shares and the summed inverse mass, kept in
        // the snapshot's impulse array, which is dead once matching is done.
        if (live) {
            for (uint32_t i = sl; i < nv; i += G) {
                const uint32_t phys = s.vlist[i];
                const ContactRec* c = &s.con[phys];
                const float inv_mass_a = md.invmi[c->indices[0]].x, inv_mass_b = md.invmi[c->indices[1]].x;
                const float inv_mass_sum = inv_mass_a + inv_mass_b;
                const float pos_correction = a.baumgarte * fmaxf(c->position_pen[3] - a.slop, 0.0f);
                const float bias = pos_correction / a.dt;
                s.pimp[phys] = make_float4(bias, pos_correction * (inv_mass_a / inv_mass_sum),
                                           pos_correction * (inv_mass_b / inv_mass_sum), inv_mass_sum);
            }
        }
        wave_sync<HBM>();
        }  // do_prep
        tick(PH_NARROW);
        // ---- H: solve_joints, iterations x colours (world.zig:1163-1195, S3) ----------
        // Phases are same-type runs inside a colour (build_joint_program); the type is
        // uniform, so each phase takes one scalar branch. Lane pair (2k, 2k+1) of the env's
        // lanes takes constraint k. The phase loop is software-pipelined: descriptors and
        // solve records are read-only, so while phase t runs, the descriptor of phase t + 2
        // and the lane's first solve record of phase t + 1 are loaded; a phase then starts
        // with only its bodies' state to read.
        if (do_solve) {
            const uint32_t nph = a.iters * a.njph;
            const uint32_t kf = (uint32_t)sl >> 1;
            const bool odd = (sl & 1) != 0;
            const uint32_t half = odd ? kJHalfQuads : 0u;
            JointPhase ph = md.jph[0], ph1 = md.jph[a.njph > 1 ? 1u : 0u];
            uint32_t p2 = a.njph > 2 ? 2u : 0u;
            JHalf rec;
            {
                const uint32_t st = __builtin_amdgcn_readfirstlane(ph.start), cn = __builtin_amdgcn_readfirstlane(ph.count);
                rec = load_half(md.jrec + (st + (kf < cn ? kf : 0u)) * kJRecQuads + half);
            }
            // One phase: solves with `cur` (this lane's first record of the phase) while the
            // next phase's record is loaded into `nxt`. The loop runs two phases per trip with
            // the two record buffers swapping roles, so no record is copied between phases.
            auto phase = [&](const JHalf& cur, JHalf& nxt) {
                const uint32_t type = __builtin_amdgcn_readfirstlane(ph.type);
                const uint32_t start = __builtin_amdgcn_readfirstlane(ph.start);
                const uint32_t cnt = __builtin_amdgcn_readfirstlane(ph.count);
                const JointPhase ph2 = md.jph[p2];
                {
                    const uint32_t st = __builtin_amdgcn_readfirstlane(ph1.start), cn = __builtin_amdgcn_readfirstlane(ph1.count);
                    nxt = load_half(md.jrec + (st + (kf < cn ? kf : 0u)) * kJRecQuads + half);
                }
                if (live && kf < cnt) solve_joint(type, cur, load_jstate(cur, s, odd), md.jrec + (start + kf) * kJRecQuads, s, odd);
                if (live) {
                    for (uint32_t k = kf + G / 2; k < cnt; k += G / 2) {
                        const float4* r = md.jrec + (start + k) * kJRecQuads;
                        const JHalf hk = load_half(r + half);
                        solve_joint(type, hk, load_jstate(hk, s, odd), r, s, odd);
                    }
                }
                wave_sync<HBM>();
                ph = ph1;
                ph1 = ph2;
                p2 = p2 + 1 == a.njph ? 0u : p2 + 1;
            };
            JHalf rec2;
            uint32_t t = 0;
            for (; t + 2 <= nph; t += 2) {
                phase(rec, rec2);
                phase(rec2, rec);
            }
            if (t < nph) phase(rec, rec2);
        }
        tick(PH_JOINTS);
        if (SPLIT) __syncthreads();  // split barrier 2: the contact levels are in place
        uint32_t max_lev = 0;
        for (int e2 = 0; e2 < EPW; ++e2) {
            const uint32_t* m2 = HBM ? s.misc : (const uint32_t*)(env_base + e2 * a.lds.bytes + a.lds.misc);
            if (wave_id * EPW + e2 < a.E && m2[2] > max_lev) max_lev = m2[2];
        }
        const uint32_t my_nlev = live ? s.misc[2] : 0u;
        // ---- I: solve_contacts, iterations x levels (world.zig:1199-1213, S4) --------
        // Lane pair (2k, 2k+1) takes the k-th slot of each level (and k + G/2, ... when a
        // level holds more). The level lists and the slots' static parts are read ahead over
        // the sequence of (iteration, level) steps: at step f the lane's slot record of step
        // f + 1, its slot index of step f + 2 and the level bounds of step f + 3 are loaded,
        // so a step starts with its record in registers and reads only the bodies' state.
        if (do_solve && max_lev > 0) {
            const bool odd = (sl & 1) != 0;
            const uint32_t kf = (uint32_t)sl >> 1;
            const uint32_t nsteps = a.iters * max_lev;
            // Level bounds of step f: the level's first slot index and its end, read raw (the
            // lane's slot is first + kf); `ok` when the step exists for the lane's env. The
            // comparison with the end happens a step later, once the read has landed.
            auto bounds = [&](uint32_t f, uint32_t lv, uint32_t& first, uint32_t& end) -> bool {
                first = s.loff[lv - 1];
                end = s.loff[lv];
                return f < nsteps && live && lv <= my_nlev;
            };
            auto next_lv = [&](uint32_t lv) -> uint32_t { return lv == max_lev ? 1u : lv + 1u; };
            uint32_t j0, e0, j1, e1, j2, e2;
            uint32_t lv3 = 1;
            bool v0 = bounds(0, lv3, j0, e0);
            lv3 = next_lv(lv3);
            bool v1 = bounds(1, lv3, j1, e1);
            lv3 = next_lv(lv3);
            bool v2 = bounds(2, lv3, j2, e2);
            lv3 = next_lv(lv3);
            j0 += kf; v0 = v0 && j0 < e0;
            j1 += kf; v1 = v1 && j1 < e1;
            CRec cA = load_crec(s, v0 ? s.lst[j0] : 0u), cB;
            bool cv = v0;
            uint32_t ce = e0, cj = j0;
            uint32_t p1 = v1 ? s.lst[j1] : 0u;
            // One step with `cur` while the next step's record is loaded into `nxt`; two
            // steps per trip with the record buffers swapping roles (no record copies).
            auto cstep = [&](uint32_t f, const CRec& cur, CRec& nxt) {
                uint32_t j3, e3;
                const bool ok3 = bounds(f + 3, lv3, j3, e3);
                lv3 = next_lv(lv3);
                j2 += kf;
                v2 = v2 && j2 < e2;
                const uint32_t p2 = v2 ? s.lst[j2] : 0u;
                nxt = load_crec(s, p1);
                if (cv) {
                    solve_contact_rec(md, s, cur, odd);
                    for (uint32_t j = cj + G / 2; j < ce; j += G / 2) solve_contact2(md, s, s.lst[j], odd);
                }
                wave_sync<HBM>();
                cv = v1; ce = e1; cj = j1;
                p1 = p2; v1 = v2; e1 = e2; j1 = j2;
                v2 = ok3; e2 = e3; j2 = j3;
            };
            uint32_t f = 0;
            for (; f + 2 <= nsteps; f += 2) {
                cstep(f, cA, cB);
                cstep(f + 1, cB, cA);
            }
            if (f < nsteps) cstep(f, cA, cB);
        }
        tick(PH_CONTACTS);
        if (SPLIT) __syncthreads();  // split barrier 3: the contact list is final for this substep
        // ---- J: xpbd_update_velocities (:1922-1961) ----------------------------------
        if (live && do_solve) {
            const float inv_dt = 1.0f / a.dt;
            const bool acc_here = j_acc && step + 1 == a.substeps;
            uint32_t kb = 0;
            for (uint32_t b = bf + sl; b < B; b += G, ++kb) {
                if (HBM && ((early_bits >> kb) & 1u) != 0u) continue;
                const float imass = md.invmi[b].x;
                // Poses in LDS are read beside the model record (both in flight together); in
                // HBM only for the bodies that move.
                float4 P, PP, Q, PQ;
                if constexpr (!HBM) { P = s.pos[b]; PP = s.ppos[b]; Q = s.quat[b]; PQ = s.pquat[b]; }
                if (imass < 1e-8f) continue;
                if constexpr (HBM) { P = s.pos[b]; PP = s.ppos[b]; Q = s.quat[b]; PQ = s.pquat[b]; }
                const float4 v = tof4(scale(sub(xyz(P), xyz(PP)), inv_dt), 0.0f);
                s.vel[b] = v;
                q4 dq = qmul(toq(Q), qconj(toq(PQ)));
                if (dq.w < 0) dq = qneg(dq);
                s.angvel[b] = tof4(scale(sscale(2.0f, xyz(dq)), inv_dt), 0.0f);
                if (acc_here) {
                    const float4 v0 = s.vb[b];
                    a.acc[(size_t)env * B + b] = make_float4((v.x - v0.x) * a.inv_step, (v.y - v0.y) * a.inv_step, (v.z - v0.z) * a.inv_step, 0.0f);
                }
            }
        }
        wave_sync<HBM>();
        // ---- K: update_joint_states (:1550-1638) ------------------------------------
        if (live && do_solve) {
            for (uint32_t j = sl; j < a.J; j += G) {
                const JointRec& jr = md.joints[j];
                const uint32_t type = (uint32_t)jr.params[0];
                const uint32_t ja = (uint32_t)jr.params[1], jb = (uint32_t)jr.params[2];
                float jp = 0.0f, jv = 0.0f;
                // Working sets in HBM: the orientations are read only by the joint types that
                // use them.
                const bool uses_q = !HBM || type == JOINT_REVOLUTE || type == JOINT_PRISMATIC;
                const q4 q_a = uses_q ? toq(s.quat[ja]) : mk4(0.0f, 0.0f, 0.0f, 1.0f);
                const q4 q_b = uses_q ? toq(s.quat[jb]) : mk4(0.0f, 0.0f, 0.0f, 1.0f);
                if (type == JOINT_REVOLUTE) {
                    const f3 axis_local = mk3(jr.axis[0], jr.axis[1], jr.axis[2]);
                    const f3 aw = qrot(axis_local, q_a);
                    const q4 q_rel = qmul(qconj(q_a), q_b);
                    jp = 2.0f * z_atan2f(dot(xyz(q_rel), axis_local), q_rel.w);
                    jv = dot(sub(xyz(s.angvel[jb]), xyz(s.angvel[ja])), aw);
                } else if (type == JOINT_PRISMATIC) {
                    const f3 aw = qrot(mk3(jr.axis[0], jr.axis[1], jr.axis[2]), q_a);
                    const f3 r_a = qrot(mk3(jr.anchor_parent[0], jr.anchor_parent[1], jr.anchor_parent[2]), q_a);
                    const f3 r_b = qrot(mk3(jr.anchor_child[0], jr.anchor_child[1], jr.anchor_child[2]), q_b);
                    jp = dot(sub(add(xyz(s.pos[jb]), r_b), add(xyz(s.pos[ja]), r_a)), aw);
                    const f3 vpa = add(xyz(s.vel[ja]), cross(xyz(s.angvel[ja]), r_a));
                    const f3 vpb = add(xyz(s.vel[jb]), cross(xyz(s.angvel[jb]), r_b));
                    jv = dot(sub(vpb, vpa), aw);
                }
                s.jp[j] = jp;
                s.jv[j] = jv;
            }
        }
        wave_sync<HBM>();
        // ---- L: read_sensors (:1799-1893); cache_contacts is the next snapshot --------
        // The row is assembled in the working set and written back with the state. Entries
        // that no sensor writes are 0 (nothing else ever writes the observation buffer).
        if (stepped && do_solve && step + 1 == a.substeps) {
            float* obs = s.obs;
            for (uint32_t k = sl; k < a.obsp; k += G) obs[k] = 0.0f;
            wave_sync<HBM>();
            for (uint32_t k = sl; k < a.S; k += G) {
                const SensorRec& sr = md.sensors[k];
                const uint32_t obj = sr.type_object[1];
                float* o = obs + (uint32_t)sr.params[3];
                switch (sr.type_object[0]) {
                    case S_JOINT_POS: o[0] = s.jp[obj]; break;
                    case S_JOINT_VEL: o[0] = s.jv[obj]; break;
                    case S_ACCELEROMETER: {
                        f3 lg = qrot(mk3(a.gx, a.gy, a.gz), qconj(toq(s.quat[obj])));
                        o[0] = lg.x; o[1] = lg.y; o[2] = lg.z;
                        break;
                    }
                    case S_GYRO: case S_FRAMEANGVEL: { float4 w = s.angvel[obj]; o[0] = w.x; o[1] = w.y; o[2] = w.z; break; }
                    case S_FRAMEPOS: { float4 p = s.pos[obj]; o[0] = p.x; o[1] = p.y; o[2] = p.z; break; }
                    case S_FRAMEQUAT: { float4 q = s.quat[obj]; o[0] = q.x; o[1] = q.y; o[2] = q.z; o[3] = q.w; break; }
                    case S_FRAMELINVEL: { float4 v = s.vel[obj]; o[0] = v.x; o[1] = v.y; o[2] = v.z; break; }
                    default: break;
                }
            }
        }
        pcount = count;
        wave_sync<HBM>();
        tick(PH_POST);
    }

    // ---- Write back (LDS -> HBM) ------------------------------------------------------
    if (!live) return;
    const uint32_t n_out = count < M ? count : M;
    if (stepped) {
        const size_t eb = (size_t)env * B;
        const StepArgs::HostViews& hv = a.hv;
        if (do_solve) {
        // With the pose arrays aliased on the state, only the accelerations (and any held
        // views) are written, so the pose reads are skipped when no view needs them.
        const bool pose_out = !alias || hv.pos || hv.quat || hv.angvel;
        if (!HBM) {
        for (uint32_t b = sl; b < B; b += G) {
            const float4 p = s.pos[b], q = s.quat[b], v = s.vel[b], v0 = s.vb[b], w = s.angvel[b];
            const float4 acc = make_float4((v.x - v0.x) * a.inv_step, (v.y - v0.y) * a.inv_step, (v.z - v0.z) * a.inv_step, 0.0f);
            a.pos[eb + b] = p;
            a.quat[eb + b] = q;
            a.vel[eb + b] = v;
            a.angvel[eb + b] = w;
            a.acc[eb + b] = acc;
            if (hv.pos) hv.pos[eb + b] = p;
            if (hv.quat) hv.quat[eb + b] = q;
            if (hv.vel) hv.vel[eb + b] = v;
            if (hv.angvel) hv.angvel[eb + b] = w;
            if (hv.acc) hv.acc[eb + b] = acc;
        }
        } else {
        for (uint32_t b = sl; b < B; b += G) {
            if (j_acc && !(md.invmi[b].x < 1e-8f)) continue;  // written by the velocity update
            const float4 v = s.vel[b], v0 = s.vb[b];
            const float4 acc = make_float4((v.x - v0.x) * a.inv_step, (v.y - v0.y) * a.inv_step, (v.z - v0.z) * a.inv_step, 0.0f);
            a.acc[eb + b] = acc;
            if (hv.vel) hv.vel[eb + b] = v;
            if (hv.acc) hv.acc[eb + b] = acc;
            if (pose_out) {
                const float4 p = s.pos[b], q = s.quat[b], w = s.angvel[b];
                if (!alias) {
                    a.pos[eb + b] = p;
                    a.quat[eb + b] = q;
                    a.vel[eb + b] = v;
                    a.angvel[eb + b] = w;
                }
                if (hv.pos) hv.pos[eb + b] = p;
                if (hv.quat) hv.quat[eb + b] = q;
                if (hv.angvel) hv.angvel[eb + b] = w;
            }
        }
        }  // HBM
        for (uint32_t j = sl; j < a.J; j += G) {
            const size_t o = (size_t)env * Jp + j;
            a.jtrq[o] = s.jt[j];
            a.jpos[o] = s.jp[j];
            a.jvel[o] = s.jv[j];
            if (hv.jtrq) hv.jtrq[o] = s.jt[j];
            if (hv.jpos) hv.jpos[o] = s.jp[j];
            if (hv.jvel) hv.jvel[o] = s.jv[j];
        }
        for (uint32_t k = sl; k < a.obsp; k += G) {
            const size_t o = (size_t)env * a.obsp + k;
            a.obs[o] = s.obs[k];
            if (hv.obs) hv.obs[o] = s.obs[k];
        }
        }  // do_solve
        if (do_prep) {
        ContactRec* gc = a.contacts + (size_t)env * M;
        for (uint32_t k = sl; k < n_out; k += G) {
            const float4* src = (const float4*)&s.con[s.perm[k]];
            const float4 c0 = src[0], c1 = src[1], c2 = src[2], c3 = src[3];
            float4* d = (float4*)&gc[k];
            d[0] = c0; d[1] = c1; d[2] = c2; d[3] = c3;
            if (hv.contacts) {
                float4* h = (float4*)&hv.contacts[(size_t)env * M + k];
                h[0] = c0; h[1] = c1; h[2] = c2; h[3] = c3;
            }
        }
        if (sl == 0) {
            a.counts[env] = count;
            if (hv.counts) hv.counts[env] = count;
        }
        }  // do_prep
    } else if (do_prep) {
        // Not advanced: keep visible state, record the advanced contact list as the
        // previous-contact snapshot (world.zig:880-928 restores everything else).
        ContactRec* pc = a.prev_out + (size_t)env * M;
        for (uint32_t k = sl; k < n_out; k += G) {
            const float4* src = (const float4*)&s.con[s.perm[k]];
            float4* d = (float4*)&pc[k];
            d[0] = src[0]; d[1] = src[1]; d[2] = src[2]; d[3] = src[3];
        }
    }
    if (do_solve) {
        for (uint32_t i = sl; i < N; i += G) a.lam[(size_t)env * N + i] = s.lam[i];
    }
    if (do_prep && sl == 0) {
        a.pcounts[env] = count;
        if (a.prev_detached_out) a.prev_detached_out[env] = stepped ? 0 : 1;
    }
    tick(PH_STORE);
    if (timer) {
        for (int ph = 0; ph < kPhaseCount; ++ph) a.phase_ticks[ph] = t_acc[ph];
    }
}

#define ZA_CHECK(x)                      \
    do {                                 \
        hipError_t _e = (x);             \
        if (_e != hipSuccess) return _e; \
    } while (0)

template <int EPW, int PL, bool HASH, bool GROUP = false, bool SPLIT = false>
hipError_t allow_lds(size_t shmem) {
    // Workgroups above 64 KB of dynamic LDS must opt in per kernel (gfx950 has 160 KB / CU).
    static size_t granted = 64 * 1024;
    if (shmem <= granted) return hipSuccess;
    hipError_t e = hipFuncSetAttribute((const void*)step_kernel<EPW, PL, HASH, GROUP, SPLIT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem);
    if (e == hipSuccess) granted = shmem;
    return e;
}

template <int EPW, int PL, bool HASH, bool GROUP = false, bool SPLIT = false>
int resident_as(size_t shmem, int waves = 1) {
    // A shape that does not fit is an answer here, not an error: the failed query's error
    // is taken off HIP's last-error slot so that later hipGetLastError checks (of this or
    // another world) do not report it.
    int n = 0;
    if (allow_lds<EPW, PL, HASH, GROUP, SPLIT>(shmem) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, step_kernel<EPW, PL, HASH, GROUP, SPLIT>, kWave * waves, shmem) !=
            hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

template <int EPW, int PL, bool HASH, bool GROUP = false, bool SPLIT = false>
hipError_t launch_as(const StepArgs& a, uint32_t blocks, size_t shmem, hipStream_t stream, int waves = 1) {
    ZA_CHECK((allow_lds<EPW, PL, HASH, GROUP, SPLIT>(shmem)));
    hipLaunchKernelGGL((step_kernel<EPW, PL, HASH, GROUP, SPLIT>), dim3(blocks), dim3(kWave * waves), shmem, stream, a);
    return hipGetLastError();
}

}  // namespace

size_t max_lds_per_workgroup(int device) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) != hipSuccess || v <= 0) return 64 * 1024;
    return (size_t)v;
}

int resident_workgroups(int envs_per_wave, uint32_t placement, bool hash, size_t shmem, int waves, bool split) {
    if (waves < 1 || waves > kMaxWaves) return 0;
    if (hash || placement != PL_LDS) {
        if (envs_per_wave != 1 || waves != 1 || split) return 0;
        switch (placement) {
            case PL_LDS: return resident_as<1, PL_LDS, true>(shmem);
            case PL_MODEL_HBM: return hash ? resident_as<1, PL_MODEL_HBM, true>(shmem) : resident_as<1, PL_MODEL_HBM, false>(shmem);
            case PL_ALL_HBM: return hash ? resident_as<1, PL_ALL_HBM, true>(shmem) : resident_as<1, PL_ALL_HBM, false>(shmem);
            case PL_WORK_HBM: return hash ? resident_as<1, PL_WORK_HBM, true>(shmem) : resident_as<1, PL_WORK_HBM, false>(shmem);
            default: return 0;
        }
    }
    if (split) {
        switch (envs_per_wave) {
            case 1: return resident_as<1, PL_LDS, false, false, true>(shmem, 2 * waves);
            case 2: return resident_as<2, PL_LDS, false, false, true>(shmem, 2 * waves);
            case 4: return resident_as<4, PL_LDS, false, false, true>(shmem, 2 * waves);
            case 8: return resident_as<8, PL_LDS, false, false, true>(shmem, 2 * waves);
            default: return 0;
        }
    }
    switch (envs_per_wave) {
        case 1: return resident_as<1, PL_LDS, false>(shmem, waves);
        case 2: return resident_as<2, PL_LDS, false>(shmem, waves);
        case 4: return resident_as<4, PL_LDS, false>(shmem, waves);
        case 8: return resident_as<8, PL_LDS, false>(shmem, waves);
        default: return 0;
    }
}

hipError_t launch_step(const StepArgs& a, int envs_per_wave, int waves, hipStream_t stream, bool split) {
    if (a.E == 0) return hipSuccess;
    if (waves < 1 || waves > kMaxWaves) return hipErrorInvalidValue;
    if (split && (a.placement != PL_LDS || a.hash)) return hipErrorInvalidValue;
    const uint32_t per_group = (uint32_t)envs_per_wave * (uint32_t)waves;
    const uint32_t blocks = (a.E + per_group - 1) / per_group;
    if ((a.placement != PL_LDS || a.hash) && (envs_per_wave != 1 || waves != 1)) return hipErrorInvalidValue;
    if ((a.placement >= PL_ALL_HBM) != (a.work != nullptr)) return hipErrorInvalidValue;
    const size_t env_lds = (size_t)a.lds.bytes * (size_t)envs_per_wave;
    const size_t shmem = (size_t)a.ml.bytes + env_lds * (size_t)waves;
    // Extended-contact mode with one environment per workgroup: the instance whose narrow
    // phase visits the slots grouped by geom-type pair (same results, less divergence).
    if (a.ext_contacts && a.M >= 64 && envs_per_wave == 1 && !split) {
        switch (a.placement) {
            case PL_WORK_HBM:
                return a.hash ? launch_as<1, PL_WORK_HBM, true, true>(a, blocks, 0, stream)
                              : launch_as<1, PL_WORK_HBM, false, true>(a, blocks, 0, stream);
            case PL_ALL_HBM:
                return a.hash ? launch_as<1, PL_ALL_HBM, true, true>(a, blocks, a.lds_small.bytes, stream)
                              : launch_as<1, PL_ALL_HBM, false, true>(a, blocks, a.lds_small.bytes, stream);
            case PL_MODEL_HBM:
                return a.hash ? launch_as<1, PL_MODEL_HBM, true, true>(a, blocks, env_lds, stream)
                              : launch_as<1, PL_MODEL_HBM, false, true>(a, blocks, env_lds, stream);
            case PL_LDS:
                return a.hash ? launch_as<1, PL_LDS, true, true>(a, blocks, shmem, stream)
                              : launch_as<1, PL_LDS, false, true>(a, blocks, shmem, stream, waves);
            default: return hipErrorInvalidValue;
        }
    }
    switch (a.placement) {
        case PL_WORK_HBM:
            return a.hash ? launch_as<1, PL_WORK_HBM, true>(a, blocks, 0, stream)
                          : launch_as<1, PL_WORK_HBM, false>(a, blocks, 0, stream);
        case PL_ALL_HBM:
            return a.hash ? launch_as<1, PL_ALL_HBM, true>(a, blocks, a.lds_small.bytes, stream)
                          : launch_as<1, PL_ALL_HBM, false>(a, blocks, a.lds_small.bytes, stream);
        case PL_MODEL_HBM:
            return a.hash ? launch_as<1, PL_MODEL_HBM, true>(a, blocks, env_lds, stream)
                          : launch_as<1, PL_MODEL_HBM, false>(a, blocks, env_lds, stream);
        case PL_LDS: break;
        default: return hipErrorInvalidValue;
    }
    if (a.hash) return launch_as<1, PL_LDS, true>(a, blocks, shmem, stream);
    if (split) {
        switch (envs_per_wave) {
            case 1: return launch_as<1, PL_LDS, false, false, true>(a, blocks, shmem, stream, 2 * waves);
            case 2: return launch_as<2, PL_LDS, false, false, true>(a, blocks, shmem, stream, 2 * waves);
            case 4: return launch_as<4, PL_LDS, false, false, true>(a, blocks, shmem, stream, 2 * waves);
            case 8: return launch_as<8, PL_LDS, false, false, true>(a, blocks, shmem, stream, 2 * waves);
            default: return hipErrorInvalidValue;
        }
    }
    switch (envs_per_wave) {
        case 1: return launch_as<1, PL_LDS, false>(a, blocks, shmem, stream, waves);
        case 2: return launch_as<2, PL_LDS, false>(a, blocks, shmem, stream, waves);
        case 4: return launch_as<4, PL_LDS, false>(a, blocks, shmem, stream, waves);
        case 8: return launch_as<8, PL_LDS, false>(a, blocks, shmem, stream, waves);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace za
