/*
 * CPU oracle for Lulzx/zeno's batched physics step.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline. The product never links
 * it. Each function below restates one MSL kernel of src/shaders/all_shaders.metal for a
 * single environment, in the order World.stepOnce dispatches them
 * (src/world/world.zig:934-1293). Build with -ffp-contract=off and without fast-math.
 *
 * How each function is pinned (tests/, by checks that do not restate its code; every
 * function is pinned, none is left "parity unpinned"):
 *   zo_atan2f, zo_asinf        float64 ground truth within 3 ulp, IEEE special cases
 *                              (test_oracle.py)
 *   k_apply_actions            the reference's actuator KATs, clamp order (test_oracle.py,
 *                              test_oracle_pins.py)
 *   k_compute_forces           gravity torque (R c) x m g on an offset-COM body (test_oracle_pins.py)
 *   k_update_kinematic         closed form of a kinematic body (test_oracle.py)
 *   k_apply_joint_forces       motors on hinges and slides, parent reaction, 1e-6 threshold
 *                              (test_oracle.py, test_oracle_pins.py)
 *   k_save_prev, k_integrate   free-body closed form, world-frame angular velocity, order and
 *                              renormalisation (test_oracle.py, test_oracle_pins.py)
 *   k_broad_phase              fixtures C1-C3, margin, contype/conaffinity rule, plane rule
 *                              (test_oracle.py, test_oracle_pins.py, test_count_wrap.py)
 *   k_broad_phase_hash         cell closed forms, the pair set and order, threshold, filters,
 *                              overflow (test_hash.py)
 *   k_sort_contacts            stable sort by (min<<16)|max, wraps (test_oracle.py, test_count_wrap.py)
 *   k_narrow_phase             reference KATs, capsule endpoint, overlap midpoint, friction
 *                              mean, plane height (test_oracle.py, test_oracle_pins.py)
 *   k_match_cached             hand-built cases: radius, nearest, ties (test_oracle.py)
 *   k_solve_joints             closed forms per constraint type, COM levers, targets, limits
 *                              (test_oracle.py, test_oracle_pins.py)
 *   k_solve_contacts           physical laws of one contact step, restitution, correction
 *                              split (test_contact_solve.py, test_oracle_pins.py)
 *   k_warm_start, k_store_lambda   the 0.8 factor and the stored lambda (test_contact_solve.py,
 *                              test_oracle_pins.py)
 *   k_update_velocities        shortest-arc angular velocity (test_oracle_pins.py)
 *   k_update_joint_states      hinge and slide states (test_oracle.py, test_oracle_pins.py)
 *   k_read_sensors             frame, accelerometer and gyro sensors (test_oracle.py,
 *                              test_oracle_pins.py, test_contact_solve.py)
 *   k_cache_contacts, zo_step  snapshot, substep dt, accelerations (test_oracle_pins.py)
 *   zo_collide_env             extended-contact slots (test_ext_contacts.py)
 *   zo_build_templates         fixtures C1-C4, template fields per joint type, colouring
 *                              (test_oracle.py, test_model.py)
 *   zo_detect_collision(s)     float64 geometry per pair, dispatch flips (test_narrow_ext.py)
 * tests/test_oracle_mutants.py plants plausible misreadings of the reference in a copy of
 * this file; each must fail at least one of those pins.
 *
 * Where the reference runs unordered atomics or races, this oracle fixes one sequential
 * schedule (the HIP kernel reproduces the same):
 *   S1 broad-phase appends in (g, g') order;
 *   S2 per-body joint-force sums in ascending joint order, body_a before body_b;
 *   S3 joint constraints per colour, in colour-sorted template order;
 *   S4 contact slots Gauss-Seidel in slot order, each slot seeing earlier slots' writes.
 */
#include "zeno_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
/* The thread count of a call that passes none: OpenMP's default (OMP_NUM_THREADS, else the
 * processor count) read once when the library loads. A call's count goes to its own loop
 * only (num_threads clause), never to the process-wide setting, which would stay for every
 * later call. */
static int zo_default_threads = 1;
__attribute__((constructor)) static void zo_read_default_threads(void) { zo_default_threads = omp_get_max_threads(); }
#endif

/* ------------------------------------------------------------------------------------
 * Vector helpers with MSL semantics (all_shaders.metal:76-100). Expressions evaluate left
 * to right; dot(a,b) = a.x*b.x + a.y*b.y + a.z*b.z; length = sqrt(dot).
 * ---------------------------------------------------------------------------------- */
typedef struct { float x, y, z; } v3;
typedef struct { float x, y, z, w; } q4;

static inline v3 V(float x, float y, float z) { v3 r = {x, y, z}; return r; }
static inline v3 vadd(v3 a, v3 b) { return V(a.x + b.x, a.y + b.y, a.z + b.z); }
static inline v3 vsub(v3 a, v3 b) { return V(a.x - b.x, a.y - b.y, a.z - b.z); }
static inline v3 vmul(v3 a, v3 b) { return V(a.x * b.x, a.y * b.y, a.z * b.z); }
static inline v3 vscale(v3 a, float s) { return V(a.x * s, a.y * s, a.z * s); }
static inline v3 sscale(float s, v3 a) { return V(s * a.x, s * a.y, s * a.z); }
static inline v3 vdivs(v3 a, float s) { return V(a.x / s, a.y / s, a.z / s); }
static inline v3 vneg(v3 a) { return V(-a.x, -a.y, -a.z); }
static inline float vdot(v3 a, v3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
static inline float vlen(v3 a) { return sqrtf(vdot(a, a)); }
static inline v3 vcross(v3 a, v3 b) {
    return V(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
static inline v3 ld3(const float* p) { return V(p[0], p[1], p[2]); }
static inline void st3(float* p, v3 a) { p[0] = a.x; p[1] = a.y; p[2] = a.z; }
static inline q4 Q(float x, float y, float z, float w) { q4 r = {x, y, z, w}; return r; }
static inline q4 ld4(const float* p) { return Q(p[0], p[1], p[2], p[3]); }
static inline void st4(float* p, q4 a) { p[0] = a.x; p[1] = a.y; p[2] = a.z; p[3] = a.w; }
static inline q4 qadd(q4 a, q4 b) { return Q(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
static inline q4 qsub(q4 a, q4 b) { return Q(a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w); }
static inline q4 qscale(q4 a, float s) { return Q(a.x * s, a.y * s, a.z * s, a.w * s); }
static inline q4 qneg(q4 a) { return Q(-a.x, -a.y, -a.z, -a.w); }
static inline v3 qxyz(q4 a) { return V(a.x, a.y, a.z); }

/* all_shaders.metal:77-84 */
static inline q4 qmul(q4 a, q4 b) {
    return Q(a.w * b.x + a.x * b.w + a.y * b.z - a.z * b.y,
             a.w * b.y - a.x * b.z + a.y * b.w + a.z * b.x,
             a.w * b.z + a.x * b.y - a.y * b.x + a.z * b.w,
             a.w * b.w - a.x * b.x - a.y * b.y - a.z * b.z);
}
/* :86-88 */
static inline q4 qconj(q4 q) { return Q(-q.x, -q.y, -q.z, q.w); }
/* :90-95 */
static inline v3 qrot(v3 v, q4 q) {
    v3 qv = V(q.x, q.y, q.z);
    v3 uv = vcross(qv, v);
    v3 uuv = vcross(qv, uv);
    return V(v.x + 2.0f * (q.w * uv.x + uuv.x), v.y + 2.0f * (q.w * uv.y + uuv.y),
             v.z + 2.0f * (q.w * uv.z + uuv.z));
}
static inline float qlen(q4 q) { return sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w); }
/* :97-100 */
static inline q4 qnormalize(q4 q) {
    float len = qlen(q);
    return len > 1e-8f ? Q(q.x / len, q.y / len, q.z / len, q.w / len) : Q(0, 0, 0, 1);
}
/* MSL clamp(x, lo, hi) = fmin(fmax(x, lo), hi). */
static inline float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }

/* ------------------------------------------------------------------------------------
 * atan2 / asin: S. Moshier's Cephes single-precision routines (atanf.c, asinf.c):
 * argument reduction at tan(3pi/8) and tan(pi/8) plus a degree-9 odd polynomial for atan,
 * and the 0.5 split with sqrt reduction plus a degree-11 odd polynomial for asin. Both stay
 * within 3 ulp of the exact value (tests/test_oracle.py checks this against numpy float64).
 * ---------------------------------------------------------------------------------- */
#define ZO_PI 3.14159265358979323846f
#define ZO_PIO2 1.57079632679489661923f
#define ZO_PIO4 0.78539816339744830962f

static float atan_pos(float x) { /* x >= 0 */
    float y0, t;
    if (x > 2.414213562373095f) { y0 = ZO_PIO2; t = -1.0f / x; }
    else if (x > 0.4142135623730950f) { y0 = ZO_PIO4; t = (x - 1.0f) / (x + 1.0f); }
    else { y0 = 0.0f; t = x; }
    float z = t * t;
    float p = (((8.05374449538e-2f * z - 1.38776856032e-1f) * z + 1.99777106478e-1f) * z - 3.33329491539e-1f) * z * t + t;
    return y0 + p;
}

float zo_atan2f(float y, float x) {
    if (isnan(x) || isnan(y)) return x + y;
    if (x == 0.0f) {
        if (y > 0.0f) return ZO_PIO2;
        if (y < 0.0f) return -ZO_PIO2;
        return signbit(x) ? (signbit(y) ? -ZO_PI : ZO_PI) : y;
    }
    if (y == 0.0f) return signbit(x) ? (signbit(y) ? -ZO_PI : ZO_PI) : y;
    float ax = fabsf(x), ay = fabsf(y);
    float r;
    if (isinf(ax)) {
        if (isinf(ay)) r = x > 0.0f ? ZO_PIO4 : 3.0f * ZO_PIO4;
        else r = x > 0.0f ? 0.0f : ZO_PI;
    } else if (isinf(ay)) {
        r = ZO_PIO2;
    } else {
        float a = atan_pos(ay / ax);
        r = x > 0.0f ? a : ZO_PI - a;
    }
    return y < 0.0f ? -r : r;
}

float zo_asinf(float x) {
    if (isnan(x)) return x;
    float a = fabsf(x);
    if (a > 1.0f) return NAN;
    float z, t;
    int flag = a > 0.5f;
    if (flag) { z = 0.5f * (1.0f - a); t = sqrtf(z); }
    else { t = a; z = a * a; }
    float p = ((((4.2163199048e-2f * z + 2.4181311049e-2f) * z + 4.5470025998e-2f) * z + 7.4953002686e-2f) * z + 1.6666752422e-1f) * z * t + t;
    if (flag) p = ZO_PIO2 - (p + p);
    return x < 0.0f ? -p : p;
}

/* ------------------------------------------------------------------------------------
 * Per-env views.
 * ---------------------------------------------------------------------------------- */
typedef struct {
    const ZoModel* m;
    uint32_t env, B, J, Jp, A, M, N, obsp;
    float dt;
    float *pos, *quat, *vel, *angvel, *invmi, *frc, *trq, *ppos, *pquat;
    float *jpos, *jvel, *jtrq, *obs;
    ZoContact *con, *pcon;
    uint32_t *count, *pcount;
    ZoConstraint* cs;
    uint32_t* cell_ids; /* [G], spatial-hash mode */
} Env;

#define P4(arr, b) (&(arr)[4 * (size_t)(b)])

/* warm_start_constraints, all_shaders.metal:1408-1426 (factor buffer = 0.8, world.zig:478) */
static void k_warm_start(Env* e) {
    for (uint32_t i = 0; i < e->N; ++i) e->cs[i].state[0] = 0.8f * e->cs[i].state[1];
}

/* apply_actions, :196-229 */
static void k_apply_actions(Env* e, const float* actions) {
    for (uint32_t a = 0; a < e->A; ++a) {
        const ZoActuator* act = &e->m->actuators[a];
        uint32_t joint_id = (uint32_t)act->params[0];
        float ctrl = clampf(actions[a], act->params[1], act->params[2]);
        float torque = ctrl * act->params[3];
        torque = clampf(torque, act->params2[0], act->params2[1]);
        e->jtrq[joint_id] = torque;
    }
}

/* compute_forces, :345-388 */
static void k_compute_forces(Env* e) {
    const float* g = e->m->gravity;
    for (uint32_t b = 0; b < e->B; ++b) {
        float inv_mass = P4(e->invmi, b)[0];
        if (inv_mass < 1e-8f) {
            st4(P4(e->frc, b), Q(0, 0, 0, 0));
            st4(P4(e->trq, b), Q(0, 0, 0, 0));
            continue;
        }
        float mass = 1.0f / inv_mass;
        v3 force = V(g[0] * mass, g[1] * mass, g[2] * mass);
        st4(P4(e->frc, b), Q(force.x, force.y, force.z, 0));
        v3 com_world = qrot(ld3(e->m->bodies[b].com_offset), ld4(P4(e->quat, b)));
        v3 t = vcross(com_world, force);
        st4(P4(e->trq, b), Q(t.x, t.y, t.z, 0));
    }
}

/* update_kinematic, :304-339 (body type 1 only) */
static void k_update_kinematic(Env* e) {
    for (uint32_t b = 0; b < e->B; ++b) {
        if ((uint32_t)e->m->bodies[b].params[1] != 1u) continue;
        v3 vel = ld3(P4(e->vel, b));
        v3 pos = vadd(ld3(P4(e->pos, b)), vscale(vel, e->dt));
        st4(P4(e->pos, b), Q(pos.x, pos.y, pos.z, 0));
        v3 om = ld3(P4(e->angvel, b));
        q4 q = ld4(P4(e->quat, b));
        v3 h = vscale(vscale(om, e->dt), 0.5f);
        q4 dq = qmul(Q(h.x, h.y, h.z, 0), q);
        st4(P4(e->quat, b), qnormalize(qadd(q, dq)));
    }
}

/* apply_joint_forces, :122-190, summed in schedule S2. */
static void add3(float* p, v3 d) { p[0] = p[0] + d.x; p[1] = p[1] + d.y; p[2] = p[2] + d.z; }
static void k_apply_joint_forces(Env* e) {
    for (uint32_t j = 0; j < e->J; ++j) {
        const ZoJoint* jt = &e->m->joints[j];
        float f = e->jtrq[j];
        if (fabsf(f) < 1e-6f) continue;
        uint32_t type = (uint32_t)jt->params[0];
        uint32_t a = (uint32_t)jt->params[1], b = (uint32_t)jt->params[2];
        v3 axis_world = qrot(ld3(jt->axis), ld4(P4(e->quat, a)));
        v3 w = vscale(axis_world, f);
        float* dst = type == 2 ? e->frc : e->trq;
        if (a > 0) add3(P4(dst, a), vneg(w));
        if (b > 0) add3(P4(dst, b), w);
    }
}

/* save_prev_state, :1900-1913 */
static void k_save_prev(Env* e) {
    memcpy(e->ppos, e->pos, sizeof(float) * 4 * e->B);
    memcpy(e->pquat, e->quat, sizeof(float) * 4 * e->B);
}

/* integrate, :394-462 */
static void k_integrate(Env* e) {
    const float dt = e->dt;
    for (uint32_t b = 0; b < e->B; ++b) {
        const float* imi = P4(e->invmi, b);
        float inv_mass = imi[0];
        if (inv_mass < 1e-8f) continue;
        v3 force = ld3(P4(e->frc, b));
        v3 vel = ld3(P4(e->vel, b));
        v3 pos = ld3(P4(e->pos, b));
        v3 accel = vscale(force, inv_mass);
        vel = vadd(vel, vscale(accel, dt));
        vel = vscale(vel, 0.999f);
        pos = vadd(pos, vscale(vel, dt));
        st4(P4(e->vel, b), Q(vel.x, vel.y, vel.z, 0));
        st4(P4(e->pos, b), Q(pos.x, pos.y, pos.z, 0));
        v3 inv_inertia = V(imi[1], imi[2], imi[3]);
        v3 torque = ld3(P4(e->trq, b));
        v3 omega = ld3(P4(e->angvel, b));
        q4 quat = ld4(P4(e->quat, b));
        omega = vadd(omega, vscale(vmul(inv_inertia, torque), dt));
        omega = vscale(omega, 0.999f);
        v3 h = vscale(vscale(omega, dt), 0.5f);
        q4 dq = qmul(Q(h.x, h.y, h.z, 0), quat);
        quat = qadd(quat, dq);
        float ql = qlen(quat);
        if (ql > 1e-8f) quat = Q(quat.x / ql, quat.y / ql, quat.z / ql, quat.w / ql);
        else quat = Q(0, 0, 0, 1);
        st4(P4(e->angvel, b), Q(omega.x, omega.y, omega.z, 0));
        st4(P4(e->quat, b), quat);
    }
}

/* broad_phase, :468-533, appended in schedule S1. */
static void k_broad_phase(const ZoModel* m, const float* pos, uint32_t B_unused, ZoContact* con, uint32_t* count) {
    (void)B_unused;
    const uint32_t G = m->num_geoms, M = m->max_contacts;
    for (uint32_t g = 0; g < G; ++g) {
        const ZoGeom* ga = &m->geoms[g];
        uint32_t body_a = ga->type_body[1];
        v3 pos_a = vadd(ld3(P4(pos, body_a)), ld3(ga->pos_size0));
        float radius_a = ga->pos_size0[3];
        uint32_t type_a = ga->type_body[0], group_a = ga->type_body[3], mask_a = ga->type_body[2];
        for (uint32_t o = g + 1; o < G; ++o) {
            const ZoGeom* gb = &m->geoms[o];
            uint32_t body_b = gb->type_body[1];
            if (body_a == body_b) continue;
            uint32_t type_b = gb->type_body[0], group_b = gb->type_body[3], mask_b = gb->type_body[2];
            if ((group_a & mask_b) == 0 && (group_b & mask_a) == 0) continue;
            v3 pos_b = vadd(ld3(P4(pos, body_b)), ld3(gb->pos_size0));
            float radius_b = gb->pos_size0[3];
            int is_plane_pair = (type_a == 3 || type_b == 3);
            if (!is_plane_pair) {
                v3 diff = vsub(pos_b, pos_a);
                float dist_sq = vdot(diff, diff);
                float min_dist = radius_a + radius_b + 0.1f;
                if (dist_sq >= min_dist * min_dist) continue;
            }
            uint32_t c = (*count)++;
            if (c < M) {
                ZoContact* ct = &con[c];
                ct->indices[0] = body_a; ct->indices[1] = body_b; ct->indices[2] = g; ct->indices[3] = o;
            }
        }
    }
}

/* ------------------------------------------------------------------------------------
 * Spatial-hash broad phase (all_shaders.metal:556-703), which World.stepOnce runs instead
 * of broad_phase when the scene has more than 512 geoms (world.zig:534,1043-1096): a
 * 64^3 grid of unit cells (world.zig:542-563, inv_cell_size 1.0).
 *
 * Cell of a geom (:574-580): floor(pos * inv_cell_size) per axis, converted to int and
 * clamped to [0, 63]. The GPU's float->int conversion saturates and maps NaN to 0, so a
 * NaN, negative or huge coordinate lands in cell 0 or 63 of that axis.
 *
 * Emission order. The reference appends through an atomic counter from every thread at
 * once, and its scatter/query barrier (:631) spans one threadgroup only, so its order is
 * a race. This restatement runs it sequentially: every geom scattered (in ascending geom
 * order, so each cell lists its geoms in ascending order) before any query; then geom g
 * in ascending order queries dz, dy, dx = -1..1 (that loop nesting, :644-646) and the
 * cell's geoms in list order, appending (body_a, body_b, g, other) for other > g that
 * pass the same filters as broad_phase (:659-681). The set of pairs is the reference's;
 * the order is one of its possible interleavings.
 * ---------------------------------------------------------------------------------- */
#define ZO_HASH_DIM 64u
#define ZO_HASH_MIN_GEOMS 512u /* world.zig:534: hash when num_geoms > 512 */

static uint32_t hash_axis(float p) {
    float f = floorf(p * 1.0f);
    if (!(f >= 0.0f)) return 0u; /* negative, or NaN (converts to 0) */
    if (f >= (float)(ZO_HASH_DIM - 1u)) return ZO_HASH_DIM - 1u;
    return (uint32_t)f;
}

static int cmp_u64(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

static void k_broad_phase_hash(const ZoModel* m, const float* pos, uint32_t* cell_ids, ZoContact* con, uint32_t* count) {
    const uint32_t G = m->num_geoms, M = m->max_contacts, D = ZO_HASH_DIM;
    uint32_t* cx = (uint32_t*)malloc(sizeof(uint32_t) * 3 * (G ? G : 1));
    uint64_t* cells = (uint64_t*)malloc(sizeof(uint64_t) * (G ? G : 1)); /* (cell << 32) | geom */
    /* broad_phase_count_cells (:556-584) */
    for (uint32_t g = 0; g < G; ++g) {
        const ZoGeom* ga = &m->geoms[g];
        v3 p = vadd(ld3(P4(pos, ga->type_body[1])), ld3(ga->pos_size0));
        cx[3 * g + 0] = hash_axis(p.x);
        cx[3 * g + 1] = hash_axis(p.y);
        cx[3 * g + 2] = hash_axis(p.z);
        uint32_t id = cx[3 * g + 0] + cx[3 * g + 1] * D + cx[3 * g + 2] * D * D;
        if (cell_ids) cell_ids[g] = id;
        cells[g] = ((uint64_t)id << 32) | g;
    }
    /* broad_phase_prefix_sum + scatter (:588-629): the cells' lists back to back */
    qsort(cells, G, sizeof(uint64_t), cmp_u64);
    /* broad_phase_detect queries (:632-700) */
    for (uint32_t g = 0; g < G; ++g) {
        const ZoGeom* ga = &m->geoms[g];
        uint32_t body_a = ga->type_body[1];
        v3 pos_a = vadd(ld3(P4(pos, body_a)), ld3(ga->pos_size0));
        float radius_a = ga->pos_size0[3];
        uint32_t type_a = ga->type_body[0], group_a = ga->type_body[3], mask_a = ga->type_body[2];
        for (int dz = -1; dz <= 1; ++dz) for (int dy = -1; dy <= 1; ++dy) for (int dx = -1; dx <= 1; ++dx) {
            int nx = (int)cx[3 * g + 0] + dx, ny = (int)cx[3 * g + 1] + dy, nz = (int)cx[3 * g + 2] + dz;
            if (nx < 0 || ny < 0 || nz < 0 || nx >= (int)D || ny >= (int)D || nz >= (int)D) continue;
            uint64_t ncid = (uint64_t)((uint32_t)nx + (uint32_t)ny * D + (uint32_t)nz * D * D);
            /* first list entry of cell ncid */
            uint32_t lo = 0, hi = G;
            while (lo < hi) {
                uint32_t mid = lo + (hi - lo) / 2;
                if ((cells[mid] >> 32) < ncid) lo = mid + 1; else hi = mid;
            }
            for (uint32_t s = lo; s < G && (cells[s] >> 32) == ncid; ++s) {
                uint32_t o = (uint32_t)(cells[s] & 0xFFFFFFFFu);
                if (o <= g) continue;
                const ZoGeom* gb = &m->geoms[o];
                uint32_t body_b = gb->type_body[1];
                if (body_a == body_b) continue;
                uint32_t group_b = gb->type_body[3], mask_b = gb->type_body[2];
                if ((group_a & mask_b) == 0 && (group_b & mask_a) == 0) continue;
                uint32_t type_b = gb->type_body[0];
                v3 pos_b = vadd(ld3(P4(pos, body_b)), ld3(gb->pos_size0));
                float radius_b = gb->pos_size0[3];
                if (!(type_a == 3 || type_b == 3)) {
                    v3 diff = vsub(pos_b, pos_a);
                    float dist_sq = vdot(diff, diff);
                    float min_dist = radius_a + radius_b + 0.1f;
                    if (dist_sq >= min_dist * min_dist) continue;
                }
                uint32_t c = (*count)++;
                if (c < M) {
                    ZoContact* ct = &con[c];
                    ct->indices[0] = body_a; ct->indices[1] = body_b; ct->indices[2] = g; ct->indices[3] = o;
                }
            }
        }
    }
    free(cells);
    free(cx);
}

/* sort_contacts, :711-745 (stable insertion sort by (min<<16)|max) */
static void k_sort_contacts(uint32_t M, ZoContact* con, uint32_t raw_count) {
    uint32_t count = raw_count < M ? raw_count : M;
    if (count <= 1) return;
    for (uint32_t i = 1; i < count; ++i) {
        ZoContact key = con[i];
        uint32_t ka = key.indices[0] < key.indices[1] ? key.indices[0] : key.indices[1];
        uint32_t kb = key.indices[0] < key.indices[1] ? key.indices[1] : key.indices[0];
        uint32_t key_val = (ka << 16) | kb;
        int j = (int)i - 1;
        while (j >= 0) {
            const ZoContact* cj = &con[j];
            uint32_t ja = cj->indices[0] < cj->indices[1] ? cj->indices[0] : cj->indices[1];
            uint32_t jb = cj->indices[0] < cj->indices[1] ? cj->indices[1] : cj->indices[0];
            uint32_t j_val = (ja << 16) | jb;
            if (j_val <= key_val) break;
            con[j + 1] = con[j];
            --j;
        }
        con[j + 1] = key;
    }
}

/* narrow_phase, :751-894 */
static void k_narrow_phase(const ZoModel* m, const float* pos, const float* quat, ZoContact* con, uint32_t raw_count) {
    const uint32_t M = m->max_contacts;
    for (uint32_t s = 0; s < M; ++s) {
        if (s >= raw_count) break;
        ZoContact* c = &con[s];
        uint32_t body_a = c->indices[0], body_b = c->indices[1];
        const ZoGeom* ga = &m->geoms[c->indices[2]];
        const ZoGeom* gb = &m->geoms[c->indices[3]];
        v3 pos_a = vadd(ld3(P4(pos, body_a)), ld3(ga->pos_size0));
        v3 pos_b = vadd(ld3(P4(pos, body_b)), ld3(gb->pos_size0));
        uint32_t type_a = ga->type_body[0], type_b = gb->type_body[0];
        v3 normal = V(0, 0, 0), contact_point = V(0, 0, 0);
        float penetration = 0.0f;
        int has_contact = 0;
        if (type_a == 0 && type_b == 0) {
            float ra = ga->pos_size0[3], rb = gb->pos_size0[3];
            v3 diff = vsub(pos_b, pos_a);
            float dist = vlen(diff);
            float min_dist = ra + rb;
            if (dist < min_dist && dist > 1e-6f) {
                normal = vdivs(diff, dist);
                penetration = min_dist - dist;
                contact_point = vadd(pos_a, vscale(normal, ra - penetration * 0.5f));
                has_contact = 1;
            }
        } else if ((type_a == 0 && type_b == 3) || (type_a == 3 && type_b == 0)) {
            v3 sphere_pos, plane_pos, plane_normal = V(0, 0, 1);
            float sphere_radius;
            if (type_a == 0) { sphere_pos = pos_a; sphere_radius = ga->pos_size0[3]; plane_pos = pos_b; }
            else { sphere_pos = pos_b; sphere_radius = gb->pos_size0[3]; plane_pos = pos_a; }
            float signed_dist = vdot(vsub(sphere_pos, plane_pos), plane_normal);
            if (signed_dist < sphere_radius) {
                normal = plane_normal;
                penetration = sphere_radius - signed_dist;
                contact_point = vsub(sphere_pos, vscale(plane_normal, signed_dist + penetration * 0.5f));
                has_contact = 1;
                if (type_a == 3) normal = vneg(normal);
            }
        } else if ((type_a == 1 && type_b == 3) || (type_a == 3 && type_b == 1)) {
            v3 cap_pos;
            float cap_r, cap_hl;
            q4 cap_q;
            v3 plane_normal = V(0, 0, 1);
            if (type_a == 1) { cap_pos = pos_a; cap_r = ga->pos_size0[3]; cap_hl = ga->params[0]; cap_q = ld4(ga->quat); }
            else { cap_pos = pos_b; cap_r = gb->pos_size0[3]; cap_hl = gb->params[0]; cap_q = ld4(gb->quat); }
            v3 axis = qrot(V(0, 0, 1), cap_q);
            v3 p1 = vsub(cap_pos, vscale(axis, cap_hl));
            v3 p2 = vadd(cap_pos, vscale(axis, cap_hl));
            float d1 = p1.z - cap_r;
            float d2 = p2.z - cap_r;
            if (d1 < 0 || d2 < 0) {
                v3 deepest = d1 < d2 ? p1 : p2;
                float dist = fminf(d1, d2);
                normal = type_a == 1 ? plane_normal : vneg(plane_normal);
                penetration = -dist;
                contact_point = deepest;
                contact_point.z = 0;
                has_contact = 1;
            }
        } else if (m->extended_contacts) {
            /* Extended-contact mode: detectCollision (narrow_phase.zig:28-123) on the geoms
             * and their bodies' poses; a contact fills the slot as above. solve_contact
             * moves body a along +normal, so the normal must point from b to a:
             * detectCollision's does for mixed pairs; capsule-capsule and box-box give a
             * to b and are negated. */
            ZoCollider ca, cb;
            ZoContactResult r;
            memset(&ca, 0, sizeof ca);
            memset(&cb, 0, sizeof cb);
            ca.type = type_a; ca.size[0] = ga->pos_size0[3]; ca.size[1] = ga->params[0]; ca.size[2] = ga->params[1];
            cb.type = type_b; cb.size[0] = gb->pos_size0[3]; cb.size[1] = gb->params[0]; cb.size[2] = gb->params[1];
            memcpy(ca.local_pos, ga->pos_size0, 12);
            memcpy(cb.local_pos, gb->pos_size0, 12);
            memcpy(ca.position, P4(pos, body_a), 12);
            memcpy(cb.position, P4(pos, body_b), 12);
            memcpy(ca.quaternion, P4(quat, body_a), 16);
            memcpy(cb.quaternion, P4(quat, body_b), 16);
            if (zo_detect_collision(&ca, &cb, &r)) {
                normal = type_a == type_b ? vneg(ld3(r.normal)) : ld3(r.normal);
                penetration = r.penetration;
                contact_point = ld3(r.point);
                has_contact = 1;
            }
        }
        if (has_contact) {
            float mu = sqrtf(ga->params[2] * gb->params[2]);
            c->position_pen[0] = contact_point.x; c->position_pen[1] = contact_point.y;
            c->position_pen[2] = contact_point.z; c->position_pen[3] = penetration;
            c->normal_friction[0] = normal.x; c->normal_friction[1] = normal.y;
            c->normal_friction[2] = normal.z; c->normal_friction[3] = mu;
            c->impulses[0] = 0; c->impulses[1] = 0; c->impulses[2] = 0; c->impulses[3] = m->restitution;
        } else {
            c->position_pen[3] = -1.0f;
        }
    }
}

/* match_cached_contacts, :1483-1544 */
static void k_match_cached(Env* e) {
    const uint32_t M = e->M;
    uint32_t count = *e->count, prev_count = *e->pcount;
    for (uint32_t s = 0; s < M; ++s) {
        if (s >= count) break;
        ZoContact* c = &e->con[s];
        if (c->position_pen[3] < 0) continue;
        uint32_t a = c->indices[0], b = c->indices[1];
        v3 p = ld3(c->position_pen);
        float best = 0.04f;
        int best_i = -1;
        for (uint32_t i = 0; i < prev_count && i < M; ++i) {
            const ZoContact* pc = &e->pcon[i];
            if (pc->position_pen[3] < 0) continue;
            int same = (pc->indices[0] == a && pc->indices[1] == b) || (pc->indices[0] == b && pc->indices[1] == a);
            if (!same) continue;
            v3 d = vsub(ld3(pc->position_pen), p);
            float dsq = vdot(d, d);
            if (dsq < best) { best = dsq; best_i = (int)i; }
        }
        if (best_i >= 0) {
            const ZoContact* pc = &e->pcon[best_i];
            c->impulses[0] = pc->impulses[0] * 0.8f;
            c->impulses[1] = pc->impulses[1] * 0.8f;
            c->impulses[2] = pc->impulses[2] * 0.8f;
        }
    }
}

/* solve_joints, :909-1399, for one constraint record of this env. */
static void solve_constraint(Env* e, ZoConstraint* cp) {
    ZoConstraint c = *cp;
    uint32_t type = c.indices[3] & 0xFFu;
    if (type > 10) return;
    uint32_t ia = c.indices[0], ib = c.indices[1];
    const float* imi_a = P4(e->invmi, ia);
    const float* imi_b = P4(e->invmi, ib);
    float inv_mass_a = imi_a[0], inv_mass_b = imi_b[0];
    v3 iI_a = V(imi_a[1], imi_a[2], imi_a[3]);
    v3 iI_b = V(imi_b[1], imi_b[2], imi_b[3]);
    float inv_mass_sum = inv_mass_a + inv_mass_b;
    if (inv_mass_sum < 1e-8f) return;
    float* Pa = P4(e->pos, ia);
    float* Pb = P4(e->pos, ib);
    float* Qa = P4(e->quat, ia);
    float* Qb = P4(e->quat, ib);
    v3 pos_a = ld3(Pa), pos_b = ld3(Pb);
    q4 quat_a = ld4(Qa), quat_b = ld4(Qb);
    float compliance = c.anchor_a[3];
    float dt = e->dt;
    float alpha_tilde = compliance / (dt * dt);
    float C;

    if (type == 2) {
        v3 r_a = qrot(ld3(c.anchor_a), quat_a);
        v3 r_b = qrot(ld3(c.anchor_b), quat_b);
        v3 diff = vsub(vadd(pos_a, r_a), vadd(pos_b, r_b));
        C = vlen(diff);
        if (C > 1e-6f) {
            v3 n = vdivs(diff, C);
            v3 rn_a = vcross(r_a, n), rn_b = vcross(r_b, n);
            float w_a = inv_mass_a + vdot(vmul(rn_a, iI_a), rn_a);
            float w_b = inv_mass_b + vdot(vmul(rn_b, iI_b), rn_b);
            float w = w_a + w_b;
            float lambda_prev = c.state[0];
            float d_lambda = (-C - alpha_tilde * lambda_prev) / (w + alpha_tilde);
            c.state[0] = lambda_prev + d_lambda;
            v3 impulse = sscale(d_lambda, n);
            v3 rc_a = vsub(r_a, qrot(ld3(e->m->bodies[ia].com_offset), quat_a));
            v3 rc_b = vsub(r_b, qrot(ld3(e->m->bodies[ib].com_offset), quat_b));
            if (inv_mass_a > 0) {
                st3(Pa, vadd(ld3(Pa), vscale(impulse, inv_mass_a)));
                v3 d_omega = vmul(vcross(rc_a, impulse), iI_a);
                q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), quat_a), 0.5f);
                st4(Qa, qnormalize(qadd(quat_a, dq)));
            }
            if (inv_mass_b > 0) {
                st3(Pb, vsub(ld3(Pb), vscale(impulse, inv_mass_b)));
                v3 d_omega = vmul(vcross(rc_b, impulse), iI_b);
                q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), quat_b), 0.5f);
                st4(Qb, qnormalize(qsub(quat_b, dq)));
            }
        }
    } else if (type == 7) {
        v3 r_a = qrot(ld3(c.anchor_a), quat_a);
        v3 r_b = qrot(ld3(c.anchor_b), quat_b);
        v3 diff = vsub(vadd(pos_a, r_a), vadd(pos_b, r_b));
        C = vlen(diff);
        if (C > 1e-6f) {
            v3 n = vdivs(diff, C);
            v3 rn_b = vcross(r_b, n);
            float w_b = inv_mass_b + vdot(vmul(rn_b, iI_b), rn_b);
            if (w_b > 1e-8f) {
                float d_lambda = (-C) / (w_b + alpha_tilde);
                v3 impulse = sscale(d_lambda, n);
                st3(Pb, vsub(ld3(Pb), vscale(impulse, inv_mass_b)));
                v3 d_omega = vmul(vcross(r_b, impulse), iI_b);
                q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), quat_b), 0.5f);
                st4(Qb, qnormalize(qsub(quat_b, dq)));
            }
        }
        q4 target = ld4(c.axis_target);
        q4 qa = ld4(Qa), qb = ld4(Qb);
        q4 q_rel = qmul(qconj(qa), qb);
        q4 q_err = qmul(q_rel, qconj(target));
        if (q_err.w < 0) q_err = qneg(q_err);
        v3 exyz = qxyz(q_err);
        float s = vlen(exyz);
        if (s > 1e-6f) {
            v3 axis_rel = vdivs(exyz, s);
            float angle = 2.0f * zo_atan2f(s, q_err.w);
            v3 axis_world = qrot(axis_rel, qa);
            float w_b = vdot(vmul(axis_world, iI_b), axis_world);
            if (w_b > 1e-8f) {
                float d_lambda_ang = angle / (w_b + alpha_tilde);
                v3 ang_impulse = sscale(d_lambda_ang, axis_world);
                if (inv_mass_b > 0) {
                    v3 d_omega = vmul(ang_impulse, iI_b);
                    q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), qb), 0.5f);
                    st4(Qb, qnormalize(qsub(qb, dq)));
                }
            }
        }
    } else if (type == 3) {
        q4 qa = ld4(Qa), qb = ld4(Qb);
        v3 axa = qrot(ld3(c.anchor_a), qa);
        v3 axb = qrot(ld3(c.anchor_b), qb);
        v3 cr = vcross(axa, axb);
        float sin_angle = vlen(cr);
        if (sin_angle > 1e-6f) {
            v3 n = vdivs(cr, sin_angle);
            float ang_C = zo_asinf(clampf(sin_angle, -1.0f, 1.0f));
            float w_a = vdot(vmul(n, iI_a), n);
            float w_b = vdot(vmul(n, iI_b), n);
            float w = w_a + w_b;
            if (w > 1e-8f) {
                float d_lambda = -ang_C / (w + alpha_tilde);
                if (inv_mass_a > 0) {
                    v3 d_omega = vmul(sscale(d_lambda, n), iI_a);
                    q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), qa), 0.5f);
                    st4(Qa, qnormalize(qadd(qa, dq)));
                }
                if (inv_mass_b > 0) {
                    v3 d_omega = vmul(sscale(-d_lambda, n), iI_b);
                    q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), qb), 0.5f);
                    st4(Qb, qnormalize(qadd(qb, dq)));
                }
            }
        }
    } else if (type == 4) {
        v3 axis_local = ld3(c.anchor_a);
        float lower = c.limits[0], upper = c.limits[1];
        q4 qa = ld4(Qa), qb = ld4(Qb);
        q4 q_rel = qmul(qconj(qa), qb);
        float sin_half = vdot(qxyz(q_rel), axis_local);
        float angle = 2.0f * zo_atan2f(sin_half, q_rel.w);
        float violation = 0.0f;
        if (angle < lower) violation = lower - angle;
        else if (angle > upper) violation = upper - angle;
        if (fabsf(violation) > 1e-6f) {
            v3 axis_world = qrot(axis_local, qa);
            float w_a = vdot(vmul(axis_world, iI_a), axis_world);
            float w_b = vdot(vmul(axis_world, iI_b), axis_world);
            float w = w_a + w_b;
            if (w > 1e-8f) {
                float d_lambda = violation / (w + alpha_tilde);
                v3 ang_impulse = sscale(d_lambda, axis_world);
                if (inv_mass_a > 0) {
                    v3 d_omega = vmul(ang_impulse, iI_a);
                    q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), qa), 0.5f);
                    st4(Qa, qnormalize(qadd(qa, dq)));
                }
                if (inv_mass_b > 0) {
                    v3 d_omega = vmul(ang_impulse, iI_b);
                    q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), qb), 0.5f);
                    st4(Qb, qnormalize(qsub(qb, dq)));
                }
            }
        }
    } else if (type == 5) {
        v3 axis_local = ld3(c.anchor_a);
        float lower = c.limits[0], upper = c.limits[1];
        q4 qa = ld4(Qa), qb = ld4(Qb);
        v3 r_a = qrot(V(0, 0, 0), qa);
        v3 r_b = qrot(ld3(c.anchor_b), qb);
        v3 axis_world = qrot(axis_local, qa);
        v3 diff = vsub(vadd(pos_b, r_b), vadd(pos_a, r_a));
        float dist = vdot(diff, axis_world);
        float violation = 0.0f;
        if (dist < lower) violation = lower - dist;
        else if (dist > upper) violation = upper - dist;
        if (fabsf(violation) > 1e-6f) {
            v3 n = violation > 0 ? axis_world : vneg(axis_world);
            float abs_v = fabsf(violation);
            v3 rn_a = vcross(r_a, n), rn_b = vcross(r_b, n);
            float w_a = inv_mass_a + vdot(vmul(rn_a, iI_a), rn_a);
            float w_b = inv_mass_b + vdot(vmul(rn_b, iI_b), rn_b);
            float w = w_a + w_b;
            if (w > 1e-8f) {
                float d_lambda = abs_v / (w + alpha_tilde);
                v3 impulse = sscale(d_lambda, n);
                if (inv_mass_a > 0) st3(Pa, vsub(ld3(Pa), vscale(impulse, inv_mass_a)));
                if (inv_mass_b > 0) st3(Pb, vadd(ld3(Pb), vscale(impulse, inv_mass_b)));
            }
        }
    } else if (type == 10) {
        v3 r_a = qrot(ld3(c.anchor_a), quat_a);
        v3 r_b = qrot(ld3(c.anchor_b), quat_b);
        v3 diff = vsub(vadd(pos_a, r_a), vadd(pos_b, r_b));
        v3 axis_world = qrot(ld3(c.axis_target), quat_a);
        float along = vdot(diff, axis_world);
        v3 perp = vsub(diff, sscale(along, axis_world));
        float perp_len = vlen(perp);
        if (perp_len > 1e-6f) {
            v3 n = vdivs(perp, perp_len);
            v3 rn_a = vcross(r_a, n), rn_b = vcross(r_b, n);
            float w_a = inv_mass_a + vdot(vmul(rn_a, iI_a), rn_a);
            float w_b = inv_mass_b + vdot(vmul(rn_b, iI_b), rn_b);
            float w = w_a + w_b;
            float d_lambda = (-perp_len) / (w + alpha_tilde);
            v3 impulse = sscale(d_lambda, n);
            if (inv_mass_a > 0) {
                st3(Pa, vadd(ld3(Pa), vscale(impulse, inv_mass_a)));
                v3 d_omega = vmul(vcross(r_a, impulse), iI_a);
                q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), quat_a), 0.5f);
                st4(Qa, qnormalize(qadd(quat_a, dq)));
            }
            if (inv_mass_b > 0) {
                st3(Pb, vsub(ld3(Pb), vscale(impulse, inv_mass_b)));
                v3 d_omega = vmul(vcross(r_b, impulse), iI_b);
                q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), quat_b), 0.5f);
                st4(Qb, qnormalize(qsub(quat_b, dq)));
            }
        }
        q4 target = Q(c.limits[0], c.limits[1], c.limits[2], c.limits[3]);
        q4 qa = ld4(Qa), qb = ld4(Qb);
        q4 q_rel = qmul(qconj(qa), qb);
        q4 q_err = qmul(q_rel, qconj(target));
        if (q_err.w < 0) q_err = qneg(q_err);
        v3 exyz = qxyz(q_err);
        float s = vlen(exyz);
        if (s > 1e-6f) {
            v3 axis_err = vdivs(exyz, s);
            float angle_err = 2.0f * zo_atan2f(s, q_err.w);
            v3 aw = qrot(axis_err, qa);
            float w_a = vdot(vmul(aw, iI_a), aw);
            float w_b = vdot(vmul(aw, iI_b), aw);
            float w = w_a + w_b;
            if (w > 1e-8f) {
                float d_lambda_ang = angle_err / (w + alpha_tilde);
                v3 ang_impulse = sscale(d_lambda_ang, aw);
                if (inv_mass_a > 0) {
                    v3 d_omega = vmul(ang_impulse, iI_a);
                    q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), qa), 0.5f);
                    st4(Qa, qnormalize(qadd(qa, dq)));
                }
                if (inv_mass_b > 0) {
                    v3 d_omega = vmul(ang_impulse, iI_b);
                    q4 dq = qscale(qmul(Q(d_omega.x, d_omega.y, d_omega.z, 0), qb), 0.5f);
                    st4(Qb, qnormalize(qsub(qb, dq)));
                }
            }
        }
    }
    *cp = c;
}

/* Group H, world.zig:1163-1195 (schedule S3) */
static void k_solve_joints(Env* e, uint32_t iterations) {
    if (e->N == 0) return;
    for (uint32_t it = 0; it < iterations; ++it) {
        for (uint32_t col = 0; col < e->m->num_colors; ++col) {
            uint32_t off = e->m->color_ranges[2 * col], cnt = e->m->color_ranges[2 * col + 1];
            for (uint32_t k = 0; k < cnt; ++k) solve_constraint(e, &e->cs[off + k]);
        }
    }
}

/* solve_contacts, :1644-1793, one slot (schedule S4: caller iterates slots in order). */
static void solve_contact(Env* e, uint32_t s) {
    ZoContact c = e->con[s];
    if (c.position_pen[3] < 0) return;
    uint32_t ia = c.indices[0], ib = c.indices[1];
    const float* imi_a = P4(e->invmi, ia);
    const float* imi_b = P4(e->invmi, ib);
    float inv_mass_a = imi_a[0], inv_mass_b = imi_b[0];
    v3 iI_a = V(imi_a[1], imi_a[2], imi_a[3]);
    v3 iI_b = V(imi_b[1], imi_b[2], imi_b[3]);
    float inv_mass_sum = inv_mass_a + inv_mass_b;
    if (inv_mass_sum < 1e-8f) return;
    v3 normal = ld3(c.normal_friction);
    float penetration = c.position_pen[3];
    float friction = c.normal_friction[3];
    v3 cp = ld3(c.position_pen);
    float* Pa = P4(e->pos, ia);
    float* Pb = P4(e->pos, ib);
    float* Va = P4(e->vel, ia);
    float* Vb = P4(e->vel, ib);
    float* Wa = P4(e->angvel, ia);
    float* Wb = P4(e->angvel, ib);
    v3 pos_a = ld3(Pa), pos_b = ld3(Pb);
    v3 r_a = vsub(cp, pos_a), r_b = vsub(cp, pos_b);
    v3 omega_a = ld3(Wa), omega_b = ld3(Wb);
    v3 vel_a = vadd(ld3(Va), vcross(omega_a, r_a));
    v3 vel_b = vadd(ld3(Vb), vcross(omega_b, r_b));
    v3 rel_vel = vsub(vel_a, vel_b);
    float vel_normal = vdot(rel_vel, normal);
    v3 vel_tangent = vsub(rel_vel, sscale(vel_normal, normal));
    float tangent_speed = vlen(vel_tangent);
    v3 rn_a = vcross(r_a, normal), rn_b = vcross(r_b, normal);
    float w_n_a = inv_mass_a + vdot(vmul(rn_a, iI_a), rn_a);
    float w_n_b = inv_mass_b + vdot(vmul(rn_b, iI_b), rn_b);
    float w_normal = w_n_a + w_n_b;
    if (w_normal < 1e-8f) return;
    const float beta = e->m->baumgarte, slop = e->m->slop;
    float bias = beta * fmaxf(penetration - slop, 0.0f) / e->dt;
    float restitution = c.impulses[3];
    float vel_restitution = vel_normal < -0.5f ? restitution * vel_normal : 0.0f;
    float j_n = (-(vel_normal + vel_restitution) + bias) / w_normal;
    j_n = fmaxf(j_n, 0.0f);
    v3 impulse_n = sscale(j_n, normal);
    float pos_correction = beta * fmaxf(penetration - slop, 0.0f);
    if (inv_mass_a > 1e-8f) {
        st3(Va, vadd(ld3(Va), vscale(impulse_n, inv_mass_a)));
        st3(Wa, vadd(ld3(Wa), vmul(vcross(r_a, impulse_n), iI_a)));
        float ratio = inv_mass_a / inv_mass_sum;
        st3(Pa, vadd(ld3(Pa), sscale(pos_correction * ratio, normal)));
    }
    if (inv_mass_b > 1e-8f) {
        st3(Vb, vsub(ld3(Vb), vscale(impulse_n, inv_mass_b)));
        st3(Wb, vsub(ld3(Wb), vmul(vcross(r_b, impulse_n), iI_b)));
        float ratio = inv_mass_b / inv_mass_sum;
        st3(Pb, vsub(ld3(Pb), sscale(pos_correction * ratio, normal)));
    }
    float j_n_acc = e->con[s].impulses[0] + j_n;
    if (tangent_speed > 1e-6f && j_n_acc > 1e-6f) {
        v3 tangent = vdivs(vel_tangent, tangent_speed);
        v3 rt_a = vcross(r_a, tangent), rt_b = vcross(r_b, tangent);
        float w_t_a = inv_mass_a + vdot(vmul(rt_a, iI_a), rt_a);
        float w_t_b = inv_mass_b + vdot(vmul(rt_b, iI_b), rt_b);
        float w_tangent = w_t_a + w_t_b;
        if (w_tangent > 1e-8f) {
            float j_t_desired = tangent_speed / w_tangent;
            float j_t_max = friction * j_n_acc;
            float j_t = fminf(j_t_desired, j_t_max);
            v3 impulse_t = sscale(j_t, tangent);
            if (inv_mass_a > 1e-8f) {
                st3(Va, vsub(ld3(Va), vscale(impulse_t, inv_mass_a)));
                st3(Wa, vsub(ld3(Wa), vmul(vcross(r_a, impulse_t), iI_a)));
            }
            if (inv_mass_b > 1e-8f) {
                st3(Vb, vadd(ld3(Vb), vscale(impulse_t, inv_mass_b)));
                st3(Wb, vadd(ld3(Wb), vmul(vcross(r_b, impulse_t), iI_b)));
            }
        }
    }
    e->con[s].impulses[0] = j_n;
}

/* Group I, world.zig:1199-1213 */
static void k_solve_contacts(Env* e, uint32_t iterations) {
    uint32_t count = *e->count;
    for (uint32_t it = 0; it < iterations; ++it)
        for (uint32_t s = 0; s < e->M && s < count; ++s) solve_contact(e, s);
}

/* xpbd_update_velocities, :1922-1961 */
static void k_update_velocities(Env* e) {
    float inv_dt = 1.0f / e->dt;
    for (uint32_t b = 0; b < e->B; ++b) {
        if (P4(e->invmi, b)[0] < 1e-8f) continue;
        v3 v = vscale(vsub(ld3(P4(e->pos, b)), ld3(P4(e->ppos, b))), inv_dt);
        st4(P4(e->vel, b), Q(v.x, v.y, v.z, 0));
        q4 dq = qmul(ld4(P4(e->quat, b)), qconj(ld4(P4(e->pquat, b))));
        if (dq.w < 0) dq = qneg(dq);
        v3 w = vscale(sscale(2.0f, qxyz(dq)), inv_dt);
        st4(P4(e->angvel, b), Q(w.x, w.y, w.z, 0));
    }
}

/* update_joint_states, :1550-1638 */
static void k_update_joint_states(Env* e) {
    for (uint32_t j = 0; j < e->J; ++j) {
        const ZoJoint* jt = &e->m->joints[j];
        uint32_t type = (uint32_t)jt->params[0];
        e->jpos[j] = 0;
        e->jvel[j] = 0;
        uint32_t a = (uint32_t)jt->params[1], b = (uint32_t)jt->params[2];
        q4 q_a = ld4(P4(e->quat, a)), q_b = ld4(P4(e->quat, b));
        v3 p_a = ld3(P4(e->pos, a)), p_b = ld3(P4(e->pos, b));
        v3 v_a = ld3(P4(e->vel, a)), v_b = ld3(P4(e->vel, b));
        v3 w_a = ld3(P4(e->angvel, a)), w_b = ld3(P4(e->angvel, b));
        if (type == 1) {
            v3 axis_local = ld3(jt->axis);
            v3 axis_world_a = qrot(axis_local, q_a);
            q4 q_rel = qmul(qconj(q_a), q_b);
            float sin_half = vdot(qxyz(q_rel), axis_local);
            e->jpos[j] = 2.0f * zo_atan2f(sin_half, q_rel.w);
            e->jvel[j] = vdot(vsub(w_b, w_a), axis_world_a);
        } else if (type == 2) {
            v3 axis_world_a = qrot(ld3(jt->axis), q_a);
            v3 r_a = qrot(ld3(jt->anchor_parent), q_a);
            v3 r_b = qrot(ld3(jt->anchor_child), q_b);
            v3 diff = vsub(vadd(p_b, r_b), vadd(p_a, r_a));
            e->jpos[j] = vdot(diff, axis_world_a);
            v3 v_pt_a = vadd(v_a, vcross(w_a, r_a));
            v3 v_pt_b = vadd(v_b, vcross(w_b, r_b));
            e->jvel[j] = vdot(vsub(v_pt_b, v_pt_a), axis_world_a);
        }
    }
}

/* read_sensors, :1799-1893 */
static void k_read_sensors(Env* e) {
    const ZoModel* m = e->m;
    for (uint32_t si = 0; si < m->num_sensors; ++si) {
        const ZoSensor* s = &m->sensors[si];
        uint32_t type = s->type_object[0], obj = s->type_object[1];
        uint32_t off = (uint32_t)s->params[3];
        float* o = e->obs + off;
        switch (type) {
            case 0: o[0] = e->jpos[obj]; break;
            case 1: o[0] = e->jvel[obj]; break;
            case 2: {
                q4 q = ld4(P4(e->quat, obj));
                v3 lg = qrot(V(m->gravity[0], m->gravity[1], m->gravity[2]), qconj(q));
                o[0] = lg.x; o[1] = lg.y; o[2] = lg.z;
                break;
            }
            case 3: case 10: { const float* w = P4(e->angvel, obj); o[0] = w[0]; o[1] = w[1]; o[2] = w[2]; break; }
            case 7: { const float* p = P4(e->pos, obj); o[0] = p[0]; o[1] = p[1]; o[2] = p[2]; break; }
            case 8: { const float* q = P4(e->quat, obj); o[0] = q[0]; o[1] = q[1]; o[2] = q[2]; o[3] = q[3]; break; }
            case 9: { const float* v = P4(e->vel, obj); o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; break; }
            default: break;
        }
    }
}

/* cache_contacts, :1454-1478 */
static void k_cache_contacts(Env* e) {
    uint32_t count = *e->count;
    *e->pcount = count;
    for (uint32_t s = 0; s < e->M && s < count; ++s) e->pcon[s] = e->con[s];
}

/* store_lambda_prev, :1428-1444 */
static void k_store_lambda(Env* e) {
    for (uint32_t i = 0; i < e->N; ++i) e->cs[i].state[1] = e->cs[i].state[0];
}

/* World.stepOnce, world.zig:934-1293, for one env. */
static void step_once(Env* e, const float* actions) {
    k_warm_start(e);
    k_apply_actions(e, actions);
    k_compute_forces(e);
    k_update_kinematic(e);
    k_apply_joint_forces(e);
    k_save_prev(e);
    k_integrate(e);
    if (e->m->num_geoms > ZO_HASH_MIN_GEOMS) k_broad_phase_hash(e->m, e->pos, e->cell_ids, e->con, e->count);
    else k_broad_phase(e->m, e->pos, e->B, e->con, e->count);
    k_sort_contacts(e->M, e->con, *e->count);
    k_narrow_phase(e->m, e->pos, e->quat, e->con, *e->count);
    k_match_cached(e);
    k_solve_joints(e, e->m->contact_iterations);
    k_solve_contacts(e, e->m->contact_iterations);
    k_update_velocities(e);
    k_update_joint_states(e);
    k_read_sensors(e);
    k_cache_contacts(e);
    k_store_lambda(e);
}

static void bind_env(const ZoModel* m, ZoState* s, uint32_t env, float dt, Env* e) {
    const size_t B = m->num_bodies;
    e->m = m;
    e->env = env;
    e->B = m->num_bodies;
    e->J = m->num_joints;
    e->Jp = m->num_joints > 0 ? m->num_joints : 1;
    e->A = m->num_actuators;
    e->M = m->max_contacts;
    e->N = m->num_constraints;
    e->obsp = m->obs_dim > 0 ? m->obs_dim : 1;
    e->dt = dt;
    e->pos = s->positions + 4 * B * env;
    e->quat = s->quaternions + 4 * B * env;
    e->vel = s->velocities + 4 * B * env;
    e->angvel = s->angular_velocities + 4 * B * env;
    e->invmi = s->inv_mass_inertia + 4 * B * env;
    e->frc = s->forces + 4 * B * env;
    e->trq = s->torques + 4 * B * env;
    e->ppos = s->prev_positions + 4 * B * env;
    e->pquat = s->prev_quaternions + 4 * B * env;
    e->jpos = s->joint_positions + (size_t)e->Jp * env;
    e->jvel = s->joint_velocities + (size_t)e->Jp * env;
    e->jtrq = s->joint_torques + (size_t)e->Jp * env;
    e->obs = s->observations + (size_t)e->obsp * env;
    e->con = s->contacts + (size_t)e->M * env;
    e->pcon = s->prev_contacts + (size_t)e->M * env;
    e->count = s->contact_counts + env;
    e->pcount = s->prev_contact_counts + env;
    e->cs = s->constraints + (size_t)e->N * env;
    e->cell_ids = s->cell_ids ? s->cell_ids + (size_t)m->num_geoms * env : NULL;
}

int zo_step(const ZoModel* m, ZoState* s, const float* actions, uint32_t substeps,
            uint32_t env_begin, uint32_t env_end, int nthreads) {
    uint32_t actual = substeps == 0 ? m->config_substeps : substeps;
    uint32_t div = actual > 1 ? actual : 1;
    float dt = m->timestep / (float)div;
    float inv_step = m->timestep > 0 ? 1.0f / m->timestep : 0.0f;
    const size_t B = m->num_bodies;
    const uint32_t A = m->num_actuators;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : zo_default_threads)
#endif
    for (int64_t ei = (int64_t)env_begin; ei < (int64_t)env_end; ++ei) {
        uint32_t env = (uint32_t)ei;
        Env e;
        bind_env(m, s, env, dt, &e);
        const float* act = actions + (size_t)A * env;
        float* pv = s->prev_velocities + 4 * B * env;
        memcpy(pv, e.vel, sizeof(float) * 4 * B);
        for (uint32_t k = 0; k < actual; ++k) step_once(&e, act);
        float* acc = s->accelerations + 4 * B * env;
        for (size_t b = 0; b < B; ++b) {
            acc[4 * b + 0] = (e.vel[4 * b + 0] - pv[4 * b + 0]) * inv_step;
            acc[4 * b + 1] = (e.vel[4 * b + 1] - pv[4 * b + 1]) * inv_step;
            acc[4 * b + 2] = (e.vel[4 * b + 2] - pv[4 * b + 2]) * inv_step;
            acc[4 * b + 3] = 0.0f;
        }
    }
    return 0;
}

void zo_match_cached(uint32_t max_contacts, ZoContact* contacts, uint32_t count,
                     ZoContact* prev_contacts, uint32_t prev_count) {
    Env e;
    memset(&e, 0, sizeof e);
    e.M = max_contacts;
    e.con = contacts;
    e.pcon = prev_contacts;
    e.count = &count;
    e.pcount = &prev_count;
    k_match_cached(&e);
}

/* solve_contacts (all_shaders.metal:1644-1793) on one slot, exposed for unit tests: the
 * slot's bodies index [num_bodies] records of inverse mass and inertia, positions,
 * velocities and angular velocities (4 floats each), updated in place with the slot. */
void zo_solve_contact_slot(uint32_t num_bodies, const float* inv_mass_inertia, float* positions, float* velocities,
                           float* angular_velocities, ZoContact* contact, float baumgarte, float slop, float dt) {
    ZoModel m;
    Env e;
    uint32_t count = 1;
    memset(&m, 0, sizeof m);
    memset(&e, 0, sizeof e);
    m.baumgarte = baumgarte;
    m.slop = slop;
    e.m = &m;
    e.B = num_bodies;
    e.M = 1;
    e.dt = dt;
    e.invmi = (float*)inv_mass_inertia;
    e.pos = positions;
    e.vel = velocities;
    e.angvel = angular_velocities;
    e.con = contact;
    e.count = &count;
    solve_contact(&e, 0);
}

void zo_broad_phase_hash(const ZoModel* m, const float* positions, uint32_t* cell_ids,
                         ZoContact* contacts, uint32_t* count) {
    k_broad_phase_hash(m, positions, cell_ids, contacts, count);
}

void zo_sort_contacts(uint32_t max_contacts, ZoContact* contacts, uint32_t count) {
    k_sort_contacts(max_contacts, contacts, count);
}

void zo_collide_env(const ZoModel* m, const float* positions, const float* quaternions,
                    ZoContact* contacts, uint32_t* count) {
    if (m->num_geoms > ZO_HASH_MIN_GEOMS) {
        uint32_t* ids = (uint32_t*)malloc(sizeof(uint32_t) * m->num_geoms);
        k_broad_phase_hash(m, positions, ids, contacts, count);
        free(ids);
    } else {
        k_broad_phase(m, positions, m->num_bodies, contacts, count);
    }
    k_sort_contacts(m->max_contacts, contacts, *count);
    k_narrow_phase(m, positions, quaternions, contacts, *count);
}

/* ------------------------------------------------------------------------------------
 * Constraint templates and colouring (joint.zig:202-350, world.zig:311-501,
 * xpbd.zig:533-640). The host-side rotation in world.zig:194-212 has its own operation
 * order.
 * ---------------------------------------------------------------------------------- */
static v3 host_rot(v3 v, q4 q) {
    float t0 = 2.0f * (q.y * v.z - q.z * v.y);
    float t1 = 2.0f * (q.z * v.x - q.x * v.z);
    float t2 = 2.0f * (q.x * v.y - q.y * v.x);
    return V(v.x + q.w * t0 + (q.y * t2 - q.z * t1), v.y + q.w * t1 + (q.z * t0 - q.x * t2),
             v.z + q.w * t2 + (q.x * t1 - q.y * t0));
}

static void tmpl(ZoConstraint* c, uint32_t a, uint32_t b, uint32_t type) {
    memset(c, 0, sizeof *c);
    c->indices[0] = a; c->indices[1] = b; c->indices[2] = 0; c->indices[3] = type;
}

uint32_t zo_build_templates(const ZoJoint* joints, const uint8_t* limited, uint32_t num_joints,
                            const ZoBody* bodies, uint32_t num_bodies,
                            ZoConstraint* out, uint32_t* ranges, uint32_t* num_colors) {
    uint32_t n = 0;
    for (uint32_t j = 0; j < num_joints; ++j) {
        const ZoJoint* jd = &joints[j];
        uint32_t type = (uint32_t)jd->params[0];
        uint32_t a = (uint32_t)jd->params[1], b = (uint32_t)jd->params[2];
        float lower = jd->params[3], upper = jd->params2[0], damping = jd->params2[1];
        int has_limits = limited[j] && lower < upper;
        v3 ap = ld3(jd->anchor_parent), ac = ld3(jd->anchor_child), ax = ld3(jd->axis);
        q4 qa = ld4(bodies[a].quaternion), qb = ld4(bodies[b].quaternion);
        ZoConstraint* c;
        switch (type) {
            case 0: /* fixed -> weld */ {
                c = &out[n++]; tmpl(c, a, b, 7);
                st3(c->anchor_a, ap); st3(c->anchor_b, ac);
                st4(c->axis_target, qmul(qconj(qa), qb));
                break;
            }
            case 1: /* revolute -> point, hinge, [angular limit] */ {
                c = &out[n++]; tmpl(c, a, b, 2);
                st3(c->anchor_a, ap); st3(c->anchor_b, ac);
                c = &out[n++]; tmpl(c, a, b, 3);
                v3 axb = host_rot(host_rot(ax, qa), qconj(qb));
                st3(c->anchor_a, ax); st3(c->anchor_b, axb); c->anchor_b[3] = damping;
                if (has_limits) {
                    c = &out[n++]; tmpl(c, a, b, 4);
                    st3(c->anchor_a, ax); c->limits[0] = lower; c->limits[1] = upper;
                }
                break;
            }
            case 2: /* prismatic -> slider, [linear limit] */ {
                c = &out[n++]; tmpl(c, a, b, 10);
                st3(c->anchor_a, ap); st3(c->anchor_b, ac); c->anchor_b[3] = damping;
                st3(c->axis_target, ax);
                st4(c->limits, qmul(qconj(qa), qb));
                if (has_limits) {
                    c = &out[n++]; tmpl(c, a, b, 5);
                    st3(c->anchor_a, ax); st3(c->anchor_b, ac);
                    c->limits[0] = lower; c->limits[1] = upper;
                }
                break;
            }
            case 3: /* ball -> point, [cone limit as symmetric angular limit] */ {
                c = &out[n++]; tmpl(c, a, b, 2);
                st3(c->anchor_a, ap); st3(c->anchor_b, ac);
                if (has_limits) {
                    c = &out[n++]; tmpl(c, a, b, 4);
                    st3(c->anchor_a, ax); c->limits[0] = -upper; c->limits[1] = upper;
                }
                break;
            }
            case 5: /* universal -> point, hinge(axis), hinge(axis2 = (0,1,0)) */ {
                c = &out[n++]; tmpl(c, a, b, 2);
                st3(c->anchor_a, ap); st3(c->anchor_b, ac);
                c = &out[n++]; tmpl(c, a, b, 3);
                st3(c->anchor_a, ax); st3(c->anchor_b, host_rot(host_rot(ax, qa), qconj(qb)));
                v3 ax2 = V(0, 1, 0);
                c = &out[n++]; tmpl(c, a, b, 3);
                st3(c->anchor_a, ax2); st3(c->anchor_b, host_rot(host_rot(ax2, qa), qconj(qb)));
                break;
            }
            default: break; /* free: no constraints */
        }
    }
    /* Greedy colouring in template order; a constraint takes the smallest colour unused
     * by earlier constraints sharing either body. */
    uint32_t max_color = 0;
    for (uint32_t i = 0; i < n; ++i) {
        unsigned char used[256];
        memset(used, 0, sizeof used);
        uint32_t a = out[i].indices[0], b = out[i].indices[1];
        for (uint32_t k = 0; k < i; ++k) {
            uint32_t ka = out[k].indices[0], kb = out[k].indices[1];
            int shares = 0;
            if (a < num_bodies && (ka == a || kb == a)) shares = 1;
            if (b < num_bodies && b != a && (ka == b || kb == b)) shares = 1;
            if (shares) used[(out[k].indices[3] >> 8) & 0xFF] = 1;
        }
        uint32_t col = 0;
        while (col < 255 && used[col]) ++col;
        out[i].indices[3] = (out[i].indices[3] & 0xFFu) | (col << 8);
        if (col > max_color) max_color = col;
    }
    *num_colors = n ? max_color + 1 : 0;
    /* Stable sort by colour (insertion sort keeps equal keys in order). */
    for (uint32_t i = 1; i < n; ++i) {
        ZoConstraint key = out[i];
        uint32_t kc = (key.indices[3] >> 8) & 0xFF;
        int j = (int)i - 1;
        while (j >= 0 && ((out[j].indices[3] >> 8) & 0xFF) > kc) { out[j + 1] = out[j]; --j; }
        out[j + 1] = key;
    }
    for (uint32_t c2 = 0; c2 < 2 * (*num_colors); ++c2) ranges[c2] = 0;
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t col = (out[i].indices[3] >> 8) & 0xFF;
        if (ranges[2 * col + 1] == 0) ranges[2 * col] = i;
        ranges[2 * col + 1]++;
    }
    return n;
}

/* ------------------------------------------------------------------------------------
 * Extended narrow phase: narrow_phase.detectCollision and the primitive pairs it
 * dispatches to (src/collision/narrow_phase.zig:28-512, helpers :786-925), with
 * body.Transform (src/physics/body.zig:141-268) and primitives.Geom accessors
 * (src/collision/primitives.zig:223-240,413-415). Heightfield, mesh and cylinder pairs
 * (GJK/EPA, :513-785) are not restated: those return no contact here.
 *
 * Zig semantics kept: no FMA contraction, correctly rounded sqrt and division,
 * std.math.clamp(x, lo, hi) = @max(lo, @min(x, hi)) where @min/@max return the non-NaN
 * operand (between +0 and -0 this restatement returns the second operand), @abs = fabs.
 * Axes come from the body transform only (a geom's own local rotation is not applied),
 * as in the reference.
 * ---------------------------------------------------------------------------------- */
#define ZO_NP_EPS 1e-6f /* constants.EPSILON (src/physics/constants.zig:13) */

static float np_min(float a, float b) { return a != a ? b : (b != b ? a : (a < b ? a : b)); }
static float np_max(float a, float b) { return a != a ? b : (b != b ? a : (a > b ? a : b)); }
static float np_clamp(float x, float lo, float hi) { return np_max(lo, np_min(x, hi)); }

/* rotateByQuat, body.zig:254-264 */
static v3 np_rot(v3 v, const float* q) {
    v3 qv = V(q[0], q[1], q[2]);
    v3 uv = vcross(qv, v);
    v3 uuv = vcross(qv, uv);
    return V(v.x + 2.0f * (q[3] * uv.x + uuv.x), v.y + 2.0f * (q[3] * uv.y + uuv.y), v.z + 2.0f * (q[3] * uv.z + uuv.z));
}
/* Transform.transformPoint, body.zig:192-199 */
static v3 np_point(const ZoCollider* c, v3 local) {
    v3 r = np_rot(local, c->quaternion);
    return V(r.x + c->position[0], r.y + c->position[1], r.z + c->position[2]);
}
static v3 np_axis(const ZoCollider* c, float x, float y, float z) { return np_rot(V(x, y, z), c->quaternion); }

static int np_emit(ZoContactResult* out, v3 point, v3 normal, float pen, v3 la, v3 lb) {
    out->point[0] = point.x; out->point[1] = point.y; out->point[2] = point.z;
    out->penetration = pen;
    out->normal[0] = normal.x; out->normal[1] = normal.y; out->normal[2] = normal.z;
    out->valid = 1;
    out->local_a[0] = la.x; out->local_a[1] = la.y; out->local_a[2] = la.z; out->local_a[3] = 0.0f;
    out->local_b[0] = lb.x; out->local_b[1] = lb.y; out->local_b[2] = lb.z; out->local_b[3] = 0.0f;
    return 1;
}

/* flipContact, :912-920 */
static void np_flip(ZoContactResult* r) {
    for (int i = 0; i < 3; ++i) {
        r->normal[i] = r->normal[i] * -1.0f;
        float t = r->local_a[i]; r->local_a[i] = r->local_b[i]; r->local_b[i] = t;
    }
}

/* sphereSphere, :125-153 */
static int np_sphere_sphere(v3 pa, float ra, v3 pb, float rb, ZoContactResult* out) {
    v3 diff = vsub(pb, pa);
    float dist_sq = vdot(diff, diff);
    float min_dist = ra + rb;
    if (dist_sq >= min_dist * min_dist) return 0;
    float dist = sqrtf(dist_sq);
    v3 n = dist > ZO_NP_EPS ? vscale(diff, 1.0f / dist) : V(0.0f, 0.0f, 1.0f);
    float pen = min_dist - dist;
    v3 point = vadd(pa, vscale(n, ra - pen * 0.5f));
    return np_emit(out, point, n, pen, vscale(n, ra), vscale(n, -rb));
}

/* closestPointOnSegment, :815-825 */
static v3 np_closest_on_segment(v3 p, v3 s, v3 e) {
    v3 seg = vsub(e, s);
    float len_sq = vdot(seg, seg);
    if (len_sq < ZO_NP_EPS) return s;
    float t = np_clamp(vdot(vsub(p, s), seg) / len_sq, 0.0f, 1.0f);
    return vadd(s, vscale(seg, t));
}

/* sphereCapsule, :156-197 */
static int np_sphere_capsule(v3 sp, float sr, v3 cp, const ZoCollider* cap, ZoContactResult* out) {
    float cr = cap->size[0], hl = cap->size[1];
    v3 axis = np_axis(cap, 0.0f, 0.0f, 1.0f);
    v3 p1 = vsub(cp, vscale(axis, hl));
    v3 p2 = vadd(cp, vscale(axis, hl));
    v3 closest = np_closest_on_segment(sp, p1, p2);
    v3 diff = vsub(sp, closest);
    float dist_sq = vdot(diff, diff);
    float min_dist = sr + cr;
    if (dist_sq >= min_dist * min_dist) return 0;
    float dist = sqrtf(dist_sq);
    v3 n = dist > ZO_NP_EPS ? vscale(diff, 1.0f / dist) : V(0.0f, 0.0f, 1.0f);
    float pen = min_dist - dist;
    v3 point = vadd(closest, vscale(n, cr - pen * 0.5f));
    return np_emit(out, point, n, pen, vscale(n, sr), vscale(n, -cr));
}

/* spherePlane, :200-228 */
static int np_sphere_plane(v3 sp, float sr, const ZoCollider* pl, ZoContactResult* out) {
    v3 n = np_axis(pl, 0.0f, 0.0f, 1.0f);
    v3 pp = np_point(pl, ld3(pl->local_pos));
    float signed_dist = vdot(vsub(sp, pp), n) - pl->size[0];
    if (signed_dist >= sr) return 0;
    float pen = sr - signed_dist;
    v3 point = vsub(sp, vscale(n, signed_dist + pen * 0.5f));
    return np_emit(out, point, n, pen, vscale(n, -sr), V(0.0f, 0.0f, 0.0f));
}

/* boxFaceNormal, :890-910 */
static v3 np_box_face_normal(v3 p, const float* he) {
    float maxd = -INFINITY;
    float pc[3] = {p.x, p.y, p.z};
    float nrm[3] = {0.0f, 0.0f, 1.0f};
    for (int i = 0; i < 3; ++i) {
        float dpos = he[i] - pc[i];
        float dneg = he[i] + pc[i];
        if (dpos > maxd) { maxd = dpos; nrm[0] = nrm[1] = nrm[2] = 0.0f; nrm[i] = 1.0f; }
        if (dneg > maxd) { maxd = dneg; nrm[0] = nrm[1] = nrm[2] = 0.0f; nrm[i] = -1.0f; }
    }
    return V(nrm[0], nrm[1], nrm[2]);
}

/* sphereBox, :231-277 (the box's inverse transform per Transform.inverse, body.zig:223-235) */
static int np_sphere_box(v3 sp, float sr, const ZoCollider* box, ZoContactResult* out) {
    const float* q = box->quaternion;
    float iq[4] = {-q[0], -q[1], -q[2], q[3]};
    v3 ipos = np_rot(V(-box->position[0], -box->position[1], -box->position[2]), iq);
    v3 r = np_rot(sp, iq);
    v3 ls = V(r.x + ipos.x, r.y + ipos.y, r.z + ipos.z);
    const float* he = box->size;
    v3 cl = V(np_clamp(ls.x, -he[0], he[0]), np_clamp(ls.y, -he[1], he[1]), np_clamp(ls.z, -he[2], he[2]));
    v3 diff = vsub(ls, cl);
    float dist_sq = vdot(diff, diff);
    if (dist_sq >= sr * sr) return 0;
    float dist = sqrtf(dist_sq);
    v3 ln = dist > ZO_NP_EPS ? vscale(diff, 1.0f / dist) : np_box_face_normal(ls, he);
    v3 wc = np_point(box, cl);
    v3 n = np_rot(ln, q);
    float pen = sr - dist;
    v3 point = vadd(wc, vscale(n, pen * 0.5f));
    return np_emit(out, point, n, pen, vscale(n, -sr), vsub(cl, ld3(box->local_pos)));
}

/* closestPointsBetweenSegments, :832-888 */
static void np_closest_between_segments(v3 a1, v3 a2, v3 b1, v3 b2, v3* pa, v3* pb) {
    v3 d1 = vsub(a2, a1), d2 = vsub(b2, b1), r = vsub(a1, b1);
    float a = vdot(d1, d1), e = vdot(d2, d2), f = vdot(d2, r);
    float s = 0.0f, t = 0.0f;
    if (a < ZO_NP_EPS && e < ZO_NP_EPS) { *pa = a1; *pb = b1; return; }
    if (a < ZO_NP_EPS) {
        t = np_clamp(f / e, 0.0f, 1.0f);
    } else {
        float c = vdot(d1, r);
        if (e < ZO_NP_EPS) {
            s = np_clamp(-c / a, 0.0f, 1.0f);
        } else {
            float b = vdot(d1, d2);
            float denom = a * e - b * b;
            if (denom != 0.0f) s = np_clamp((b * f - c * e) / denom, 0.0f, 1.0f);
            t = (b * s + f) / e;
            if (t < 0.0f) {
                t = 0.0f;
                s = np_clamp(-c / a, 0.0f, 1.0f);
            } else if (t > 1.0f) {
                t = 1.0f;
                s = np_clamp((b - c) / a, 0.0f, 1.0f);
            }
        }
    }
    *pa = vadd(a1, vscale(d1, s));
    *pb = vadd(b1, vscale(d2, t));
}

/* capsuleCapsule, :280-331 */
static int np_capsule_capsule(v3 pa, const ZoCollider* ca, v3 pb, const ZoCollider* cb, ZoContactResult* out) {
    float ra = ca->size[0], rb = cb->size[0], ha = ca->size[1], hb = cb->size[1];
    v3 xa = np_axis(ca, 0.0f, 0.0f, 1.0f), xb = np_axis(cb, 0.0f, 0.0f, 1.0f);
    v3 a1 = vsub(pa, vscale(xa, ha)), a2 = vadd(pa, vscale(xa, ha));
    v3 b1 = vsub(pb, vscale(xb, hb)), b2 = vadd(pb, vscale(xb, hb));
    v3 qa, qb;
    np_closest_between_segments(a1, a2, b1, b2, &qa, &qb);
    v3 diff = vsub(qb, qa);
    float dist_sq = vdot(diff, diff);
    float min_dist = ra + rb;
    if (dist_sq >= min_dist * min_dist) return 0;
    float dist = sqrtf(dist_sq);
    v3 n = dist > ZO_NP_EPS ? vscale(diff, 1.0f / dist) : V(0.0f, 0.0f, 1.0f);
    float pen = min_dist - dist;
    v3 wa = vadd(qa, vscale(n, ra));
    v3 wb = vsub(qb, vscale(n, rb));
    v3 point = vscale(vadd(wa, wb), 0.5f);
    return np_emit(out, point, n, pen, vscale(n, ra), vscale(n, -rb));
}

/* capsulePlane, :334-370 */
static int np_capsule_plane(v3 cp, const ZoCollider* cap, const ZoCollider* pl, ZoContactResult* out) {
    float radius = cap->size[0], hl = cap->size[1];
    v3 axis = np_axis(cap, 0.0f, 0.0f, 1.0f);
    v3 n = np_axis(pl, 0.0f, 0.0f, 1.0f);
    v3 pp = np_point(pl, ld3(pl->local_pos));
    v3 p1 = vsub(cp, vscale(axis, hl));
    v3 p2 = vadd(cp, vscale(axis, hl));
    float d1 = vdot(vsub(p1, pp), n) - radius;
    float d2 = vdot(vsub(p2, pp), n) - radius;
    if (d1 >= 0.0f && d2 >= 0.0f) return 0;
    v3 deepest = d1 < d2 ? p1 : p2;
    float dist = np_min(d1, d2);
    v3 point = vsub(deepest, vscale(n, dist * 0.5f + radius));
    return np_emit(out, point, n, -dist, vscale(n, -radius), V(0.0f, 0.0f, 0.0f));
}

/* boxPlane, :373-423 */
static int np_box_plane(const ZoCollider* box, const ZoCollider* pl, ZoContactResult* out) {
    const float* h = box->size;
    v3 n = np_axis(pl, 0.0f, 0.0f, 1.0f);
    v3 pp = np_point(pl, ld3(pl->local_pos));
    const float sx[8] = {-1, 1, -1, 1, -1, 1, -1, 1}, sy[8] = {-1, -1, 1, 1, -1, -1, 1, 1}, sz[8] = {-1, -1, -1, -1, 1, 1, 1, 1};
    float min_dist = INFINITY;
    v3 dc = V(0.0f, 0.0f, 0.0f), dw = V(0.0f, 0.0f, 0.0f);
    for (int k = 0; k < 8; ++k) {
        v3 corner = V(sx[k] < 0 ? -h[0] : h[0], sy[k] < 0 ? -h[1] : h[1], sz[k] < 0 ? -h[2] : h[2]);
        v3 wc = np_point(box, corner);
        float dist = vdot(vsub(wc, pp), n);
        if (dist < min_dist) { min_dist = dist; dc = corner; dw = wc; }
    }
    if (min_dist >= 0.0f) return 0;
    return np_emit(out, dw, n, -min_dist, dc, V(0.0f, 0.0f, 0.0f));
}

/* testAxis, :788-813; returns 0 for a separating axis */
static int np_test_axis(v3 axis, v3 d, const v3* xa, const float* ha, const v3* xb, const float* hb, float* overlap) {
    float proj_a = ha[0] * fabsf(vdot(axis, xa[0])) + ha[1] * fabsf(vdot(axis, xa[1])) + ha[2] * fabsf(vdot(axis, xa[2]));
    float proj_b = hb[0] * fabsf(vdot(axis, xb[0])) + hb[1] * fabsf(vdot(axis, xb[1])) + hb[2] * fabsf(vdot(axis, xb[2]));
    float dist = fabsf(vdot(d, axis));
    if (dist > proj_a + proj_b) return 0;
    *overlap = proj_a + proj_b - dist;
    return 1;
}

/* boxBox (SAT over 15 axes), :426-512 */
static int np_box_box(v3 pa, const ZoCollider* ba, v3 pb, const ZoCollider* bb, ZoContactResult* out) {
    v3 xa[3] = {np_axis(ba, 1.0f, 0.0f, 0.0f), np_axis(ba, 0.0f, 1.0f, 0.0f), np_axis(ba, 0.0f, 0.0f, 1.0f)};
    v3 xb[3] = {np_axis(bb, 1.0f, 0.0f, 0.0f), np_axis(bb, 0.0f, 1.0f, 0.0f), np_axis(bb, 0.0f, 0.0f, 1.0f)};
    v3 d = vsub(pb, pa);
    float min_overlap = INFINITY, ov;
    v3 best = V(0.0f, 0.0f, 1.0f);
    for (int i = 0; i < 3; ++i) {
        if (!np_test_axis(xa[i], d, xa, ba->size, xb, bb->size, &ov)) return 0;
        if (ov < min_overlap) { min_overlap = ov; best = xa[i]; }
    }
    for (int i = 0; i < 3; ++i) {
        if (!np_test_axis(xb[i], d, xa, ba->size, xb, bb->size, &ov)) return 0;
        if (ov < min_overlap) { min_overlap = ov; best = xb[i]; }
    }
    for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j) {
            v3 edge = vcross(xa[i], xb[j]);
            float len = sqrtf(vdot(edge, edge));
            if (len < ZO_NP_EPS) continue;
            v3 nrm = vscale(edge, 1.0f / len);
            if (!np_test_axis(nrm, d, xa, ba->size, xb, bb->size, &ov)) return 0;
            if (ov < min_overlap) { min_overlap = ov; best = nrm; }
        }
    }
    if (vdot(best, d) < 0.0f) best = vscale(best, -1.0f);
    v3 point = vadd(pa, vscale(d, 0.5f));
    return np_emit(out, point, best, min_overlap, V(0.0f, 0.0f, 0.0f), V(0.0f, 0.0f, 0.0f));
}

/* detectCollision, :28-123 (types 0 sphere, 1 capsule, 2 box, 3 plane) */
int zo_detect_collision(const ZoCollider* a, const ZoCollider* b, ZoContactResult* out) {
    memset(out, 0, sizeof *out);
    v3 pa = np_point(a, ld3(a->local_pos));
    v3 pb = np_point(b, ld3(b->local_pos));
    const uint32_t ta = a->type, tb = b->type;
    int hit = 0;
    if (ta == 0) {
        if (tb == 0) hit = np_sphere_sphere(pa, a->size[0], pb, b->size[0], out);
        else if (tb == 1) hit = np_sphere_capsule(pa, a->size[0], pb, b, out);
        else if (tb == 2) hit = np_sphere_box(pa, a->size[0], b, out);
        else if (tb == 3) hit = np_sphere_plane(pa, a->size[0], b, out);
    } else if (ta == 1) {
        if (tb == 0) { hit = np_sphere_capsule(pb, b->size[0], pa, a, out); if (hit) np_flip(out); }
        else if (tb == 1) hit = np_capsule_capsule(pa, a, pb, b, out);
        else if (tb == 3) hit = np_capsule_plane(pa, a, b, out);
    } else if (ta == 2) {
        if (tb == 0) { hit = np_sphere_box(pb, b->size[0], a, out); if (hit) np_flip(out); }
        else if (tb == 3) hit = np_box_plane(a, b, out);
        else if (tb == 2) hit = np_box_box(pa, a, pb, b, out);
    } else if (ta == 3) {
        if (tb == 0) { hit = np_sphere_plane(pb, b->size[0], a, out); if (hit) np_flip(out); }
        else if (tb == 1) { hit = np_capsule_plane(pb, b, a, out); if (hit) np_flip(out); }
        else if (tb == 2) { hit = np_box_plane(b, a, out); if (hit) np_flip(out); }
    }
    if (!hit) memset(out, 0, sizeof *out);
    return hit;
}

/* detectCollision over n pairs (the CPU baseline of the batched kernel); OpenMP over pairs. */
void zo_detect_collisions(const ZoCollider* a, const ZoCollider* b, uint32_t n, ZoContactResult* out, int nthreads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : zo_default_threads)
#endif
    for (int64_t i = 0; i < (int64_t)n; ++i) zo_detect_collision(&a[i], &b[i], &out[i]);
    (void)nthreads;
}
