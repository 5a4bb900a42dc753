"""Mutation check of the oracle pins: each plausible misreading of the reference, planted in a
copy of the oracle's C source, must make at least one of the oracle-pinning CPU test files
fail. A misreading that survives marks a behaviour no pin covers, and the GPU kernel, which
equals the oracle bit for bit, would share it unseen.

Every mutant is compiled into a temporary directory and the pin files run in a child pytest
with ZENO_ORACLE_LIB pointing at it; the children run a few at a time. The unmutated copy
must pass the same run, so a failure is the mutation's doing.
"""
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "oracle" / "zeno_oracle.c"
PINS = ["tests/test_oracle.py", "tests/test_model.py", "tests/test_hash.py", "tests/test_contact_solve.py",
        "tests/test_oracle_pins.py", "tests/test_narrow_ext.py", "tests/test_ext_contacts.py"]

# The two builders of constraint templates (the product's and the oracle's) are compared with
# each other outside this check; here they are left out, so that a mutant of the oracle's
# builder must be caught by a pin of what the templates hold.
DESELECT = ["--deselect", "tests/test_oracle.py::test_template_builders_agree"]

# (name, original text, mutated text, occurrences); the original must occur exactly that many
# times in the source, and every occurrence is replaced. Leading whitespace picks one site
# where the same line appears at two depths.
MUTANTS = [
    # contact solve (all_shaders.metal:1644-1793)
    ("friction sign of body a",
     "st3(Va, vsub(ld3(Va), vscale(impulse_t, inv_mass_a)));",
     "st3(Va, vadd(ld3(Va), vscale(impulse_t, inv_mass_a)));", 1),
    ("friction sign of body b",
     "st3(Vb, vadd(ld3(Vb), vscale(impulse_t, inv_mass_b)));",
     "st3(Vb, vsub(ld3(Vb), vscale(impulse_t, inv_mass_b)));", 1),
    ("friction cone clamp min -> max",
     "float j_t = fminf(j_t_desired, j_t_max);",
     "float j_t = fmaxf(j_t_desired, j_t_max);", 1),
    ("friction cone without the stored impulse",
     "float j_n_acc = e->con[s].impulses[0] + j_n;",
     "float j_n_acc = j_n;", 1),
    ("stored impulse is the running sum",
     "    e->con[s].impulses[0] = j_n;\n}",
     "    e->con[s].impulses[0] = j_n_acc;\n}", 1),
    ("restitution threshold sign",
     "float vel_restitution = vel_normal < -0.5f ? restitution * vel_normal : 0.0f;",
     "float vel_restitution = vel_normal > -0.5f ? restitution * vel_normal : 0.0f;", 1),
    ("restitution dropped",
     "float j_n = (-(vel_normal + vel_restitution) + bias) / w_normal;",
     "float j_n = (-(vel_normal) + bias) / w_normal;", 1),
    # warm start and sensors (:1408-1444, 1838-1858)
    ("warm start factor 0.8 -> 0.5",
     "e->cs[i].state[0] = 0.8f * e->cs[i].state[1];",
     "e->cs[i].state[0] = 0.5f * e->cs[i].state[1];", 1),
    ("accelerometer rotates by q instead of its conjugate",
     "v3 lg = qrot(V(m->gravity[0], m->gravity[1], m->gravity[2]), qconj(q));",
     "v3 lg = qrot(V(m->gravity[0], m->gravity[1], m->gravity[2]), q);", 1),
    ("gyro reads the linear velocity",
     "case 3: case 10: { const float* w = P4(e->angvel, obj);",
     "case 3: case 10: { const float* w = P4(e->vel, obj);", 1),
    ("frame position sensor reads the velocity",
     "case 7: { const float* p = P4(e->pos, obj);",
     "case 7: { const float* p = P4(e->vel, obj);", 1),
    ("frame linear-velocity sensor reads the position",
     "case 9: { const float* v = P4(e->vel, obj);",
     "case 9: { const float* v = P4(e->pos, obj);", 1),
    # compute_forces (:345-388)
    ("gravity torque: cross product order swapped",
     "v3 t = vcross(com_world, force);",
     "v3 t = vcross(force, com_world);", 1),
    ("gravity torque: COM offset not rotated",
     "v3 com_world = qrot(ld3(e->m->bodies[b].com_offset), ld4(P4(e->quat, b)));",
     "v3 com_world = ld3(e->m->bodies[b].com_offset);", 1),
    # apply_joint_forces (:122-190)
    ("joint force: parent reaction sign flipped",
     "if (a > 0) add3(P4(dst, a), vneg(w));",
     "if (a > 0) add3(P4(dst, a), w);", 1),
    ("joint force: axis rotated by the child",
     "v3 axis_world = qrot(ld3(jt->axis), ld4(P4(e->quat, a)));",
     "v3 axis_world = qrot(ld3(jt->axis), ld4(P4(e->quat, b)));", 1),
    ("joint force: threshold 1e-6 -> 0.1",
     "if (fabsf(f) < 1e-6f) continue;",
     "if (fabsf(f) < 0.1f) continue;", 1),
    # integrate (:394-462)
    ("integrate: linear damping dropped",
     "vel = vscale(vel, 0.999f);", "vel = vel;", 1),
    ("integrate: angular damping dropped",
     "omega = vscale(omega, 0.999f);", "omega = omega;", 1),
    ("integrate: body-frame angular velocity",
     "q4 dq = qmul(Q(h.x, h.y, h.z, 0), quat);",
     "q4 dq = qmul(quat, Q(h.x, h.y, h.z, 0));", 1),
    # broad phase (:468-533) and its hash form (:556-703)
    ("broad phase: margin 0.1 -> 0.2 (both sites)",
     "float min_dist = radius_a + radius_b + 0.1f;",
     "float min_dist = radius_a + radius_b + 0.2f;", 2),
    ("broad phase: margin 0.1 -> 0.2 (hash site only)",
     "                    float min_dist = radius_a + radius_b + 0.1f;",
     "                    float min_dist = radius_a + radius_b + 0.2f;", 1),
    ("broad phase: contype/conaffinity 'or' -> 'and' (both sites)",
     "if ((group_a & mask_b) == 0 && (group_b & mask_a) == 0) continue;",
     "if ((group_a & mask_b) == 0 || (group_b & mask_a) == 0) continue;", 2),
    ("broad phase: same-body pairs kept (both sites)",
     "if (body_a == body_b) continue;", "if (0) continue;", 2),
    # narrow phase (:751-894)
    ("capsule-plane: shallower endpoint chosen",
     "                v3 deepest = d1 < d2 ? p1 : p2;",
     "                v3 deepest = d1 < d2 ? p2 : p1;", 1),
    ("sphere-sphere: contact point ra + pen/2",
     "contact_point = vadd(pos_a, vscale(normal, ra - penetration * 0.5f));",
     "contact_point = vadd(pos_a, vscale(normal, ra + penetration * 0.5f));", 1),
    ("sphere-sphere: normal from b to a",
     "normal = vdivs(diff, dist);", "normal = vneg(vdivs(diff, dist));", 1),
    ("sphere-plane: plane position ignored",
     "float signed_dist = vdot(vsub(sphere_pos, plane_pos), plane_normal);",
     "float signed_dist = vdot(sphere_pos, plane_normal);", 1),
    ("friction: arithmetic mean instead of geometric",
     "float mu = sqrtf(ga->params[2] * gb->params[2]);",
     "float mu = 0.5f * (ga->params[2] + gb->params[2]);", 1),
    # solve_joints (:909-1399)
    ("point constraint: parent COM lever dropped",
     "v3 rc_a = vsub(r_a, qrot(ld3(e->m->bodies[ia].com_offset), quat_a));",
     "v3 rc_a = r_a;", 1),
    ("point constraint: child COM lever dropped",
     "v3 rc_b = vsub(r_b, qrot(ld3(e->m->bodies[ib].com_offset), quat_b));",
     "v3 rc_b = r_b;", 1),
    ("slider: relative-quaternion target not conjugated",
     "        q4 target = Q(c.limits[0], c.limits[1], c.limits[2], c.limits[3]);\n"
     "        q4 qa = ld4(Qa), qb = ld4(Qb);\n"
     "        q4 q_rel = qmul(qconj(qa), qb);\n"
     "        q4 q_err = qmul(q_rel, qconj(target));",
     "        q4 target = Q(c.limits[0], c.limits[1], c.limits[2], c.limits[3]);\n"
     "        q4 qa = ld4(Qa), qb = ld4(Qb);\n"
     "        q4 q_rel = qmul(qconj(qa), qb);\n"
     "        q4 q_err = qmul(q_rel, target);", 1),
    ("weld: relative-quaternion target not conjugated",
     "        q4 target = ld4(c.axis_target);\n"
     "        q4 qa = ld4(Qa), qb = ld4(Qb);\n"
     "        q4 q_rel = qmul(qconj(qa), qb);\n"
     "        q4 q_err = qmul(q_rel, qconj(target));",
     "        q4 target = ld4(c.axis_target);\n"
     "        q4 qa = ld4(Qa), qb = ld4(Qb);\n"
     "        q4 q_rel = qmul(qconj(qa), qb);\n"
     "        q4 q_err = qmul(q_rel, target);", 1),
    # xpbd_update_velocities (:1922-1961)
    ("velocity update: hemisphere flip dropped",
     "if (dq.w < 0) dq = qneg(dq);", "(void)0;", 1),
    # update_joint_states (:1550-1638)
    ("hinge angle: world axis instead of the local one",
     "            float sin_half = vdot(qxyz(q_rel), axis_local);\n"
     "            e->jpos[j] = 2.0f * zo_atan2f(sin_half, q_rel.w);",
     "            float sin_half = vdot(qxyz(q_rel), axis_world_a);\n"
     "            e->jpos[j] = 2.0f * zo_atan2f(sin_half, q_rel.w);", 1),
    ("hinge angle: relative rotation q_b conj(q_a)",
     "q4 q_rel = qmul(qconj(q_a), q_b);", "q4 q_rel = qmul(q_b, qconj(q_a));", 1),
    ("hinge rate: local axis instead of the parent-frame one",
     "e->jvel[j] = vdot(vsub(w_b, w_a), axis_world_a);",
     "e->jvel[j] = vdot(vsub(w_b, w_a), axis_local);", 1),
    ("slide state: child anchor dropped from the position",
     "v3 diff = vsub(vadd(p_b, r_b), vadd(p_a, r_a));",
     "v3 diff = vsub(p_b, vadd(p_a, r_a));", 1),
    ("slide state: child lever dropped from the velocity",
     "v3 v_pt_b = vadd(v_b, vcross(w_b, r_b));", "v3 v_pt_b = v_b;", 1),
    ("slide state: parent lever dropped from the velocity",
     "v3 v_pt_a = vadd(v_a, vcross(w_a, r_a));", "v3 v_pt_a = v_a;", 1),
    # World.step (world.zig:694-792)
    ("accelerations divided by the substep dt",
     "float inv_step = m->timestep > 0 ? 1.0f / m->timestep : 0.0f;",
     "float inv_step = dt > 0 ? 1.0f / dt : 0.0f;", 1),
    ("substep dt not divided by the substep count",
     "float dt = m->timestep / (float)div;", "float dt = m->timestep;", 1),
    ("velocity snapshot taken every substep",
     "        memcpy(pv, e.vel, sizeof(float) * 4 * B);\n"
     "        for (uint32_t k = 0; k < actual; ++k) step_once(&e, act);",
     "        for (uint32_t k = 0; k < actual; ++k) { memcpy(pv, e.vel, sizeof(float) * 4 * B); step_once(&e, act); }", 1),
    # apply_actions (:196-229), apply_joint_forces (:122-190)
    ("actions not clamped to the control range",
     "float ctrl = clampf(actions[a], act->params[1], act->params[2]);", "float ctrl = actions[a];", 1),
    ("torque not clamped to the force range",
     "torque = clampf(torque, act->params2[0], act->params2[1]);", "(void)0;", 1),
    ("slide joints take a torque",
     "float* dst = type == 2 ? e->frc : e->trq;", "float* dst = e->trq;", 1),
    # update_kinematic (:304-339), integrate (:394-462)
    ("kinematic rotation without the half angle",
     "v3 h = vscale(vscale(om, e->dt), 0.5f);", "v3 h = vscale(om, e->dt);", 1),
    ("explicit Euler position (old velocity)",
     "        vel = vadd(vel, vscale(accel, dt));\n"
     "        vel = vscale(vel, 0.999f);\n"
     "        pos = vadd(pos, vscale(vel, dt));",
     "        pos = vadd(pos, vscale(vel, dt));\n"
     "        vel = vadd(vel, vscale(accel, dt));\n"
     "        vel = vscale(vel, 0.999f);", 1),
    ("integration skips the quaternion renormalisation",
     "if (ql > 1e-8f) quat = Q(quat.x / ql, quat.y / ql, quat.z / ql, quat.w / ql);",
     "if (0) quat = Q(quat.x / ql, quat.y / ql, quat.z / ql, quat.w / ql);", 1),
    # broad phase, sort (:711-745), narrow phase, match (:1483-1544)
    ("planes take the distance test",
     "            if (!is_plane_pair) {", "            if (1) {", 1),
    ("sort not stable (equal keys move past each other)",
     "if (j_val <= key_val) break;", "if (j_val < key_val) break;", 1),
    ("sort key of the ordered pair (a, b) instead of (min, max)",
     "uint32_t key_val = (ka << 16) | kb;",
     "uint32_t key_val = (key.indices[0] << 16) | key.indices[1]; (void)ka; (void)kb;", 1),
    ("capsule-plane depth of the shallower endpoint",
     "float dist = fminf(d1, d2);", "float dist = fmaxf(d1, d2);", 1),
    ("contact restitution not stored",
     "c->impulses[3] = m->restitution;", "c->impulses[3] = 0.0f;", 1),
    ("cache match radius inclusive",
     "if (dsq < best) { best = dsq; best_i = (int)i; }", "if (dsq <= best) { best = dsq; best_i = (int)i; }", 1),
    ("cache match scales the normal impulse by 0.9",
     "c->impulses[0] = pc->impulses[0] * 0.8f;", "c->impulses[0] = pc->impulses[0] * 0.9f;", 1),
    # solve_contacts (:1644-1793)
    ("Baumgarte bias without the slop",
     "float bias = beta * fmaxf(penetration - slop, 0.0f) / e->dt;", "float bias = beta * penetration / e->dt;", 1),
    ("position correction without the slop",
     "float pos_correction = beta * fmaxf(penetration - slop, 0.0f);", "float pos_correction = beta * penetration;", 1),
    ("position correction split by the other body's inverse mass",
     "float ratio = inv_mass_a / inv_mass_sum;", "float ratio = inv_mass_b / inv_mass_sum;", 1),
    # solve_joints (:909-1399), lambda (:1427-1444)
    ("lambda not stored for the next warm start",
     "e->cs[i].state[1] = e->cs[i].state[0];", "(void)0;", 1),
    ("hinge alignment with the opposite sign",
     "float d_lambda = -ang_C / (w + alpha_tilde);", "float d_lambda = ang_C / (w + alpha_tilde);", 1),
    ("angular limit violation with the opposite sign",
     "if (angle < lower) violation = lower - angle;", "if (angle < lower) violation = angle - lower;", 1),
    ("linear limit pushes the wrong way",
     "v3 n = violation > 0 ? axis_world : vneg(axis_world);", "v3 n = violation > 0 ? vneg(axis_world) : axis_world;", 1),
    ("weld acts only against a static parent",
     "            if (w_b > 1e-8f) {\n                float d_lambda = (-C) / (w_b + alpha_tilde);",
     "            if (w_b > 1e-8f && inv_mass_a == 0.0f) {\n                float d_lambda = (-C) / (w_b + alpha_tilde);", 1),
    # read_sensors (:1799-1893)
    ("joint position sensor reads the velocity",
     "case 0: o[0] = e->jpos[obj]; break;", "case 0: o[0] = e->jvel[obj]; break;", 1),
    # extended narrow phase: detectCollision and its pairs (narrow_phase.zig:28-512, 786-925)
    ("sphere-sphere: point ra + pen/2",
     "v3 point = vadd(pa, vscale(n, ra - pen * 0.5f));\n    return np_emit",
     "v3 point = vadd(pa, vscale(n, ra + pen * 0.5f));\n    return np_emit", 1),
    ("sphere-sphere: local_b on the far side",
     "float pen = min_dist - dist;\n    v3 point = vadd(pa, vscale(n, ra - pen * 0.5f));\n    return np_emit(out, point, n, pen, vscale(n, ra), vscale(n, -rb));",
     "float pen = min_dist - dist;\n    v3 point = vadd(pa, vscale(n, ra - pen * 0.5f));\n    return np_emit(out, point, n, pen, vscale(n, ra), vscale(n, rb));", 1),
    ("sphere-capsule: point offset by the sphere radius",
     "v3 point = vadd(closest, vscale(n, cr - pen * 0.5f));",
     "v3 point = vadd(closest, vscale(n, sr - pen * 0.5f));", 1),
    ("sphere-capsule: local_a toward the capsule",
     "return np_emit(out, point, n, pen, vscale(n, sr), vscale(n, -cr));",
     "return np_emit(out, point, n, pen, vscale(n, -sr), vscale(n, -cr));", 1),
    ("sphere-plane: plane offset dropped",
     "float signed_dist = vdot(vsub(sp, pp), n) - pl->size[0];",
     "float signed_dist = vdot(vsub(sp, pp), n);", 1),
    ("sphere-plane: point on the far side",
     "v3 point = vsub(sp, vscale(n, signed_dist + pen * 0.5f));",
     "v3 point = vsub(sp, vscale(n, signed_dist - pen * 0.5f));", 1),
    ("sphere-plane: local_a sign",
     "return np_emit(out, point, n, pen, vscale(n, -sr), V(0.0f, 0.0f, 0.0f));",
     "return np_emit(out, point, n, pen, vscale(n, sr), V(0.0f, 0.0f, 0.0f));", 1),
    ("plane point without the geom offset",
     "v3 pp = np_point(pl, ld3(pl->local_pos));",
     "v3 pp = np_point(pl, V(0.0f, 0.0f, 0.0f));", 3),
    ("geom centre without the geom offset",
     "v3 pa = np_point(a, ld3(a->local_pos));\n    v3 pb = np_point(b, ld3(b->local_pos));",
     "v3 pa = V(a->position[0], a->position[1], a->position[2]);\n    v3 pb = V(b->position[0], b->position[1], b->position[2]);", 1),
    ("box face normal: positive face sign",
     "if (dpos > maxd) { maxd = dpos; nrm[0] = nrm[1] = nrm[2] = 0.0f; nrm[i] = 1.0f; }",
     "if (dpos > maxd) { maxd = dpos; nrm[0] = nrm[1] = nrm[2] = 0.0f; nrm[i] = -1.0f; }", 1),
    ("box face normal: nearest face",
     "if (dpos > maxd) { maxd = dpos;",
     "if (dpos < maxd || maxd == -INFINITY) { maxd = dpos;", 1),
    ("sphere-box: point inside the box",
     "v3 point = vadd(wc, vscale(n, pen * 0.5f));",
     "v3 point = vsub(wc, vscale(n, pen * 0.5f));", 1),
    ("sphere-box: local_b without the geom offset",
     "vsub(cl, ld3(box->local_pos))",
     "cl", 1),
    ("sphere-box: sphere rotated by q, not its inverse",
     "v3 r = np_rot(sp, iq);",
     "v3 r = np_rot(sp, q);", 1),
    ("segment point: no clamp",
     "float t = np_clamp(vdot(vsub(p, s), seg) / len_sq, 0.0f, 1.0f);",
     "float t = vdot(vsub(p, s), seg) / len_sq;", 1),
    ("segments: t>1 branch sign",
     "s = np_clamp((b - c) / a, 0.0f, 1.0f);",
     "s = np_clamp((b + c) / a, 0.0f, 1.0f);", 1),
    ("segments: t sign of f",
     "t = (b * s + f) / e;",
     "t = (b * s - f) / e;", 1),
    ("segments: degenerate a sign",
     "t = np_clamp(f / e, 0.0f, 1.0f);",
     "t = np_clamp(-f / e, 0.0f, 1.0f);", 1),
    ("segments: degenerate b sign",
     "        if (e < ZO_NP_EPS) {\n            s = np_clamp(-c / a, 0.0f, 1.0f);",
     "        if (e < ZO_NP_EPS) {\n            s = np_clamp(c / a, 0.0f, 1.0f);", 1),
    ("segments: t<0 branch keeps s",
     "                t = 0.0f;\n                s = np_clamp(-c / a, 0.0f, 1.0f);",
     "                t = 0.0f;", 1),
    ("segments: parallel s = 1",
     "if (denom != 0.0f) s = np_clamp((b * f - c * e) / denom, 0.0f, 1.0f);",
     "s = denom != 0.0f ? np_clamp((b * f - c * e) / denom, 0.0f, 1.0f) : 1.0f;", 1),
    ("capsule-capsule: point b on the far side",
     "v3 wb = vsub(qb, vscale(n, rb));",
     "v3 wb = vadd(qb, vscale(n, rb));", 1),
    ("capsule-plane: point below by dist/2 - radius",
     "v3 point = vsub(deepest, vscale(n, dist * 0.5f + radius));",
     "v3 point = vsub(deepest, vscale(n, dist * 0.5f - radius));", 1),
    ("capsule-plane: local_a sign",
     "return np_emit(out, point, n, -dist, vscale(n, -radius), V(0.0f, 0.0f, 0.0f));",
     "return np_emit(out, point, n, -dist, vscale(n, radius), V(0.0f, 0.0f, 0.0f));", 1),
    ("capsule-plane: shallower endpoint",
     "v3 deepest = d1 < d2 ? p1 : p2;\n    float dist = np_min(d1, d2);",
     "v3 deepest = d1 < d2 ? p2 : p1;\n    float dist = np_min(d1, d2);", 1),
    ("box-plane: local_a in world frame",
     "return np_emit(out, dw, n, -min_dist, dc,",
     "return np_emit(out, dw, n, -min_dist, dw,", 1),
    ("box-plane: point at the midpoint",
     "return np_emit(out, dw, n, -min_dist, dc,",
     "return np_emit(out, vsub(dw, vscale(n, min_dist * 0.5f)), n, -min_dist, dc,", 1),
    ("box-plane: plane offset applied",
     "float dist = vdot(vsub(wc, pp), n);",
     "float dist = vdot(vsub(wc, pp), n) - pl->size[0];", 1),
    ("box-box: normal toward a",
     "if (vdot(best, d) < 0.0f) best",
     "if (vdot(best, d) > 0.0f) best", 1),
    ("box-box: edge axes skipped",
     "if (len < ZO_NP_EPS) continue;",
     "continue;", 1),
    ("box-box: point at a's centre",
     "v3 point = vadd(pa, vscale(d, 0.5f));",
     "v3 point = pa;", 1),
    ("box-box: projection with b's half-extents for a",
     "float proj_a = ha[0] * fabsf(vdot(axis, xa[0]))",
     "float proj_a = hb[0] * fabsf(vdot(axis, xa[0]))", 1),
    ("flip: locals not swapped",
     "float t = r->local_a[i]; r->local_a[i] = r->local_b[i]; r->local_b[i] = t;",
     "", 1),
    ("dispatch: box-sphere not flipped",
     "hit = np_sphere_box(pb, b->size[0], a, out); if (hit) np_flip(out);",
     "hit = np_sphere_box(pb, b->size[0], a, out);", 1),
    ("dispatch: plane-capsule not flipped",
     "hit = np_capsule_plane(pb, b, a, out); if (hit) np_flip(out);",
     "hit = np_capsule_plane(pb, b, a, out);", 1),
    ("rotation: conjugate quaternion",
     "v3 qv = V(q[0], q[1], q[2]);\n    v3 uv = vcross(qv, v);",
     "v3 qv = V(-q[0], -q[1], -q[2]);\n    v3 uv = vcross(qv, v);", 1),
    # constraint templates and colouring (joint.zig:202-350, world.zig:311-501, xpbd.zig:533-640)
    ("weld target conj(q_c) q_p",
     "tmpl(c, a, b, 7);\n                st3(c->anchor_a, ap); st3(c->anchor_b, ac);\n                st4(c->axis_target, qmul(qconj(qa), qb));",
     "tmpl(c, a, b, 7);\n                st3(c->anchor_a, ap); st3(c->anchor_b, ac);\n                st4(c->axis_target, qmul(qconj(qb), qa));", 1),
    ("weld anchors swapped",
     "tmpl(c, a, b, 7);\n                st3(c->anchor_a, ap); st3(c->anchor_b, ac);",
     "tmpl(c, a, b, 7);\n                st3(c->anchor_a, ac); st3(c->anchor_b, ap);", 1),
    ("revolute point anchors swapped",
     "c = &out[n++]; tmpl(c, a, b, 2);\n                st3(c->anchor_a, ap); st3(c->anchor_b, ac);\n                c = &out[n++]; tmpl(c, a, b, 3);\n                v3 axb",
     "c = &out[n++]; tmpl(c, a, b, 2);\n                st3(c->anchor_a, ac); st3(c->anchor_b, ap);\n                c = &out[n++]; tmpl(c, a, b, 3);\n                v3 axb", 1),
    ("hinge child axis without the parent rotation",
     "v3 axb = host_rot(host_rot(ax, qa), qconj(qb));",
     "v3 axb = host_rot(ax, qconj(qb));", 1),
    ("hinge child axis left in the world frame",
     "v3 axb = host_rot(host_rot(ax, qa), qconj(qb));",
     "v3 axb = host_rot(ax, qa);", 1),
    ("hinge damping not stored",
     "st3(c->anchor_a, ax); st3(c->anchor_b, axb); c->anchor_b[3] = damping;",
     "st3(c->anchor_a, ax); st3(c->anchor_b, axb);", 1),
    ("angular limit axis in the child frame",
     "c = &out[n++]; tmpl(c, a, b, 4);\n                    st3(c->anchor_a, ax); c->limits[0] = lower;",
     "c = &out[n++]; tmpl(c, a, b, 4);\n                    st3(c->anchor_a, axb); c->limits[0] = lower;", 1),
    ("angular limit bounds swapped",
     "st3(c->anchor_a, ax); c->limits[0] = lower; c->limits[1] = upper;\n                }\n                break;\n            }\n            case 2:",
     "st3(c->anchor_a, ax); c->limits[0] = upper; c->limits[1] = lower;\n                }\n                break;\n            }\n            case 2:", 1),
    ("limit when lower == upper",
     "int has_limits = limited[j] && lower < upper;",
     "int has_limits = limited[j] && lower <= upper;", 1),
    ("slider target conj(q_c) q_p",
     "st4(c->limits, qmul(qconj(qa), qb));",
     "st4(c->limits, qmul(qconj(qb), qa));", 1),
    ("slider damping not stored",
     "st3(c->anchor_a, ap); st3(c->anchor_b, ac); c->anchor_b[3] = damping;",
     "st3(c->anchor_a, ap); st3(c->anchor_b, ac);", 1),
    ("slider axis rotated to the world",
     "st3(c->axis_target, ax);",
     "st3(c->axis_target, host_rot(ax, qa));", 1),
    ("linear limit on the parent anchor",
     "st3(c->anchor_a, ax); st3(c->anchor_b, ac);\n                    c->limits[0] = lower;",
     "st3(c->anchor_a, ax); st3(c->anchor_b, ap);\n                    c->limits[0] = lower;", 1),
    ("ball cone limit (lower, upper)",
     "c->limits[0] = -upper; c->limits[1] = upper;",
     "c->limits[0] = lower; c->limits[1] = upper;", 1),
    ("universal second axis x",
     "v3 ax2 = V(0, 1, 0);",
     "v3 ax2 = V(1, 0, 0);", 1),
    ("universal second hinge in the parent frame",
     "st3(c->anchor_a, ax2); st3(c->anchor_b, host_rot(host_rot(ax2, qa), qconj(qb)));",
     "st3(c->anchor_a, ax2); st3(c->anchor_b, ax2);", 1),
    ("colouring ignores the world body",
     "if (a < num_bodies && (ka == a || kb == a)) shares = 1;",
     "if (a > 0 && a < num_bodies && (ka == a || kb == a)) shares = 1;", 1),
    ("colour sort descending",
     "while (j >= 0 && ((out[j].indices[3] >> 8) & 0xFF) > kc)",
     "while (j >= 0 && ((out[j].indices[3] >> 8) & 0xFF) < kc)", 1),
    ("colour sort unstable",
     "while (j >= 0 && ((out[j].indices[3] >> 8) & 0xFF) > kc)",
     "while (j >= 0 && ((out[j].indices[3] >> 8) & 0xFF) >= kc)", 1),
    ("colour takes the largest used + 1",
     "while (col < 255 && used[col]) ++col;",
     "for (uint32_t u = 0; u < 255; ++u) if (used[u]) col = u + 1;", 1),
    ("host rotation by the conjugate",
     "float t0 = 2.0f * (q.y * v.z - q.z * v.y);\n    float t1 = 2.0f * (q.z * v.x - q.x * v.z);\n    float t2 = 2.0f * (q.x * v.y - q.y * v.x);\n    return V(v.x + q.w * t0",
     "float t0 = 2.0f * (q.y * v.z - q.z * v.y);\n    float t1 = 2.0f * (q.z * v.x - q.x * v.z);\n    float t2 = 2.0f * (q.x * v.y - q.y * v.x);\n    return V(v.x - q.w * t0", 1),
    # spatial-hash broad phase (all_shaders.metal:556-703, world.zig:534)
    ("hash threshold >= 512",
     "if (e->m->num_geoms > ZO_HASH_MIN_GEOMS)",
     "if (e->m->num_geoms >= ZO_HASH_MIN_GEOMS)", 1),
    ("hash cell by ceil",
     "float f = floorf(p * 1.0f);",
     "float f = ceilf(p * 1.0f);", 1),
    ("hash NaN in the last cell",
     "if (!(f >= 0.0f)) return 0u;",
     "if (f != f) return ZO_HASH_DIM - 1u;\n    if (!(f >= 0.0f)) return 0u;", 1),
    ("hash huge coordinates past the last cell",
     "if (f >= (float)(ZO_HASH_DIM - 1u)) return ZO_HASH_DIM - 1u;",
     "if (f >= (float)ZO_HASH_DIM) return ZO_HASH_DIM;", 1),
    ("hash id z-major",
     "uint32_t id = cx[3 * g + 0] + cx[3 * g + 1] * D + cx[3 * g + 2] * D * D;",
     "uint32_t id = cx[3 * g + 2] + cx[3 * g + 1] * D + cx[3 * g + 0] * D * D;", 1),
    ("hash cell without the geom offset",
     "v3 p = vadd(ld3(P4(pos, ga->type_body[1])), ld3(ga->pos_size0));\n        cx[3 * g + 0]",
     "v3 p = ld3(P4(pos, ga->type_body[1]));\n        cx[3 * g + 0]", 1),
    ("hash neighbours one-sided in x",
     "for (int dx = -1; dx <= 1; ++dx)",
     "for (int dx = 0; dx <= 1; ++dx)", 1),
    ("hash loop nesting x outermost",
     "for (int dz = -1; dz <= 1; ++dz) for (int dy = -1; dy <= 1; ++dy) for (int dx = -1; dx <= 1; ++dx) {",
     "for (int dx = -1; dx <= 1; ++dx) for (int dy = -1; dy <= 1; ++dy) for (int dz = -1; dz <= 1; ++dz) {", 1),
    ("hash pairs both ways",
     "if (o <= g) continue;",
     "if (o == g) continue;", 1),
    ("hash same-body pairs kept",
     "                if (body_a == body_b) continue;\n                uint32_t group_b",
     "                uint32_t group_b", 1),
    ("hash mask rule and",
     "if ((group_a & mask_b) == 0 && (group_b & mask_a) == 0) continue;\n                uint32_t type_b",
     "if ((group_a & mask_b) == 0 || (group_b & mask_a) == 0) continue;\n                uint32_t type_b", 1),
    ("hash planes take the distance test",
     "if (!(type_a == 3 || type_b == 3)) {\n                    v3 diff = vsub(pos_b, pos_a);",
     "if (1) {\n                    v3 diff = vsub(pos_b, pos_a);", 1),
    ("hash pair written as (o, g)",
     "                    ct->indices[0] = body_a; ct->indices[1] = body_b; ct->indices[2] = g; ct->indices[3] = o;",
     "                    ct->indices[0] = body_a; ct->indices[1] = body_b; ct->indices[2] = o; ct->indices[3] = g;", 1),
    ("hash count stops at M",
     "uint32_t c = (*count)++;\n                if (c < M) {\n                    ZoContact* ct = &con[c];\n                    ct->indices[0] = body_a; ct->indices[1] = body_b; ct->indices[2] = g;",
     "uint32_t c = *count;\n                if (c < M) {\n                    ++*count;\n                    ZoContact* ct = &con[c];\n                    ct->indices[0] = body_a; ct->indices[1] = body_b; ct->indices[2] = g;", 1),
]


def _build(src_text: str, out: Path) -> None:
    c = out.with_suffix(".c")
    c.write_text(src_text)
    shutil.copy(ROOT / "oracle" / "zeno_oracle.h", out.parent / "zeno_oracle.h")
    r = subprocess.run([shutil.which("gcc"), "-O1", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off",
                        "-fno-fast-math", str(c), "-o", str(out), "-lm"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def _run_pins(lib: Path) -> subprocess.CompletedProcess:
    env = dict(os.environ, ZENO_ORACLE_LIB=str(lib), PYTHONPATH=str(ROOT), OMP_NUM_THREADS="1")
    return subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", *PINS, *DESELECT],
                          cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=600)


def _build_and_run(src_text: str, workdir: Path) -> subprocess.CompletedProcess:
    workdir.mkdir(parents=True, exist_ok=True)
    lib = workdir / "oracle.so"
    _build(src_text, lib)
    return _run_pins(lib)


@pytest.fixture(scope="module")
def results():
    """Runs the unmutated copy and every mutant (up to 6 child processes at a time)."""
    if shutil.which("gcc") is None:
        pytest.skip("gcc is required")
    source = SRC.read_text()
    jobs = {"<unmutated>": source}
    for name, orig, mut, n in MUTANTS:
        assert source.count(orig) == n, f"mutation site for '{name}' found {source.count(orig)} times, not {n}"
        jobs[name] = source.replace(orig, mut)
    with tempfile.TemporaryDirectory() as tmp:
        with ThreadPoolExecutor(max_workers=max(2, min(6, (os.cpu_count() or 4) - 2))) as pool:
            futs = {k: pool.submit(_build_and_run, v, Path(tmp) / f"m{i}") for i, (k, v) in enumerate(jobs.items())}
            yield {k: f.result() for k, f in futs.items()}


def test_unmutated_copy_passes(results):
    r = results["<unmutated>"]
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]


@pytest.mark.parametrize("name", [m[0] for m in MUTANTS])
def test_mutant_is_caught(results, name):
    r = results[name]
    assert r.returncode != 0, f"mutant '{name}' passed every pin test"
    assert "failed" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
