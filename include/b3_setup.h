/*
 * b3_setup.h - host-side world construction for the MI355X engine.
 *
 * Scenes are built on the host into ordinary B3World structs, then handed
 * to the engine (b3_engine.h).  The functions keep the reference names and
 * argument meaning so that task code written for the reference (for example
 * examples/pufferlib/puffysics_hover/hover_task.h) builds the same worlds
 * unchanged.  The arithmetic is the same sequence of fp32 operations as the
 * reference's creation path, so a world built here is byte-identical to one
 * built there; each function cites the reference code it stands in for.
 *
 * Header-only and static inline, like the reference: capacities are the
 * includer's B3_MAX_* (see b3_types.h).
 */
#ifndef PUFFYSICS_AMD_B3_SETUP_H
#define PUFFYSICS_AMD_B3_SETUP_H

#include <math.h>
#include <string.h>
#include "b3_types.h"

#define B3S_FN static inline

/* ---- vector / quaternion helpers (src/puffysics/03_math.inl:5-369) ---- */

B3S_FN B3Vec3 b3_v(float x, float y, float z) {
    B3Vec3 r;
    r.x = x; r.y = y; r.z = z;
    return r;
}
B3S_FN B3Vec3 b3_add(B3Vec3 a, B3Vec3 b) { return b3_v(a.x + b.x, a.y + b.y, a.z + b.z); }
B3S_FN B3Vec3 b3_sub(B3Vec3 a, B3Vec3 b) { return b3_v(a.x - b.x, a.y - b.y, a.z - b.z); }
B3S_FN B3Vec3 b3_neg(B3Vec3 a) { return b3_v(-a.x, -a.y, -a.z); }
B3S_FN B3Vec3 b3_mul(B3Vec3 a, float s) { return b3_v(a.x * s, a.y * s, a.z * s); }
B3S_FN B3Vec3 b3_madd(B3Vec3 a, float s, B3Vec3 b) {
    return b3_v(a.x + s * b.x, a.y + s * b.y, a.z + s * b.z);
}
B3S_FN float b3_dot(B3Vec3 a, B3Vec3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
B3S_FN B3Vec3 b3_cross(B3Vec3 a, B3Vec3 b) {
    return b3_v(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
B3S_FN float b3_len2(B3Vec3 a) { return b3_dot(a, a); }
B3S_FN float b3_len(B3Vec3 a) { return sqrtf(b3_len2(a)); }
/* 03_math.inl:73-76: zero vectors normalise to +Y. */
B3S_FN B3Vec3 b3_norm(B3Vec3 a) {
    float l2 = b3_len2(a);
    if (l2 > 0.0f) return b3_mul(a, 1.0f / sqrtf(l2));
    return b3_v(0.0f, 1.0f, 0.0f);
}
B3S_FN float b3_minf(float a, float b) { return a < b ? a : b; }
B3S_FN float b3_maxf(float a, float b) { return a > b ? a : b; }
B3S_FN float b3_clamp(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

B3S_FN B3Quat b3_q(float x, float y, float z, float s) {
    B3Quat q;
    q.v = b3_v(x, y, z);
    q.s = s;
    return q;
}
B3S_FN B3Quat b3_q_id(void) { return b3_q(0.0f, 0.0f, 0.0f, 1.0f); }
B3S_FN float b3_qdot(B3Quat a, B3Quat b) { return b3_dot(a.v, b.v) + a.s * b.s; }
/* 03_math.inl:105-112: non-positive norms give the identity. */
B3S_FN B3Quat b3_qnorm(B3Quat q) {
    float d2 = b3_qdot(q, q);
    if (d2 <= 0.0f) return b3_q_id();
    float k = 1.0f / sqrtf(d2);
    return b3_q(q.v.x * k, q.v.y * k, q.v.z * k, q.s * k);
}
B3S_FN B3Quat b3_qneg(B3Quat q) { return b3_q(-q.v.x, -q.v.y, -q.v.z, -q.s); }
B3S_FN B3Quat b3_qmul(B3Quat a, B3Quat b) {
    B3Quat r;
    r.v = b3_add(b3_add(b3_mul(b.v, a.s), b3_mul(a.v, b.s)), b3_cross(a.v, b.v));
    r.s = a.s * b.s - b3_dot(a.v, b.v);
    return r;
}
/* conj(a) * b, 03_math.inl:273-278 */
B3S_FN B3Quat b3_qinv_mul(B3Quat a, B3Quat b) {
    B3Vec3 t = b3_cross(b.v, a.v);
    t = b3_madd(t, a.s, b.v);
    t = b3_v(t.x - b.s * a.v.x, t.y - b.s * a.v.y, t.z - b.s * a.v.z);
    return b3_q(t.x, t.y, t.z, a.s * b.s + b3_dot(a.v, b.v));
}
B3S_FN B3Vec3 b3_rotate(B3Quat q, B3Vec3 v) {
    B3Vec3 t = b3_mul(b3_cross(q.v, v), 2.0f);
    return b3_add(v, b3_add(b3_mul(t, q.s), b3_cross(q.v, t)));
}
B3S_FN B3Vec3 b3_inv_rotate(B3Quat q, B3Vec3 v) {
    return b3_rotate(b3_q(-q.v.x, -q.v.y, -q.v.z, q.s), v);
}
B3S_FN B3Vec3 b3_xf_point(B3Vec3 p, B3Quat q, B3Vec3 local) {
    return b3_add(p, b3_rotate(q, local));
}
B3S_FN void b3_axes(B3Quat q, B3Vec3* x, B3Vec3* y, B3Vec3* z) {
    *x = b3_rotate(q, b3_v(1.0f, 0.0f, 0.0f));
    *y = b3_rotate(q, b3_v(0.0f, 1.0f, 0.0f));
    *z = b3_rotate(q, b3_v(0.0f, 0.0f, 1.0f));
}
/* R diag(inv) R^T, column by column (03_math.inl:187-198). */
B3S_FN B3Mat3 b3_world_inv_i(B3Quat q, B3Vec3 inv) {
    B3Vec3 c0, c1, c2;
    b3_axes(q, &c0, &c1, &c2);
    B3Mat3 m;
    m.cx = b3_add(b3_add(b3_mul(c0, inv.x * c0.x), b3_mul(c1, inv.y * c1.x)), b3_mul(c2, inv.z * c2.x));
    m.cy = b3_add(b3_add(b3_mul(c0, inv.x * c0.y), b3_mul(c1, inv.y * c1.y)), b3_mul(c2, inv.z * c2.y));
    m.cz = b3_add(b3_add(b3_mul(c0, inv.x * c0.z), b3_mul(c1, inv.y * c1.z)), b3_mul(c2, inv.z * c2.z));
    return m;
}
/* 03_math.inl:240-245 */
B3S_FN B3Vec3 b3_perp(B3Vec3 n) {
    if (fabsf(n.x) >= 0.57735027f) return b3_norm(b3_v(-n.y, n.x, 0.0f));
    return b3_norm(b3_v(0.0f, -n.z, n.y));
}
/* 03_math.inl:321-326 (host libm sinf/cosf, setup only). */
B3S_FN B3Quat b3_q_axis_angle(B3Vec3 axis, float radians) {
    B3Vec3 a = b3_norm(axis);
    float half = 0.5f * radians;
    float s = sinf(half);
    return b3_q(s * a.x, s * a.y, s * a.z, cosf(half));
}
/* Shortest arc from +Z to z (03_math.inl:328-341). */
B3S_FN B3Quat b3_q_from_z(B3Vec3 z) {
    B3Vec3 n = b3_norm(z);
    B3Vec3 from = b3_v(0.0f, 0.0f, 1.0f);
    float d = b3_dot(from, n);
    if (d > 0.999999f) return b3_q_id();
    if (d < -0.999999f) {
        B3Vec3 p = b3_perp(from);
        return b3_q(p.x, p.y, p.z, 0.0f);
    }
    B3Vec3 c = b3_cross(from, n);
    return b3_qnorm(b3_q(c.x, c.y, c.z, 1.0f + d));
}
/* Twist about local Z, 03_math.inl:293-309 with the default libm path. */
B3S_FN float b3_twist(B3Quat q) {
    float t = q.s < 0.0f ? atan2f(-q.v.z, -q.s) : atan2f(q.v.z, q.s);
    return 2.0f * t;
}

/* ---- defaults and world lifecycle (src/puffysics/04_world.inl:5-77) ---- */

B3S_FN B3BodyDef b3_default_body(void) {
    B3BodyDef d;
    memset(&d, 0, sizeof(d));
    d.type = B3_STATIC;
    d.rotation = b3_q_id();
    d.gravity_scale = 1.0f;
    return d;
}
B3S_FN B3ShapeDef b3_default_shape(void) {
    B3ShapeDef d;
    d.density = 1000.0f;
    d.friction = 0.6f;
    d.restitution = 0.0f;
    d.rolling = 0.0f;
    d.category = ~0ull;
    d.mask = ~0ull;
    return d;
}
B3S_FN void b3_world_init(B3World* w) {
    memset(w, 0, sizeof(*w));
    w->gravity = b3_v(0.0f, -10.0f, 0.0f);
    w->contact_hertz = 30.0f;
    w->contact_damping = 10.0f;
    w->contact_speed = 3.0f;
    w->restitution_threshold = 1.0f;
    w->max_linear_speed = 400.0f;
}
B3S_FN int b3_body_capacity(void) { return B3_MAX_BODIES; }
B3S_FN int b3_shape_capacity(void) { return B3_MAX_SHAPES; }
B3S_FN int b3_contact_capacity(void) { return B3_MAX_CONTACTS; }
B3S_FN int b3_joint_capacity(void) { return B3_MAX_JOINTS; }
B3S_FN unsigned long long b3_config_signature(void) { return B3_CONFIG_SIGNATURE; }
B3S_FN int b3_config_matches(unsigned long long sig) { return sig == B3_CONFIG_SIGNATURE; }
B3S_FN void b3_clear_errors(B3World* w) {
    w->body_overflow = 0;
    w->shape_overflow = 0;
    w->joint_overflow = 0;
    w->contact_overflow = 0;
    w->contacts_dropped = 0;
}
B3S_FN int b3_world_error(const B3World* w) {
    return w->body_overflow || w->shape_overflow || w->joint_overflow || w->contact_overflow;
}
B3S_FN int b3_step_stats(const B3World* w, B3StepStats* out) {
    out->body_count = w->body_count;
    out->shape_count = w->shape_count;
    out->contact_count = w->contact_count;
    out->joint_count = w->joint_count;
    out->body_overflow = w->body_overflow;
    out->shape_overflow = w->shape_overflow;
    out->joint_overflow = w->joint_overflow;
    out->contact_overflow = w->contact_overflow;
    out->contacts_dropped = w->contacts_dropped;
    return b3_world_error(w);
}

/* ---- bodies and shapes (04_world.inl:79-169) ---- */

B3S_FN int b3_create_body(B3World* w, const B3BodyDef* def) {
    if (w->body_count >= B3_MAX_BODIES) {
        w->body_overflow = 1;
        return -1;
    }
    int id = w->body_count++;
    B3Body* b = &w->bodies[id];
    memset(b, 0, sizeof(*b));
    b->position = def->position;
    b->center = def->position;
    b->rotation = b3_qnorm(def->rotation);
    b->lin_vel = def->lin_vel;
    b->ang_vel = def->ang_vel;
    b->delta_rot = b3_q_id();
    b->linear_damping = def->linear_damping;
    b->angular_damping = def->angular_damping;
    b->gravity_scale = def->gravity_scale;
    b->type = def->type;
    b->flags = def->flags | (def->type == B3_DYNAMIC ? B3_FLAG_DYNAMIC : 0u);
    return id;
}

B3S_FN int b3_add_shape(B3World* w, int body, int type, B3Vec3 local_pos,
        B3Quat local_rot, float radius, B3Vec3 half, const B3ShapeDef* def) {
    if (w->shape_count >= B3_MAX_SHAPES || body < 0 || body >= w->body_count
            || type < B3_SPHERE || type > B3_BOX) {
        w->shape_overflow = 1;
        return -1;
    }
    int id = w->shape_count++;
    B3Shape* s = &w->shapes[id];
    s->body = body;
    s->type = type;
    s->local_pos = local_pos;
    s->local_rot = b3_qnorm(local_rot);
    s->radius = radius;
    s->half = half;
    s->friction = def->friction;
    s->restitution = def->restitution;
    s->rolling = def->rolling;
    s->density = def->density;
    s->category = def->category;
    s->mask = def->mask;
    return id;
}
B3S_FN int b3_create_sphere(B3World* w, int body, B3Vec3 c, float r, const B3ShapeDef* def) {
    return b3_add_shape(w, body, B3_SPHERE, c, b3_q_id(), r, b3_v(0.0f, 0.0f, 0.0f), def);
}
/* Capsule axis is local Y with half length half.y. */
B3S_FN int b3_create_capsule(B3World* w, int body, float half_len, float r, const B3ShapeDef* def) {
    return b3_add_shape(w, body, B3_CAPSULE, b3_v(0.0f, 0.0f, 0.0f), b3_q_id(), r,
        b3_v(0.0f, half_len, 0.0f), def);
}
B3S_FN int b3_create_box(B3World* w, int body, B3Vec3 half, const B3ShapeDef* def) {
    return b3_add_shape(w, body, B3_BOX, b3_v(0.0f, 0.0f, 0.0f), b3_q_id(), 0.0f, half, def);
}
B3S_FN int b3_create_box_local(B3World* w, int body, B3Vec3 half, B3Vec3 local_pos,
        B3Quat local_rot, const B3ShapeDef* def) {
    return b3_add_shape(w, body, B3_BOX, local_pos, local_rot, 0.0f, half, def);
}

/* ---- mass properties (04_world.inl:171-291) ---- */

B3S_FN void b3__store_inv_mass(B3Body* b, float inv_mass, B3Vec3 inertia) {
    b->inv_mass = inv_mass;
    b->inv_inertia.x = inertia.x > 0.0f ? 1.0f / inertia.x : 0.0f;
    b->inv_inertia.y = inertia.y > 0.0f ? 1.0f / inertia.y : 0.0f;
    b->inv_inertia.z = inertia.z > 0.0f ? 1.0f / inertia.z : 0.0f;
    b->inv_i_world = b3_world_inv_i(b->rotation, b->inv_inertia);
}
B3S_FN void b3_set_inertial(B3World* w, int body, float mass, B3Vec3 local_com, B3Vec3 inertia) {
    B3Body* b = &w->bodies[body];
    b->local_center = local_com;
    b->center = b3_xf_point(b->position, b->rotation, local_com);
    if (b->type != B3_DYNAMIC || mass <= 0.0f) {
        b3__store_inv_mass(b, 0.0f, b3_v(0.0f, 0.0f, 0.0f));
        return;
    }
    b3__store_inv_mass(b, 1.0f / mass, inertia);
}
/* Solid sphere, box, and capsule (cylinder plus two hemispheres along Y). */
B3S_FN void b3_shape_mass(const B3Shape* s, float* mass, B3Vec3* com, B3Vec3* inertia) {
    *com = s->local_pos;
    if (s->type == B3_SPHERE) {
        float r = s->radius;
        float m = (4.0f / 3.0f) * B3_PI * r * r * r * s->density;
        float i = 0.4f * m * r * r;
        *mass = m;
        *inertia = b3_v(i, i, i);
    } else if (s->type == B3_BOX) {
        float hx = s->half.x, hy = s->half.y, hz = s->half.z;
        float m = 8.0f * hx * hy * hz * s->density;
        *mass = m;
        *inertia = b3_v((m / 3.0f) * (hy * hy + hz * hz), (m / 3.0f) * (hx * hx + hz * hz),
            (m / 3.0f) * (hx * hx + hy * hy));
    } else {
        float r = s->radius;
        float len = 2.0f * s->half.y;
        float cyl_m = B3_PI * r * r * len * s->density;
        float sph_m = (4.0f / 3.0f) * B3_PI * r * r * r * s->density;
        float axial = 0.5f * cyl_m * r * r + 0.4f * sph_m * r * r;
        float across = (1.0f / 12.0f) * cyl_m * (3.0f * r * r + len * len)
            + 0.4f * sph_m * r * r + 0.125f * sph_m * (3.0f * r + 2.0f * len) * len;
        *mass = cyl_m + sph_m;
        *inertia = b3_v(across, axial, across);
    }
}
/* Mass, COM and rotation-aware diagonal inertia from shape densities. */
B3S_FN void b3_finalize_mass(B3World* w, int body) {
    B3Body* b = &w->bodies[body];
    if (b->type != B3_DYNAMIC) {
        b3__store_inv_mass(b, 0.0f, b3_v(0.0f, 0.0f, 0.0f));
        b->center = b->position;
        return;
    }
    float mass = 0.0f;
    B3Vec3 com = b3_v(0.0f, 0.0f, 0.0f);
    for (int i = 0; i < w->shape_count; i++) {
        const B3Shape* s = &w->shapes[i];
        if (s->body != body || s->density <= 0.0f) continue;
        float sm;
        B3Vec3 sc, si;
        b3_shape_mass(s, &sm, &sc, &si);
        mass += sm;
        com = b3_madd(com, sm, sc);
    }
    if (mass <= 0.0f) {
        b->inv_mass = 0.0f;
        b->inv_inertia = b3_v(0.0f, 0.0f, 0.0f);
        return;
    }
    com = b3_mul(com, 1.0f / mass);
    b->local_center = com;
    b->center = b3_xf_point(b->position, b->rotation, com);
    B3Vec3 diag = b3_v(0.0f, 0.0f, 0.0f);
    for (int i = 0; i < w->shape_count; i++) {
        const B3Shape* s = &w->shapes[i];
        if (s->body != body || s->density <= 0.0f) continue;
        float sm;
        B3Vec3 sc, si, ex, ey, ez;
        b3_shape_mass(s, &sm, &sc, &si);
        b3_axes(s->local_rot, &ex, &ey, &ez);
        B3Vec3 d = b3_sub(sc, com);
        float d2 = b3_dot(d, d);
        diag.x += si.x * ex.x * ex.x + si.y * ey.x * ey.x + si.z * ez.x * ez.x + sm * (d2 - d.x * d.x);
        diag.y += si.x * ex.y * ex.y + si.y * ey.y * ey.y + si.z * ez.y * ez.y + sm * (d2 - d.y * d.y);
        diag.z += si.x * ex.z * ex.z + si.y * ey.z * ey.z + si.z * ez.z * ez.z + sm * (d2 - d.z * d.z);
    }
    b3__store_inv_mass(b, 1.0f / mass, diag);
}

/* ---- joints (src/puffysics/06_joints.inl:5-159) ---- */

B3S_FN B3Joint* b3_add_joint(B3World* w, int type, int body_a, int body_b, B3Vec3 anchor_a,
        B3Vec3 anchor_b, B3Quat rot_a, B3Quat rot_b) {
    if (w->joint_count >= B3_MAX_JOINTS || body_a < 0 || body_a >= w->body_count
            || body_b < 0 || body_b >= w->body_count) {
        w->joint_overflow = 1;
        return NULL;
    }
    B3Joint* j = &w->joints[w->joint_count++];
    memset(j, 0, sizeof(*j));
    j->type = type;
    j->body_a = body_a;
    j->body_b = body_b;
    j->local_anchor_a = anchor_a;
    j->local_anchor_b = anchor_b;
    j->local_rot_a = b3_qnorm(rot_a);
    j->local_rot_b = b3_qnorm(rot_b);
    j->constraint_hertz = 90.0f;
    j->constraint_damping = 2.0f;
    return j;
}
B3S_FN int b3_create_weld(B3World* w, int body_a, int body_b, B3Vec3 anchor_a, B3Vec3 anchor_b) {
    if (body_a < 0 || body_a >= w->body_count || body_b < 0 || body_b >= w->body_count) {
        w->joint_overflow = 1;
        return -1;
    }
    B3Quat rot_b = b3_qinv_mul(w->bodies[body_b].rotation, w->bodies[body_a].rotation);
    B3Joint* j = b3_add_joint(w, B3_JOINT_WELD, body_a, body_b, anchor_a, anchor_b, b3_q_id(), rot_b);
    return j ? (int)(j - w->joints) : -1;
}
/* Hinge about local_axis_a of body A; angle zero at creation. */
B3S_FN int b3_create_revolute(B3World* w, int body_a, int body_b, B3Vec3 anchor_a,
        B3Vec3 anchor_b, B3Vec3 local_axis_a) {
    if (body_a < 0 || body_a >= w->body_count || body_b < 0 || body_b >= w->body_count) {
        w->joint_overflow = 1;
        return -1;
    }
    B3Quat rot_a = b3_q_from_z(local_axis_a);
    B3Quat frame = b3_qmul(w->bodies[body_a].rotation, rot_a);
    B3Quat rot_b = b3_qinv_mul(w->bodies[body_b].rotation, frame);
    B3Joint* j = b3_add_joint(w, B3_JOINT_REVOLUTE, body_a, body_b, anchor_a, anchor_b, rot_a, rot_b);
    return j ? (int)(j - w->joints) : -1;
}
B3S_FN void b3_joint_enable_motor(B3World* w, int joint, int enable) {
    B3Joint* j = &w->joints[joint];
    if (j->enable_motor != enable) j->motor_impulse = 0.0f;
    j->enable_motor = enable;
}
B3S_FN void b3_joint_set_motor(B3World* w, int joint, float speed, float max_torque) {
    w->joints[joint].motor_speed = speed;
    w->joints[joint].max_motor_torque = b3_maxf(max_torque, 0.0f);
}
B3S_FN void b3_joint_enable_limit(B3World* w, int joint, int enable) {
    B3Joint* j = &w->joints[joint];
    if (j->enable_limit != enable) {
        j->lower_impulse = 0.0f;
        j->upper_impulse = 0.0f;
    }
    j->enable_limit = enable;
}
B3S_FN void b3_joint_set_limits(B3World* w, int joint, float lower, float upper) {
    float lim = 0.99f * B3_PI;
    w->joints[joint].lower_angle = b3_clamp(b3_minf(lower, upper), -lim, lim);
    w->joints[joint].upper_angle = b3_clamp(b3_maxf(lower, upper), -lim, lim);
}
B3S_FN void b3_joint_enable_spring(B3World* w, int joint, int enable) {
    B3Joint* j = &w->joints[joint];
    if (j->enable_spring != enable) j->spring_impulse = 0.0f;
    j->enable_spring = enable;
}
B3S_FN void b3_joint_set_spring(B3World* w, int joint, float target, float hertz, float damping) {
    B3Joint* j = &w->joints[joint];
    j->target_angle = b3_clamp(target, -B3_PI, B3_PI);
    j->hertz = b3_maxf(hertz, 0.0f);
    j->damping_ratio = b3_maxf(damping, 0.0f);
}
B3S_FN float b3_joint_angle(const B3World* w, int joint) {
    const B3Joint* j = &w->joints[joint];
    B3Quat qa = b3_qmul(w->bodies[j->body_a].rotation, j->local_rot_a);
    B3Quat qb = b3_qmul(w->bodies[j->body_b].rotation, j->local_rot_b);
    if (b3_qdot(qa, qb) < 0.0f) qb = b3_qneg(qb);
    return b3_twist(b3_qinv_mul(qa, qb));
}
B3S_FN float b3_joint_speed(const B3World* w, int joint) {
    const B3Joint* j = &w->joints[joint];
    B3Vec3 axis = b3_rotate(b3_qmul(w->bodies[j->body_a].rotation, j->local_rot_a),
        b3_v(0.0f, 0.0f, 1.0f));
    return b3_dot(b3_sub(w->bodies[j->body_b].ang_vel, w->bodies[j->body_a].ang_vel), axis);
}

/* ---- host-side force accumulation (src/puffysics/09_step.inl:132-146) ---- */

B3S_FN void b3_apply_force(B3World* w, int body, B3Vec3 force) {
    w->bodies[body].force = b3_add(w->bodies[body].force, force);
}
B3S_FN void b3_apply_torque(B3World* w, int body, B3Vec3 torque) {
    w->bodies[body].torque = b3_add(w->bodies[body].torque, torque);
}
B3S_FN void b3_apply_linear_impulse(B3World* w, int body, B3Vec3 impulse) {
    B3Body* b = &w->bodies[body];
    if (b->type == B3_DYNAMIC) b->lin_vel = b3_madd(b->lin_vel, b->inv_mass, impulse);
}

/* ---- the CPU step (09_step.inl:262-264, b3_batch.cuh:39-48) ----
 * b3_step and b3_batch_step with the reference's names and meaning, for
 * host code such as a CPU environment step (puffysics_hover.h:38-56): the
 * engine's step built for the host, run in place on the caller's structs
 * (libb3engine.so, b3_host_step / b3_host_batch_step, given the caller's
 * B3_CONFIG_SIGNATURE).  b3_step returns without stepping for dt <= 0 (as
 * the reference) or a world whose counts or indices are out of range.
 * b3_batch_step returns 1, or 0 without touching any world when the batch,
 * dt (finite, >= 0), substeps (>= 1) or a selected world is invalid; dt == 0
 * is a successful no-op; active NULL steps every world. */
#ifdef __cplusplus
extern "C" {
#endif
void b3_host_step(void* world, unsigned long long config_signature, float dt, int substeps);
int b3_host_batch_step(B3Batch batch, unsigned long long config_signature, float dt, int substeps,
    const unsigned char* active);
#ifdef __cplusplus
}
#endif
B3S_FN void b3_step(B3World* w, float dt, int substeps) { b3_host_step(w, B3_CONFIG_SIGNATURE, dt, substeps); }
B3S_FN int b3_batch_step(B3Batch batch, float dt, int substeps, const unsigned char* active) {
    return b3_host_batch_step(batch, B3_CONFIG_SIGNATURE, dt, substeps, active);
}

/* ---- batch views (b3_batch.cuh:21-60) ---- */

B3S_FN int b3_batch_valid(B3Batch batch) {
    if (batch.count < 0) return 0;
    if (batch.count == 0) return 1;
    return batch.data != NULL && batch.stride >= sizeof(B3World)
        && batch.world_offset <= batch.stride - sizeof(B3World)
        && (size_t)batch.count <= SIZE_MAX / batch.stride;
}
B3S_FN B3World* b3_batch_world(B3Batch batch, int index) {
    return (B3World*)((unsigned char*)batch.data + (size_t)index * batch.stride + batch.world_offset);
}
/* Host copy of whole worlds from contiguous snapshots where reset[i] != 0. */
B3S_FN int b3_batch_restore(B3Batch batch, const B3World* initial, const unsigned char* reset) {
    if (!b3_batch_valid(batch) || (batch.count && !initial)) return 0;
    for (int i = 0; i < batch.count; i++)
        if (!reset || reset[i]) memcpy(b3_batch_world(batch, i), &initial[i], sizeof(B3World));
    return 1;
}

#undef B3S_FN
#endif /* PUFFYSICS_AMD_B3_SETUP_H */
