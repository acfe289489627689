/*
 * b3cpu.c - CPU oracle: plain-C restatement of the reference b3_step.
 *
 * TEST INFRASTRUCTURE ONLY (see b3cpu.h).  It exists to check the MI355X
 * engine and to time a CPU baseline; nothing in the engine links it.
 *
 * Every function keeps the reference's fp32 operation order, so when built
 * with -ffp-contract=off (no FMA contraction, no fast-math) its results are
 * bit-identical to the reference's CPU path; tests/test_oracle_golden.py checks
 * exactly that against the reference compiled from its own sources.  The
 * restatement covers the default feature set only (B3_ART_CONTACTS=0, no
 * packed/compact/cached solver experiments, libm twist, normalised-Euler
 * rotation integration).  Each function cites the reference lines it
 * follows.
 *
 * Scalars are `b3r` (float) so that the same source can be re-compiled with
 * an operation-counting scalar type.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "b3cpu.h"
#include "../include/b3_types.h"

#ifndef B3R_TYPE
typedef float b3r;
#define o_sqrt(x) sqrtf(x)
#define o_fabs(x) fabsf(x)
#define o_atan2(y, x) atan2f(y, x)
#define o_isfinite(x) isfinite(x)
#endif

#define O_FN static inline

/* ------------------------------------------------------------------ */
/* Data view: layout-identical mirrors of include/b3_types.h           */
/* ------------------------------------------------------------------ */

typedef struct { b3r x, y, z; } OV3;
typedef struct { b3r x, y; } OV2;
typedef struct { OV3 v; b3r s; } OQ;
typedef struct { OV3 cx, cy, cz; } OM3;
typedef struct { OV2 cx, cy; } OM2;
typedef struct { b3r bias_rate, mass_scale, impulse_scale; } OSoft;
typedef struct { OV3 lo, hi; } OAabb;

typedef struct {
    OV3 position; OQ rotation; OV3 center; OV3 local_center;
    OV3 lin_vel; OV3 ang_vel; OV3 force; OV3 torque;
    OV3 delta_pos; OQ delta_rot; b3r inv_mass; OV3 inv_inertia; OM3 inv_i_world;
    b3r linear_damping; b3r angular_damping; b3r gravity_scale;
    int type; uint32_t flags;
} OBody;

typedef struct {
    int body; int type; OV3 local_pos; OQ local_rot; b3r radius; OV3 half;
    b3r friction; b3r restitution; b3r rolling; b3r density;
    uint64_t category; uint64_t mask;
} OShape;

typedef struct {
    OV3 r_a; OV3 r_b; b3r base_sep; b3r rel_vel; b3r normal_impulse;
    b3r total_normal; b3r normal_mass; b3r lever; uint32_t feature;
} OPoint;

typedef struct {
    int shape_a, shape_b, body_a, body_b, point_count, static_contact;
    OV3 normal, tangent1, tangent2;
    OPoint points[B3_MAX_MANIFOLD];
    OV3 center_a, center_b;
    b3r friction, restitution, rolling, twist_mass, twist_impulse;
    OV2 friction_impulse; OV3 rolling_impulse;
    OM2 tangent_mass; OM3 rolling_mass;
    b3r inv_mass_a, inv_mass_b; OM3 inv_i_a, inv_i_b;
    OSoft softness;
} OContact;

typedef struct {
    int type, body_a, body_b, collide_connected, fixed_rotation;
    OV3 local_anchor_a, local_anchor_b; OQ local_rot_a, local_rot_b;
    b3r constraint_hertz, constraint_damping; OSoft softness;
    b3r inv_mass_a, inv_mass_b; OM3 inv_i_a, inv_i_b;
    OV3 frame_p_a, frame_p_b; OQ frame_q_a, frame_q_b;
    OV3 delta_center, linear_impulse, angular_impulse; OM3 angular_mass;
    b3r linear_hertz, linear_damping, angular_hertz, angular_damping;
    OSoft linear_spring, angular_spring;
    OV2 perp_impulse;
    b3r spring_impulse, motor_impulse, lower_impulse, upper_impulse;
    b3r hertz, damping_ratio, max_motor_torque, motor_speed;
    b3r target_angle, lower_angle, upper_angle;
    int enable_spring, enable_motor, enable_limit;
    OV3 rotation_axis, perp_x, perp_y; b3r axial_mass; OSoft spring_softness;
} OJoint;

typedef struct {
    OV3 gravity; b3r contact_hertz, contact_damping, contact_speed;
    b3r restitution_threshold, max_linear_speed;
    int body_count, shape_count, contact_count, joint_count;
    int body_overflow, shape_overflow, joint_overflow, contact_overflow, contacts_dropped;
} OHdr;

_Static_assert(sizeof(OBody) == sizeof(B3Body), "body layout");
_Static_assert(sizeof(OShape) == sizeof(B3Shape), "shape layout");
_Static_assert(sizeof(OPoint) == sizeof(B3Point), "point layout");
_Static_assert(sizeof(OContact) == sizeof(B3Contact), "contact layout");
_Static_assert(sizeof(OJoint) == sizeof(B3Joint), "joint layout");
_Static_assert(sizeof(OHdr) == sizeof(B3WorldHeader), "header layout");
_Static_assert(offsetof(OJoint, spring_softness) == offsetof(B3Joint, spring_softness), "joint tail");
_Static_assert(offsetof(OContact, softness) == offsetof(B3Contact, softness), "contact tail");

typedef struct {
    OHdr* h;
    OBody* bodies;
    OShape* shapes;
    OContact* contacts;
    OJoint* joints;
    int max_b, max_s, max_c, max_j;
} OWorld;

static int o_view(OWorld* w, void* base, unsigned long long sig) {
    B3Layout L;
    if (!b3_layout_of(sig, &L)) return 0;
    unsigned char* p = (unsigned char*)base;
    w->h = (OHdr*)p;
    w->bodies = (OBody*)(p + L.bodies_off);
    w->shapes = (OShape*)(p + L.shapes_off);
    w->contacts = (OContact*)(p + L.contacts_off);
    w->joints = (OJoint*)(p + L.joints_off);
    w->max_b = L.max_bodies;
    w->max_s = L.max_shapes;
    w->max_c = L.max_contacts;
    w->max_j = L.max_joints;
    return 1;
}

/* ------------------------------------------------------------------ */
/* Math: src/puffysics/03_math.inl                                     */
/* ------------------------------------------------------------------ */

O_FN OV3 o_v(b3r x, b3r y, b3r z) { OV3 r; r.x = x; r.y = y; r.z = z; return r; }      /* :5-11 */
O_FN OV3 o_add(OV3 a, OV3 b) { return o_v(a.x + b.x, a.y + b.y, a.z + b.z); }           /* :13 */
O_FN OV3 o_sub(OV3 a, OV3 b) { return o_v(a.x - b.x, a.y - b.y, a.z - b.z); }           /* :17 */
O_FN OV3 o_neg(OV3 a) { return o_v(-a.x, -a.y, -a.z); }                                 /* :21 */
O_FN OV3 o_scale(OV3 a, b3r s) { return o_v(a.x * s, a.y * s, a.z * s); }               /* :25 */
O_FN OV3 o_madd(OV3 a, b3r s, OV3 b) { return o_v(a.x + s * b.x, a.y + s * b.y, a.z + s * b.z); } /* :29 */
O_FN OV3 o_msub(OV3 a, b3r s, OV3 b) { return o_v(a.x - s * b.x, a.y - s * b.y, a.z - s * b.z); } /* :33 */
O_FN b3r o_dot(OV3 a, OV3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }              /* :37 */
O_FN OV3 o_cross(OV3 a, OV3 b) {                                                         /* :41-45 */
    return o_v(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
O_FN b3r o_len2(OV3 a) { return o_dot(a, a); }
O_FN b3r o_len(OV3 a) { return o_sqrt(o_len2(a)); }
/* default (non-intrinsic) reciprocal square roots, :57-71 */
O_FN b3r o_rsqrt(b3r x) { b3r one = 1.0f; return one / o_sqrt(x); }
O_FN b3r o_rsqrt_scale(b3r a, b3r x) { return a / o_sqrt(x); }
O_FN OV3 o_norm(OV3 a) {                                                                 /* :73-76 */
    b3r l2 = o_len2(a);
    if (l2 > 0.0f) return o_scale(a, o_rsqrt(l2));
    return o_v(0.0f, 1.0f, 0.0f);
}
O_FN b3r o_clamp(b3r x, b3r lo, b3r hi) { return x < lo ? lo : (x > hi ? hi : x); }    /* :78 */
O_FN b3r o_max(b3r a, b3r b) { return a > b ? a : b; }                                  /* :82 */
O_FN b3r o_min(b3r a, b3r b) { return a < b ? a : b; }                                  /* :86 */

O_FN OQ o_q(b3r x, b3r y, b3r z, b3r s) { OQ q; q.v = o_v(x, y, z); q.s = s; return q; }
O_FN OQ o_qid(void) { return o_q(0.0f, 0.0f, 0.0f, 1.0f); }
O_FN b3r o_qdot(OQ a, OQ b) { return o_dot(a.v, b.v) + a.s * b.s; }                    /* :101 */
O_FN OQ o_qnorm(OQ q) {                                                                  /* :105-112 */
    b3r d2 = o_qdot(q, q);
    if (d2 <= 0.0f) return o_qid();
    b3r k = o_rsqrt(d2);
    return o_q(q.v.x * k, q.v.y * k, q.v.z * k, q.s * k);
}
O_FN OQ o_qmul(OQ a, OQ b) {                                                             /* :114-120 */
    OQ r;
    r.v = o_add(o_add(o_scale(b.v, a.s), o_scale(a.v, b.s)), o_cross(a.v, b.v));
    r.s = a.s * b.s - o_dot(a.v, b.v);
    return r;
}
O_FN OV3 o_rot(OQ q, OV3 v) {                                                            /* :122-125 */
    OV3 t = o_scale(o_cross(q.v, v), 2.0f);
    return o_add(v, o_add(o_scale(t, q.s), o_cross(q.v, t)));
}
O_FN OV3 o_invrot(OQ q, OV3 v) { return o_rot(o_q(-q.v.x, -q.v.y, -q.v.z, q.s), v); } /* :127-130 */
/* normalised explicit Euler on the quaternion, :152-157 */
O_FN OQ o_qintegrate(OQ q, OV3 dw) {
    OQ qd = o_q(0.5f * dw.x, 0.5f * dw.y, 0.5f * dw.z, 0.0f);
    qd = o_qmul(qd, q);
    return o_qnorm(o_q(q.v.x + qd.v.x, q.v.y + qd.v.y, q.v.z + qd.v.z, q.s + qd.s));
}
O_FN void o_axes(OQ q, OV3* x, OV3* y, OV3* z) {                                         /* :160-164 */
    *x = o_rot(q, o_v(1.0f, 0.0f, 0.0f));
    *y = o_rot(q, o_v(0.0f, 1.0f, 0.0f));
    *z = o_rot(q, o_v(0.0f, 0.0f, 1.0f));
}
O_FN OV3 o_mv(OM3 m, OV3 v) {                                                            /* :166-169 */
    return o_add(o_add(o_scale(m.cx, v.x), o_scale(m.cy, v.y)), o_scale(m.cz, v.z));
}
O_FN OM3 o_madd3(OM3 a, OM3 b) {                                                         /* :171-177 */
    OM3 r;
    r.cx = o_add(a.cx, b.cx);
    r.cy = o_add(a.cy, b.cy);
    r.cz = o_add(a.cz, b.cz);
    return r;
}
O_FN OM3 o_m0(void) { OM3 m; m.cx = o_v(0.0f, 0.0f, 0.0f); m.cy = m.cx; m.cz = m.cx; return m; }
O_FN OM3 o_world_inv_i(OQ q, OV3 inv) {                                                 /* :187-198 */
    OV3 ax, ay, az;
    o_axes(q, &ax, &ay, &az);
    OM3 r;
    r.cx = o_add(o_add(o_scale(ax, inv.x * ax.x), o_scale(ay, inv.y * ay.x)), o_scale(az, inv.z * az.x));
    r.cy = o_add(o_add(o_scale(ax, inv.x * ax.y), o_scale(ay, inv.y * ay.y)), o_scale(az, inv.z * az.y));
    r.cz = o_add(o_add(o_scale(ax, inv.x * ax.z), o_scale(ay, inv.y * ay.z)), o_scale(az, inv.z * az.z));
    return r;
}
O_FN OM3 o_inv3(OM3 m) {                                                                 /* :200-215 */
    OV3 c0 = o_cross(m.cy, m.cz);
    b3r det = o_dot(m.cx, c0);
    OM3 r = o_m0();
    if (o_fabs(det) < 1.0e-12f) return r;
    b3r one = 1.0f;
    b3r inv = one / det;
    OV3 r0 = o_scale(c0, inv);
    OV3 r1 = o_scale(o_cross(m.cz, m.cx), inv);
    OV3 r2 = o_scale(o_cross(m.cx, m.cy), inv);
    r.cx = o_v(r0.x, r1.x, r2.x);
    r.cy = o_v(r0.y, r1.y, r2.y);
    r.cz = o_v(r0.z, r1.z, r2.z);
    return r;
}
O_FN OM2 o_inv2(OM2 k) {                                                                 /* :217-231 */
    b3r det = k.cx.x * k.cy.y - k.cx.y * k.cy.x;
    OM2 r;
    r.cx.x = 0.0f; r.cx.y = 0.0f; r.cy.x = 0.0f; r.cy.y = 0.0f;
    if (o_fabs(det) < 1.0e-12f) return r;
    b3r one = 1.0f;
    b3r inv = one / det;
    r.cx.x = k.cy.y * inv;
    r.cx.y = -k.cx.y * inv;
    r.cy.x = -k.cy.x * inv;
    r.cy.y = k.cx.x * inv;
    return r;
}
O_FN OV2 o_mv2(OM2 m, OV2 v) {                                                           /* :233-238 */
    OV2 r;
    r.x = m.cx.x * v.x + m.cy.x * v.y;
    r.y = m.cx.y * v.x + m.cy.y * v.y;
    return r;
}
O_FN OV3 o_perp(OV3 n) {                                                                 /* :240-245 */
    if (o_fabs(n.x) >= 0.57735027f) return o_norm(o_v(-n.y, n.x, 0.0f));
    return o_norm(o_v(0.0f, -n.z, n.y));
}
O_FN OSoft o_make_soft(b3r hertz, b3r zeta, b3r h) {                                     /* :247-263 */
    OSoft s;
    s.bias_rate = 0.0f; s.mass_scale = 0.0f; s.impulse_scale = 0.0f;
    if (hertz == 0.0f) return s;
    b3r two_pi = 2.0f * B3_PI;
    b3r omega = two_pi * hertz;
    b3r a1 = 2.0f * zeta + h * omega;
    b3r a2 = h * omega * a1;
    b3r one = 1.0f;
    b3r a3 = one / (1.0f + a2);
    s.bias_rate = omega / a1;
    s.mass_scale = a2 * a3;
    s.impulse_scale = a3;
    return s;
}
O_FN OQ o_qneg(OQ q) { return o_q(-q.v.x, -q.v.y, -q.v.z, -q.s); }                     /* :265 */
O_FN OQ o_qconj(OQ q) { return o_q(-q.v.x, -q.v.y, -q.v.z, q.s); }                     /* :269 */
O_FN OQ o_qinv_mul(OQ a, OQ b) {                                                         /* :273-278 */
    OV3 t = o_cross(b.v, a.v);
    t = o_madd(t, a.s, b.v);
    t = o_msub(t, b.s, a.v);
    return o_q(t.x, t.y, t.z, a.s * b.s + o_dot(a.v, b.v));
}
O_FN b3r o_twist(OQ q) {                                                                 /* :293-309 (libm path) */
    b3r t = q.s < 0.0f ? o_atan2(-q.v.z, -q.s) : o_atan2(q.v.z, q.s);
    return 2.0f * t;
}
O_FN void o_hinge_perps(OQ qa, OQ rel, OV3* px, OV3* py) {                               /* :311-319 */
    OV3 ex = o_v(1.0f, 0.0f, 0.0f);
    OV3 ey = o_v(0.0f, 1.0f, 0.0f);
    *px = o_scale(o_rot(qa, o_add(o_scale(ex, rel.s), o_cross(rel.v, ex))), 0.5f);
    *py = o_scale(o_rot(qa, o_add(o_scale(ey, rel.s), o_cross(rel.v, ey))), 0.5f);
}
O_FN OV3 o_solve3(OM3 a, OV3 b) { return o_mv(o_inv3(a), b); }                          /* :343-345 */
O_FN OV2 o_solve2(OM2 m, OV2 b) {                                                        /* :347-359 */
    b3r det = m.cx.x * m.cy.y - m.cx.y * m.cy.x;
    OV2 r;
    r.x = 0.0f; r.y = 0.0f;
    if (det <= 1.0e-12f) return r;
    b3r one = 1.0f;
    b3r inv = one / det;
    r.x = inv * (m.cy.y * b.x - m.cy.x * b.y);
    r.y = inv * (-m.cx.y * b.x + m.cx.x * b.y);
    return r;
}
O_FN OV3 o_xf(OV3 p, OQ q, OV3 local) { return o_add(p, o_rot(q, local)); }            /* :361-363 */
O_FN int o_overlap(OAabb a, OAabb b) {                                                  /* :365-369 */
    return a.lo.x <= b.hi.x && a.hi.x >= b.lo.x && a.lo.y <= b.hi.y && a.hi.y >= b.lo.y
        && a.lo.z <= b.hi.z && a.hi.z >= b.lo.z;
}

/* ------------------------------------------------------------------ */
/* Shape poses and bounds: src/puffysics/04_world.inl:293-336           */
/* ------------------------------------------------------------------ */

O_FN OQ o_shape_rot(const OBody* b, const OShape* s) { return o_qmul(b->rotation, s->local_rot); }
O_FN OV3 o_shape_pos(const OBody* b, const OShape* s) { return o_xf(b->position, b->rotation, s->local_pos); }
static OAabb o_shape_aabb(const OBody* b, const OShape* s) {
    OV3 p = o_shape_pos(b, s);
    OQ q = o_shape_rot(b, s);
    OAabb a;
    if (s->type == B3_SPHERE) {
        OV3 e = o_v(s->radius, s->radius, s->radius);
        a.lo = o_sub(p, e);
        a.hi = o_add(p, e);
        return a;
    }
    if (s->type == B3_CAPSULE) {
        OV3 y = o_rot(q, o_v(0.0f, s->half.y, 0.0f));
        OV3 c1 = o_sub(p, y);
        OV3 c2 = o_add(p, y);
        OV3 e = o_v(s->radius, s->radius, s->radius);
        a.lo = o_v(o_min(c1.x, c2.x), o_min(c1.y, c2.y), o_min(c1.z, c2.z));
        a.hi = o_v(o_max(c1.x, c2.x), o_max(c1.y, c2.y), o_max(c1.z, c2.z));
        a.lo = o_sub(a.lo, e);
        a.hi = o_add(a.hi, e);
        return a;
    }
    OV3 ax, ay, az;
    o_axes(q, &ax, &ay, &az);
    OV3 e = o_v(
        o_fabs(ax.x) * s->half.x + o_fabs(ay.x) * s->half.y + o_fabs(az.x) * s->half.z,
        o_fabs(ax.y) * s->half.x + o_fabs(ay.y) * s->half.y + o_fabs(az.y) * s->half.z,
        o_fabs(ax.z) * s->half.x + o_fabs(ay.z) * s->half.y + o_fabs(az.z) * s->half.z);
    a.lo = o_sub(p, e);
    a.hi = o_add(p, e);
    return a;
}

/* ------------------------------------------------------------------ */
/* Narrowphase: src/puffysics/05_collision.inl                          */
/* ------------------------------------------------------------------ */

static OV3 o_closest_seg(OV3 a, OV3 b, OV3 p) {                                          /* :5-13 */
    OV3 ab = o_sub(b, a);
    b3r d = o_len2(ab);
    if (d <= 1.0e-12f) return a;
    b3r t = o_clamp(o_dot(o_sub(p, a), ab) / d, 0.0f, 1.0f);
    return o_madd(a, t, ab);
}

static void o_closest_segs(OV3 a1, OV3 a2, OV3 b1, OV3 b2, OV3* pa, OV3* pb) {          /* :15-55 */
    OV3 d1 = o_sub(a2, a1);
    OV3 d2 = o_sub(b2, b1);
    OV3 r = o_sub(a1, b1);
    b3r a = o_len2(d1);
    b3r e = o_len2(d2);
    b3r f = o_dot(d2, r);
    b3r s, t;
    if (a <= 1.0e-12f && e <= 1.0e-12f) {
        *pa = a1;
        *pb = b1;
        return;
    }
    if (a <= 1.0e-12f) {
        s = 0.0f;
        t = o_clamp(f / e, 0.0f, 1.0f);
    } else {
        b3r c = o_dot(d1, r);
        if (e <= 1.0e-12f) {
            t = 0.0f;
            s = o_clamp(-c / a, 0.0f, 1.0f);
        } else {
            b3r b = o_dot(d1, d2);
            b3r den = a * e - b * b;
            if (den != 0.0f) s = o_clamp((b * f - c * e) / den, 0.0f, 1.0f);
            else s = 0.0f;
            t = (b * s + f) / e;
            if (t < 0.0f) {
                t = 0.0f;
                s = o_clamp(-c / a, 0.0f, 1.0f);
            } else if (t > 1.0f) {
                t = 1.0f;
                s = o_clamp((b - c) / a, 0.0f, 1.0f);
            }
        }
    }
    *pa = o_madd(a1, s, d1);
    *pb = o_madd(b1, t, d2);
}

typedef struct {                                                                        /* :57-64 */
    int count;
    OV3 normal;
    OV3 p_a[B3_MAX_MANIFOLD];
    OV3 p_b[B3_MAX_MANIFOLD];
    b3r sep[B3_MAX_MANIFOLD];
    uint32_t feature[B3_MAX_MANIFOLD];
} OMani;

O_FN void o_mani_clear(OMani* m) { m->count = 0; m->normal = o_v(0.0f, 1.0f, 0.0f); }  /* :66-69 */
O_FN void o_mani_push(OMani* m, OV3 pa, OV3 pb, b3r sep, uint32_t feat) {              /* :71-81 */
    if (m->count >= B3_MAX_MANIFOLD) return;
    int i = m->count++;
    m->p_a[i] = pa;
    m->p_b[i] = pb;
    m->sep[i] = sep;
    m->feature[i] = feat;
}

static void o_collide_balls(OMani* m, OV3 ca, b3r ra, OV3 cb, b3r rb, uint32_t feat) {  /* :83-98 */
    o_mani_clear(m);
    OV3 d = o_sub(cb, ca);
    b3r dist2 = o_len2(d);
    b3r rad = ra + rb;
    if (dist2 > rad * rad) return;
    b3r dist = o_sqrt(dist2);
    OV3 n = dist > 1.0e-8f ? o_scale(d, o_rsqrt(dist2)) : o_v(0.0f, 1.0f, 0.0f);
    m->normal = n;
    o_mani_push(m, o_madd(ca, ra, n), o_msub(cb, rb, n), dist - rad, feat);
}

static OV3 o_closest_obb(OV3 c, OQ q, OV3 half, OV3 p, int* inside, int* face) {        /* :100-129 */
    OV3 local = o_invrot(q, o_sub(p, c));
    OV3 cl = o_v(o_clamp(local.x, -half.x, half.x), o_clamp(local.y, -half.y, half.y),
        o_clamp(local.z, -half.z, half.z));
    int in = o_fabs(local.x) <= half.x && o_fabs(local.y) <= half.y && o_fabs(local.z) <= half.z;
    *inside = in;
    if (in) {
        b3r dx = half.x - o_fabs(local.x);
        b3r dy = half.y - o_fabs(local.y);
        b3r dz = half.z - o_fabs(local.z);
        if (dx <= dy && dx <= dz) {
            cl.x = local.x >= 0.0f ? half.x : -half.x;
            *face = 0;
        } else if (dy <= dz) {
            cl.y = local.y >= 0.0f ? half.y : -half.y;
            *face = 1;
        } else {
            cl.z = local.z >= 0.0f ? half.z : -half.z;
            *face = 2;
        }
    } else {
        *face = -1;
    }
    return o_xf(c, q, cl);
}

static void o_collide_ball_point(OMani* m, OV3 p, b3r r, OV3 q, int inside, OV3 n_fb,    /* :131-150 */
        uint32_t feat) {
    OV3 d = o_sub(p, q);
    b3r dist2 = o_len2(d);
    if (!inside && dist2 > r * r) return;
    OV3 n;
    b3r sep;
    if (inside) {
        n = dist2 > 1.0e-12f ? o_norm(d) : n_fb;
        sep = -o_len(d) - r;
    } else {
        b3r dist = o_sqrt(dist2);
        n = o_scale(d, o_rsqrt(dist2));
        sep = dist - r;
    }
    m->normal = n;
    o_mani_push(m, o_msub(p, r, n), q, sep, feat);
}

static void o_collide_sphere_box(OMani* m, OV3 sc, b3r r, OV3 bc, OQ bq, OV3 half) {     /* :152-162 */
    o_mani_clear(m);
    int inside, face;
    OV3 q = o_closest_obb(bc, bq, half, sc, &inside, &face);
    OV3 ax, ay, az;
    o_axes(bq, &ax, &ay, &az);
    OV3 n_fb = face == 0 ? ax : (face == 1 ? ay : az);
    o_collide_ball_point(m, sc, r, q, inside, n_fb, 3u);
}

static void o_collide_capsule_box(OMani* m, OV3 c1, OV3 c2, b3r r, OV3 bc, OQ bq,        /* :164-175 */
        OV3 half) {
    o_mani_clear(m);
    OV3 mid = o_scale(o_add(c1, c2), 0.5f);
    int inside, face;
    OV3 q = o_closest_obb(bc, bq, half, mid, &inside, &face);
    OV3 p = o_closest_seg(c1, c2, q);
    q = o_closest_obb(bc, bq, half, p, &inside, &face);
    p = o_closest_seg(c1, c2, q);
    o_collide_ball_point(m, p, r, q, inside, o_v(0.0f, 1.0f, 0.0f), 5u);
}

typedef struct { OV3 c; OV3 ax[3]; OV3 h; } OObb;                                        /* :177-181 */

O_FN OObb o_obb(OV3 c, OQ q, OV3 h) {                                                    /* :183-189 */
    OObb o;
    o.c = c;
    o.h = h;
    o_axes(q, &o.ax[0], &o.ax[1], &o.ax[2]);
    return o;
}
O_FN b3r o_half_i(OV3 h, int i) { return i == 0 ? h.x : (i == 1 ? h.y : h.z); }        /* :191-193 */
static OV3 o_support(const OObb* o, OV3 dir) {                                           /* :195-201 */
    b3r sx = o_dot(o->ax[0], dir) < 0.0f ? -o->h.x : o->h.x;
    b3r sy = o_dot(o->ax[1], dir) < 0.0f ? -o->h.y : o->h.y;
    b3r sz = o_dot(o->ax[2], dir) < 0.0f ? -o->h.z : o->h.z;
    return o_add(o->c, o_add(o_scale(o->ax[0], sx), o_add(o_scale(o->ax[1], sy), o_scale(o->ax[2], sz))));
}
static int o_clip_plane(const OV3* in, int n, OV3* out, OV3 pn, b3r po) {                /* :203-228 */
    if (n <= 0) return 0;
    int c = 0;
    OV3 prev = in[n - 1];
    b3r pd = o_dot(prev, pn) - po;
    int pin = pd <= 0.0f;
    for (int i = 0; i < n; i++) {
        OV3 cur = in[i];
        b3r cd = o_dot(cur, pn) - po;
        int cin = cd <= 0.0f;
        if (cin != pin && c < 8) {
            b3r t = pd / (pd - cd);
            out[c++] = o_madd(prev, t, o_sub(cur, prev));
        }
        if (cin && c < 8) out[c++] = cur;
        prev = cur;
        pd = cd;
        pin = cin;
    }
    return c;
}
static void o_face_pts(const OObb* o, int axis, b3r sign, OV3 out[4]) {                  /* :230-241 */
    int ta = (axis + 1) % 3;
    int tb = (axis + 2) % 3;
    OV3 c = o_madd(o->c, sign * o_half_i(o->h, axis), o->ax[axis]);
    OV3 a = o_scale(o->ax[ta], o_half_i(o->h, ta));
    OV3 b = o_scale(o->ax[tb], o_half_i(o->h, tb));
    out[0] = o_sub(o_sub(c, a), b);
    out[1] = o_add(o_sub(c, a), b);
    out[2] = o_add(o_add(c, a), b);
    out[3] = o_sub(o_add(c, a), b);
}
static int o_best_axis(const OObb* o, OV3 n) {                                           /* :243-251 */
    b3r b0 = o_fabs(o_dot(o->ax[0], n));
    b3r b1 = o_fabs(o_dot(o->ax[1], n));
    b3r b2 = o_fabs(o_dot(o->ax[2], n));
    if (b0 >= b1 && b0 >= b2) return 0;
    return b1 >= b2 ? 1 : 2;
}
static void o_mani_support(OMani* m, const OObb* a, const OObb* b, OV3 n, int feat) {   /* :253-258 */
    OV3 pa = o_support(a, n);
    OV3 pb = o_support(b, o_neg(n));
    o_mani_push(m, pa, pb, o_dot(o_sub(pb, pa), n), (uint32_t)feat);
}
/* Face axis candidate: -1 = separated beyond the speculative margin. :260-271 */
static int o_try_face(b3r s, OV3 axis, b3r side, b3r* best, OV3* n, int feat, int* out_feat) {
    if (s > B3_SPECULATIVE) return -1;
    if (s > *best) {
        *best = s;
        *n = side < 0.0f ? o_neg(axis) : axis;
        *out_feat = feat;
    }
    return 0;
}
/* Edge-edge axis candidate with the 0.002 face preference. :273-293 */
static int o_try_edge(b3r e, b3r ra, b3r rb, OV3 cr, b3r* best, OV3* n, int feat, int* out_feat) {
    b3r cl2 = o_len2(cr);
    if (cl2 <= 1.0e-3f) return 0;
    b3r inv = o_rsqrt(cl2);
    b3r s = (o_fabs(e) - ra - rb) * inv;
    if (s > B3_SPECULATIVE && cl2 > 0.05f) return -1;
    if (s > B3_SPECULATIVE) return 0;
    if (s > *best + 0.002f) {
        *best = s;
        *n = e < 0.0f ? o_scale(cr, -inv) : o_scale(cr, inv);
        *out_feat = feat;
    }
    return 0;
}
/* 15-axis SAT, then reference-face clipping or a support-point fallback. :295-461 */
static void o_collide_boxes(OMani* m, const OObb* a, const OObb* b) {
    o_mani_clear(m);
    OV3 d = o_sub(b->c, a->c);
    b3r t0 = o_dot(d, a->ax[0]), t1 = o_dot(d, a->ax[1]), t2 = o_dot(d, a->ax[2]);
    b3r r00 = o_dot(a->ax[0], b->ax[0]), r01 = o_dot(a->ax[0], b->ax[1]), r02 = o_dot(a->ax[0], b->ax[2]);
    b3r r10 = o_dot(a->ax[1], b->ax[0]), r11 = o_dot(a->ax[1], b->ax[1]), r12 = o_dot(a->ax[1], b->ax[2]);
    b3r r20 = o_dot(a->ax[2], b->ax[0]), r21 = o_dot(a->ax[2], b->ax[1]), r22 = o_dot(a->ax[2], b->ax[2]);
    b3r ar00 = o_fabs(r00), ar01 = o_fabs(r01), ar02 = o_fabs(r02);
    b3r ar10 = o_fabs(r10), ar11 = o_fabs(r11), ar12 = o_fabs(r12);
    b3r ar20 = o_fabs(r20), ar21 = o_fabs(r21), ar22 = o_fabs(r22);
    b3r hax = a->h.x, hay = a->h.y, haz = a->h.z;
    b3r hbx = b->h.x, hby = b->h.y, hbz = b->h.z;
    b3r best = -FLT_MAX;
    OV3 n = a->ax[0];
    int feat = 0;

    if (o_try_face(o_fabs(t0) - hax - (hbx * ar00 + hby * ar01 + hbz * ar02), a->ax[0], t0, &best, &n, 0, &feat) < 0) return;
    if (o_try_face(o_fabs(t1) - hay - (hbx * ar10 + hby * ar11 + hbz * ar12), a->ax[1], t1, &best, &n, 1, &feat) < 0) return;
    if (o_try_face(o_fabs(t2) - haz - (hbx * ar20 + hby * ar21 + hbz * ar22), a->ax[2], t2, &best, &n, 2, &feat) < 0) return;
    b3r u0 = t0 * r00 + t1 * r10 + t2 * r20;
    b3r u1 = t0 * r01 + t1 * r11 + t2 * r21;
    b3r u2 = t0 * r02 + t1 * r12 + t2 * r22;
    if (o_try_face(o_fabs(u0) - hbx - (hax * ar00 + hay * ar10 + haz * ar20), b->ax[0], u0, &best, &n, 3, &feat) < 0) return;
    if (o_try_face(o_fabs(u1) - hby - (hax * ar01 + hay * ar11 + haz * ar21), b->ax[1], u1, &best, &n, 4, &feat) < 0) return;
    if (o_try_face(o_fabs(u2) - hbz - (hax * ar02 + hay * ar12 + haz * ar22), b->ax[2], u2, &best, &n, 5, &feat) < 0) return;

    if (o_try_edge(t2 * r10 - t1 * r20, hay * ar20 + haz * ar10, hby * ar02 + hbz * ar01, o_cross(a->ax[0], b->ax[0]), &best, &n, 6, &feat) < 0) return;
    if (o_try_edge(t2 * r11 - t1 * r21, hay * ar21 + haz * ar11, hbz * ar00 + hbx * ar02, o_cross(a->ax[0], b->ax[1]), &best, &n, 7, &feat) < 0) return;
    if (o_try_edge(t2 * r12 - t1 * r22, hay * ar22 + haz * ar12, hbx * ar01 + hby * ar00, o_cross(a->ax[0], b->ax[2]), &best, &n, 8, &feat) < 0) return;
    if (o_try_edge(t0 * r20 - t2 * r00, haz * ar00 + hax * ar20, hby * ar12 + hbz * ar11, o_cross(a->ax[1], b->ax[0]), &best, &n, 9, &feat) < 0) return;
    if (o_try_edge(t0 * r21 - t2 * r01, haz * ar01 + hax * ar21, hbz * ar10 + hbx * ar12, o_cross(a->ax[1], b->ax[1]), &best, &n, 10, &feat) < 0) return;
    if (o_try_edge(t0 * r22 - t2 * r02, haz * ar02 + hax * ar22, hbx * ar11 + hby * ar10, o_cross(a->ax[1], b->ax[2]), &best, &n, 11, &feat) < 0) return;
    if (o_try_edge(t1 * r00 - t0 * r10, hax * ar10 + hay * ar00, hby * ar22 + hbz * ar21, o_cross(a->ax[2], b->ax[0]), &best, &n, 12, &feat) < 0) return;
    if (o_try_edge(t1 * r01 - t0 * r11, hax * ar11 + hay * ar01, hbz * ar20 + hbx * ar22, o_cross(a->ax[2], b->ax[1]), &best, &n, 13, &feat) < 0) return;
    if (o_try_edge(t1 * r02 - t0 * r12, hax * ar12 + hay * ar02, hbx * ar21 + hby * ar20, o_cross(a->ax[2], b->ax[2]), &best, &n, 14, &feat) < 0) return;

    if (o_dot(n, d) < 0.0f) n = o_neg(n);
    m->normal = n;
    if (feat >= 6) {
        o_mani_support(m, a, b, n, feat);
        return;
    }
    const OObb* ref = feat < 3 ? a : b;
    const OObb* inc = feat < 3 ? b : a;
    int ref_axis = feat < 3 ? feat : feat - 3;
    b3r rd = o_dot(ref->ax[ref_axis], n);
    b3r ref_sign = (feat < 3 ? rd < 0.0f : rd > 0.0f) ? -1.0f : 1.0f;
    OV3 rn = o_scale(ref->ax[ref_axis], ref_sign);
    int inc_axis = o_best_axis(inc, rn);
    b3r inc_sign = o_dot(inc->ax[inc_axis], rn) > 0.0f ? -1.0f : 1.0f;
    OV3 poly[8], tmp[8];
    o_face_pts(inc, inc_axis, inc_sign, poly);
    int count = 4;
    int ta = (ref_axis + 1) % 3;
    int tb = (ref_axis + 2) % 3;
    OV3 face_c = o_madd(ref->c, ref_sign * o_half_i(ref->h, ref_axis), ref->ax[ref_axis]);
    for (int i = 0; i < 4; i++) {
        int t = i < 2 ? ta : tb;
        b3r s = (i & 1) ? 1.0f : -1.0f;
        OV3 cn = o_scale(ref->ax[t], s);
        b3r co = o_dot(cn, ref->c) + o_half_i(ref->h, t);
        count = o_clip_plane(poly, count, tmp, cn, co);
        for (int k = 0; k < count; k++) poly[k] = tmp[k];
        if (count == 0) {
            o_mani_support(m, a, b, n, feat);
            return;
        }
    }
    b3r ro = o_dot(rn, face_c);
    for (int i = 0; i < count && m->count < B3_MAX_MANIFOLD; i++) {
        b3r plane_s = o_dot(poly[i], rn) - ro;
        if (plane_s <= B3_SPECULATIVE) {
            OV3 on_ref = o_msub(poly[i], plane_s, rn);
            OV3 pa = feat < 3 ? on_ref : poly[i];
            OV3 pb = feat < 3 ? poly[i] : on_ref;
            b3r sep = o_dot(o_sub(pb, pa), n);
            o_mani_push(m, pa, pb, sep, (feat < 3 ? 16u : 20u) + (uint32_t)i);
        }
    }
    if (m->count == 0) o_mani_support(m, a, b, n, feat);
}
static void o_mani_flip(OMani* m) {                                                      /* :463-470 */
    m->normal = o_neg(m->normal);
    for (int i = 0; i < m->count; i++) {
        OV3 t = m->p_a[i];
        m->p_a[i] = m->p_b[i];
        m->p_b[i] = t;
    }
}
/* Type-ordered dispatch, flip back, orient A->B, recompute separations. :472-534 */
static void o_collide_pair(OMani* m, const OBody* ba, const OShape* sa, const OBody* bb, const OShape* sb) {
    OV3 pa = o_shape_pos(ba, sa);
    OV3 pb = o_shape_pos(bb, sb);
    OV3 center_a = pa, center_b = pb;
    OQ qa = o_shape_rot(ba, sa);
    OQ qb = o_shape_rot(bb, sb);
    int ta = sa->type, tb = sb->type;
    int flip = 0;
    if (ta > tb) {
        const OShape* ts = sa; sa = sb; sb = ts;
        OV3 tp = pa; pa = pb; pb = tp;
        OQ tq = qa; qa = qb; qb = tq;
        int tt = ta; ta = tb; tb = tt;
        flip = 1;
    }
    if (ta == B3_SPHERE && tb == B3_SPHERE) {
        o_collide_balls(m, pa, sa->radius, pb, sb->radius, 1u);
    } else if (ta == B3_SPHERE && tb == B3_CAPSULE) {
        OV3 y = o_rot(qb, o_v(0.0f, sb->half.y, 0.0f));
        o_collide_balls(m, o_closest_seg(o_sub(pb, y), o_add(pb, y), pa), sb->radius, pa, sa->radius, 4u);
        o_mani_flip(m);
    } else if (ta == B3_SPHERE && tb == B3_BOX) {
        o_collide_sphere_box(m, pa, sa->radius, pb, qb, sb->half);
    } else if (ta == B3_CAPSULE && tb == B3_CAPSULE) {
        OV3 ya = o_rot(qa, o_v(0.0f, sa->half.y, 0.0f));
        OV3 yb = o_rot(qb, o_v(0.0f, sb->half.y, 0.0f));
        OV3 ca, cb;
        o_closest_segs(o_sub(pa, ya), o_add(pa, ya), o_sub(pb, yb), o_add(pb, yb), &ca, &cb);
        o_collide_balls(m, ca, sa->radius, cb, sb->radius, 2u);
    } else if (ta == B3_CAPSULE && tb == B3_BOX) {
        OV3 y = o_rot(qa, o_v(0.0f, sa->half.y, 0.0f));
        o_collide_capsule_box(m, o_sub(pa, y), o_add(pa, y), sa->radius, pb, qb, sb->half);
    } else {
        OObb oa = o_obb(pa, qa, sa->half);
        OObb ob = o_obb(pb, qb, sb->half);
        o_collide_boxes(m, &oa, &ob);
    }
    if (flip && m->count > 0) o_mani_flip(m);
    if (m->count > 0) {
        if (o_dot(m->normal, o_sub(center_b, center_a)) < 0.0f) m->normal = o_neg(m->normal);
        for (int i = 0; i < m->count; i++) m->sep[i] = o_dot(o_sub(m->p_b[i], m->p_a[i]), m->normal);
    }
}

/* ------------------------------------------------------------------ */
/* Contacts: src/puffysics/08_contacts.inl, 07_packed.inl:24-45         */
/* ------------------------------------------------------------------ */

static void o_contact_from_mani(OContact* c, int si, int sj, const OShape* sa, const OShape* sb,  /* :5-39 */
        const OBody* ba, const OBody* bb, const OMani* mani) {
    c->shape_a = si;
    c->shape_b = sj;
    c->body_a = sa->body;
    c->body_b = sb->body;
    c->point_count = mani->count;
    c->normal = mani->normal;
    c->tangent1 = o_perp(mani->normal);
    c->tangent2 = o_cross(c->tangent1, mani->normal);
    c->friction = o_sqrt(sa->friction * sb->friction);
    c->restitution = sa->restitution > sb->restitution ? sa->restitution : sb->restitution;
    c->rolling = o_max(sa->rolling, sb->rolling);
    c->static_contact = ba->type != B3_DYNAMIC || bb->type != B3_DYNAMIC;
    OV3 ca = ba->center, cb = bb->center;
    c->friction_impulse.x = 0.0f;
    c->friction_impulse.y = 0.0f;
    c->twist_impulse = 0.0f;
    c->rolling_impulse = o_v(0.0f, 0.0f, 0.0f);
    for (int p = 0; p < mani->count; p++) {
        OPoint* cp = &c->points[p];
        cp->r_a = o_sub(mani->p_a[p], ca);
        cp->r_b = o_sub(mani->p_b[p], cb);
        cp->base_sep = mani->sep[p] - o_dot(o_sub(cp->r_b, cp->r_a), mani->normal);
        cp->feature = mani->feature[p];
        cp->normal_impulse = 0.0f;
        cp->total_normal = 0.0f;
        cp->rel_vel = 0.0f;
        cp->normal_mass = 0.0f;
        cp->lever = 0.0f;
    }
}

typedef struct {                                                                        /* 02_types.inl:133-142 */
    int shape_a, shape_b, point_count;
    uint32_t feature[B3_MAX_MANIFOLD];
    b3r normal_impulse[B3_MAX_MANIFOLD];
    OV2 friction_impulse;
    b3r twist_impulse;
    OV3 rolling_impulse;
} OWarm;

/* Is there a joint with collide_connected == 0 between bodies a and b?
 * Same predicate as the connected[][] bit matrix of :95-108. */
static int o_connected(const OWorld* w, int a, int b) {
    for (int i = 0; i < w->h->joint_count; i++) {
        const OJoint* jn = &w->joints[i];
        if (jn->collide_connected) continue;
        if ((jn->body_a == a && jn->body_b == b) || (jn->body_a == b && jn->body_b == a)) return 1;
    }
    return 0;
}

static int o_broadphase_pair(const OWorld* w, int i, int j, const OAabb* aabb) {       /* :45-62 */
    const OShape* sa = &w->shapes[i];
    const OShape* sb = &w->shapes[j];
    const OBody* ba = &w->bodies[sa->body];
    const OBody* bb = &w->bodies[sb->body];
    if (sa->body == sb->body || o_connected(w, sa->body, sb->body)
            || (ba->type == B3_STATIC && bb->type == B3_STATIC)
            || (sa->category & sb->mask) == 0 || (sb->category & sa->mask) == 0
            || !o_overlap(aabb[i], aabb[j]))
        return 0;
    return 1;
}

static void o_find_contacts(OWorld* w) {                                                 /* :64-173 */
    int old_n = w->h->contact_count;
    OWarm old[old_n > 0 ? old_n : 1];
    for (int i = 0; i < old_n; i++) {
        const OContact* src = &w->contacts[i];
        old[i].shape_a = src->shape_a;
        old[i].shape_b = src->shape_b;
        old[i].point_count = src->point_count;
        old[i].friction_impulse = src->friction_impulse;
        old[i].twist_impulse = src->twist_impulse;
        old[i].rolling_impulse = src->rolling_impulse;
        for (int p = 0; p < src->point_count; p++) {
            old[i].feature[p] = src->points[p].feature;
            old[i].normal_impulse[p] = src->points[p].normal_impulse;
        }
    }
    w->h->contact_count = 0;
    int ns = w->h->shape_count;
    OAabb aabb[ns > 0 ? ns : 1];
    OV3 pad = o_v(B3_SPECULATIVE, B3_SPECULATIVE, B3_SPECULATIVE);
    for (int i = 0; i < ns; i++) {
        aabb[i] = o_shape_aabb(&w->bodies[w->shapes[i].body], &w->shapes[i]);
        aabb[i].lo = o_sub(aabb[i].lo, pad);
        aabb[i].hi = o_add(aabb[i].hi, pad);
    }
    for (int i = 0; i < ns; i++) {
        const OShape* sa = &w->shapes[i];
        const OBody* ba = &w->bodies[sa->body];
        for (int j = i + 1; j < ns; j++) {
            const OShape* sb = &w->shapes[j];
            const OBody* bb = &w->bodies[sb->body];
            if (!o_broadphase_pair(w, i, j, aabb)) continue;
            OMani mani;
            o_collide_pair(&mani, ba, sa, bb, sb);
            if (mani.count == 0) continue;
            if (w->h->contact_count >= w->max_c) {
                w->h->contact_overflow = 1;
                w->h->contacts_dropped++;
                continue;
            }
            OContact* c = &w->contacts[w->h->contact_count++];
            o_contact_from_mani(c, i, j, sa, sb, ba, bb, &mani);
            /* warm start: every matching old pair, last matching feature wins :154-170 */
            for (int k = 0; k < old_n; k++) {
                if (old[k].shape_a != i || old[k].shape_b != j) continue;
                for (int p = 0; p < c->point_count; p++)
                    for (int q = 0; q < old[k].point_count; q++)
                        if (c->points[p].feature == old[k].feature[q])
                            c->points[p].normal_impulse = old[k].normal_impulse[q];
                c->friction_impulse = old[k].friction_impulse;
                c->twist_impulse = old[k].twist_impulse;
                c->rolling_impulse = old[k].rolling_impulse;
            }
        }
    }
}

static void o_prepare_one_contact(OContact* c, const OBody* ba, const OBody* bb,          /* :234-291 */
        OSoft contact_s, OSoft static_s) {
    b3r ma = ba->type == B3_DYNAMIC ? ba->inv_mass : 0.0f;
    b3r mb = bb->type == B3_DYNAMIC ? bb->inv_mass : 0.0f;
    OM3 ia = ba->type == B3_DYNAMIC ? ba->inv_i_world : o_m0();
    OM3 ib = bb->type == B3_DYNAMIC ? bb->inv_i_world : o_m0();
    c->inv_mass_a = ma;
    c->inv_mass_b = mb;
    c->inv_i_a = ia;
    c->inv_i_b = ib;
    c->rolling_mass = o_inv3(o_madd3(ia, ib));
    c->softness = c->static_contact ? static_s : contact_s;
    OV3 n = c->normal;
    OV3 center_a = o_v(0.0f, 0.0f, 0.0f);
    OV3 center_b = o_v(0.0f, 0.0f, 0.0f);
    b3r wsum = 0.0f;
    b3r one = 1.0f;
    b3r inv_tau = one / B3_SPECULATIVE;
    for (int p = 0; p < c->point_count; p++) {
        OPoint* cp = &c->points[p];
        OV3 rn_a = o_cross(cp->r_a, n);
        OV3 rn_b = o_cross(cp->r_b, n);
        b3r kn = ma + mb + o_dot(rn_a, o_mv(ia, rn_a)) + o_dot(rn_b, o_mv(ib, rn_b));
        cp->normal_mass = kn > 0.0f ? one / kn : 0.0f;
        OV3 vra = o_add(ba->lin_vel, o_cross(ba->ang_vel, cp->r_a));
        OV3 vrb = o_add(bb->lin_vel, o_cross(bb->ang_vel, cp->r_b));
        cp->rel_vel = o_dot(n, o_sub(vrb, vra));
        cp->total_normal = 0.0f;
        b3r sep = cp->base_sep + o_dot(o_sub(cp->r_b, cp->r_a), n);
        b3r weight = o_clamp(2.0f - sep * inv_tau, B3_MIN_FRICTION_W, 1.0f);
        center_a = o_madd(center_a, weight, cp->r_a);
        center_b = o_madd(center_b, weight, cp->r_b);
        wsum += weight;
    }
    b3r invw = wsum > 0.0f ? one / wsum : 0.0f;
    c->center_a = o_scale(center_a, invw);
    c->center_b = o_scale(center_b, invw);
    for (int p = 0; p < c->point_count; p++)
        c->points[p].lever = o_len(o_sub(c->points[p].r_a, c->center_a));
    OV3 rt_a1 = o_cross(c->center_a, c->tangent1);
    OV3 rt_a2 = o_cross(c->center_a, c->tangent2);
    OV3 rt_b1 = o_cross(c->center_b, c->tangent1);
    OV3 rt_b2 = o_cross(c->center_b, c->tangent2);
    OM2 k;
    k.cx.x = ma + mb + o_dot(rt_a1, o_mv(ia, rt_a1)) + o_dot(rt_b1, o_mv(ib, rt_b1));
    k.cy.y = ma + mb + o_dot(rt_a2, o_mv(ia, rt_a2)) + o_dot(rt_b2, o_mv(ib, rt_b2));
    k.cx.y = o_dot(rt_a1, o_mv(ia, rt_a2)) + o_dot(rt_b1, o_mv(ib, rt_b2));
    k.cy.x = k.cx.y;
    c->tangent_mass = o_inv2(k);
    b3r kt = o_dot(n, o_mv(o_madd3(ia, ib), n));
    c->twist_mass = kt > 0.0f ? one / kt : 0.0f;
}

static void o_apply_impulse(OBody* b, b3r m, OM3 i, OV3 r, OV3 p, int sign) {            /* :184-192 */
    if ((b->flags & B3_FLAG_DYNAMIC) == 0) return;
    b3r s = sign > 0 ? 1.0f : -1.0f;
    b->lin_vel = o_madd(b->lin_vel, s * m, p);
    b->ang_vel = o_add(b->ang_vel, o_mv(i, o_scale(o_cross(r, p), s)));
}

static void o_warm_one_contact(OContact* c, OBody* ba, OBody* bb) {                      /* :293-313 */
    OV3 n = c->normal;
    for (int p = 0; p < c->point_count; p++) {
        OPoint* cp = &c->points[p];
        OV3 P = o_scale(n, cp->normal_impulse);
        o_apply_impulse(ba, c->inv_mass_a, c->inv_i_a, cp->r_a, P, -1);
        o_apply_impulse(bb, c->inv_mass_b, c->inv_i_b, cp->r_b, P, 1);
    }
    OV3 f = o_add(o_scale(c->tangent1, c->friction_impulse.x), o_scale(c->tangent2, c->friction_impulse.y));
    o_apply_impulse(ba, c->inv_mass_a, c->inv_i_a, c->center_a, f, -1);
    o_apply_impulse(bb, c->inv_mass_b, c->inv_i_b, c->center_b, f, 1);
    if ((ba->flags & B3_FLAG_DYNAMIC) != 0)
        ba->ang_vel = o_sub(ba->ang_vel, o_mv(c->inv_i_a, o_add(o_scale(n, c->twist_impulse), c->rolling_impulse)));
    if ((bb->flags & B3_FLAG_DYNAMIC) != 0)
        bb->ang_vel = o_add(bb->ang_vel, o_mv(c->inv_i_b, o_add(o_scale(n, c->twist_impulse), c->rolling_impulse)));
}

/* Rolling resistance on the tangent plane (07_packed.inl:24-45). */
static void o_solve_rolling(OV3 t1, OV3 t2, b3r rolling, b3r total_n, OM3 ia, OM3 ib,
        OV3* impulse, OV3* wa, OV3* wb) {
    if (rolling <= 0.0f) return;
    OM3 isum = o_madd3(ia, ib);
    OM2 k;
    k.cx.x = o_dot(t1, o_mv(isum, t1));
    k.cy.y = o_dot(t2, o_mv(isum, t2));
    k.cx.y = o_dot(t1, o_mv(isum, t2));
    k.cy.x = k.cx.y;
    OV3 wr = o_sub(*wb, *wa);
    OV2 rhs;
    rhs.x = o_dot(wr, t1);
    rhs.y = o_dot(wr, t2);
    OV2 d = o_mv2(o_inv2(k), rhs);
    OV3 next = o_sub(*impulse, o_add(o_scale(t1, d.x), o_scale(t2, d.y)));
    b3r limit = rolling * total_n;
    b3r l2 = o_len2(next);
    if (l2 > limit * limit && l2 > 0.0f) next = o_scale(next, o_rsqrt_scale(limit, l2));
    OV3 delta = o_sub(next, *impulse);
    *impulse = next;
    *wa = o_sub(*wa, o_mv(ia, delta));
    *wb = o_add(*wb, o_mv(ib, delta));
}

static void o_solve_one_contact(OContact* c, OBody* ba, OBody* bb, b3r inv_h,           /* :315-413 */
        b3r contact_speed, int use_bias) {
    OV3 va = ba->lin_vel, wa = ba->ang_vel, vb = bb->lin_vel, wb = bb->ang_vel;
    OQ dqa = ba->delta_rot, dqb = bb->delta_rot;
    OV3 dp = o_sub(bb->delta_pos, ba->delta_pos);
    OV3 n = c->normal;
    b3r total_n = 0.0f;
    b3r twist_lim = 0.0f;
    for (int p = 0; p < c->point_count; p++) {
        OPoint* cp = &c->points[p];
        OV3 ra = cp->r_a, rb = cp->r_b;
        OV3 ds = o_add(dp, o_sub(o_rot(dqb, rb), o_rot(dqa, ra)));
        b3r sep = o_dot(ds, n) + cp->base_sep;
        b3r vbias = 0.0f, mscale = 1.0f, iscale = 0.0f;
        if (sep > 0.0f) {
            vbias = sep * inv_h;
        } else if (use_bias) {
            vbias = o_max(c->softness.mass_scale * c->softness.bias_rate * sep, -contact_speed);
            mscale = c->softness.mass_scale;
            iscale = c->softness.impulse_scale;
        }
        OV3 vra = o_add(va, o_cross(wa, ra));
        OV3 vrb = o_add(vb, o_cross(wb, rb));
        b3r vn = o_dot(o_sub(vrb, vra), n);
        b3r dimp = -cp->normal_mass * (mscale * vn + vbias) - iscale * cp->normal_impulse;
        b3r nimp = o_max(cp->normal_impulse + dimp, 0.0f);
        dimp = nimp - cp->normal_impulse;
        cp->normal_impulse = nimp;
        cp->total_normal += nimp;
        total_n += nimp;
        twist_lim += cp->lever * cp->normal_impulse;
        OV3 P = o_scale(n, dimp);
        va = o_msub(va, c->inv_mass_a, P);
        wa = o_sub(wa, o_mv(c->inv_i_a, o_cross(ra, P)));
        vb = o_madd(vb, c->inv_mass_b, P);
        wb = o_add(wb, o_mv(c->inv_i_b, o_cross(rb, P)));
    }
    if (!use_bias) {
        b3r twist_s = o_dot(n, o_sub(wb, wa));
        b3r max_t = c->friction * twist_lim;
        b3r dtw = -c->twist_mass * twist_s;
        b3r old_t = c->twist_impulse;
        c->twist_impulse = o_clamp(old_t + dtw, -max_t, max_t);
        dtw = c->twist_impulse - old_t;
        wa = o_sub(wa, o_mv(c->inv_i_a, o_scale(n, dtw)));
        wb = o_add(wb, o_mv(c->inv_i_b, o_scale(n, dtw)));

        OV3 t1 = c->tangent1, t2 = c->tangent2;
        OV3 ra = c->center_a, rb = c->center_b;
        OV3 vra = o_add(va, o_cross(wa, ra));
        OV3 vrb = o_add(vb, o_cross(wb, rb));
        OV3 vr = o_sub(vrb, vra);
        OV2 vt;
        vt.x = o_dot(vr, t1);
        vt.y = o_dot(vr, t2);
        OV2 tm = o_mv2(c->tangent_mass, vt);
        OV2 ni;
        ni.x = c->friction_impulse.x - tm.x;
        ni.y = c->friction_impulse.y - tm.y;
        b3r max_f = c->friction * total_n;
        b3r fl2 = ni.x * ni.x + ni.y * ni.y;
        if (fl2 > max_f * max_f && fl2 > 0.0f) {
            b3r sc = o_rsqrt_scale(max_f, fl2);
            ni.x *= sc;
            ni.y *= sc;
        }
        OV2 df;
        df.x = ni.x - c->friction_impulse.x;
        df.y = ni.y - c->friction_impulse.y;
        c->friction_impulse = ni;
        OV3 P = o_add(o_scale(t1, df.x), o_scale(t2, df.y));
        va = o_msub(va, c->inv_mass_a, P);
        wa = o_sub(wa, o_mv(c->inv_i_a, o_cross(ra, P)));
        vb = o_madd(vb, c->inv_mass_b, P);
        wb = o_add(wb, o_mv(c->inv_i_b, o_cross(rb, P)));
        o_solve_rolling(c->tangent1, c->tangent2, c->rolling, total_n, c->inv_i_a, c->inv_i_b,
            &c->rolling_impulse, &wa, &wb);
    }
    if (ba->flags & B3_FLAG_DYNAMIC) {
        ba->lin_vel = va;
        ba->ang_vel = wa;
    }
    if (bb->flags & B3_FLAG_DYNAMIC) {
        bb->lin_vel = vb;
        bb->ang_vel = wb;
    }
}

static void o_solve_contacts(OWorld* w, b3r inv_h, b3r contact_speed, int use_bias) {    /* :415-437 */
    for (int i = 0; i < w->h->contact_count; i++) {
        OContact* c = &w->contacts[i];
        o_solve_one_contact(c, &w->bodies[c->body_a], &w->bodies[c->body_b], inv_h, contact_speed, use_bias);
    }
}

static void o_apply_restitution(OWorld* w, b3r threshold) {                              /* :439-480 */
    for (int i = 0; i < w->h->contact_count; i++) {
        OContact* c = &w->contacts[i];
        if (c->restitution == 0.0f) continue;
        OBody* ba = &w->bodies[c->body_a];
        OBody* bb = &w->bodies[c->body_b];
        OV3 va = ba->lin_vel, wa = ba->ang_vel, vb = bb->lin_vel, wb = bb->ang_vel;
        OV3 n = c->normal;
        for (int p = 0; p < c->point_count; p++) {
            OPoint* cp = &c->points[p];
            if (cp->rel_vel > -threshold || cp->total_normal == 0.0f) continue;
            OV3 vra = o_add(va, o_cross(wa, cp->r_a));
            OV3 vrb = o_add(vb, o_cross(wb, cp->r_b));
            b3r vn = o_dot(o_sub(vrb, vra), n);
            b3r imp = -cp->normal_mass * (vn + c->restitution * cp->rel_vel);
            b3r nimp = o_max(cp->normal_impulse + imp, 0.0f);
            imp = nimp - cp->normal_impulse;
            cp->normal_impulse = nimp;
            OV3 P = o_scale(n, imp);
            va = o_msub(va, c->inv_mass_a, P);
            wa = o_sub(wa, o_mv(c->inv_i_a, o_cross(cp->r_a, P)));
            vb = o_madd(vb, c->inv_mass_b, P);
            wb = o_add(wb, o_mv(c->inv_i_b, o_cross(cp->r_b, P)));
        }
        if (ba->flags & B3_FLAG_DYNAMIC) {
            ba->lin_vel = va;
            ba->ang_vel = wa;
        }
        if (bb->flags & B3_FLAG_DYNAMIC) {
            bb->lin_vel = vb;
            bb->ang_vel = wb;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Joints: src/puffysics/06_joints.inl:161-642, 07_packed.inl:48-81     */
/* ------------------------------------------------------------------ */

static void o_prepare_joints(OWorld* w, b3r h) {                                         /* 06:161-202 */
    for (int i = 0; i < w->h->joint_count; i++) {
        OJoint* j = &w->joints[i];
        const OBody* ba = &w->bodies[j->body_a];
        const OBody* bb = &w->bodies[j->body_b];
        j->inv_mass_a = ba->type == B3_DYNAMIC ? ba->inv_mass : 0.0f;
        j->inv_mass_b = bb->type == B3_DYNAMIC ? bb->inv_mass : 0.0f;
        j->inv_i_a = ba->type == B3_DYNAMIC ? ba->inv_i_world : o_m0();
        j->inv_i_b = bb->type == B3_DYNAMIC ? bb->inv_i_world : o_m0();
        OM3 isum = o_madd3(j->inv_i_a, j->inv_i_b);
        j->fixed_rotation = o_dot(isum.cx, o_cross(isum.cy, isum.cz)) < 1.0e-20f;
        j->softness = o_make_soft(j->constraint_hertz, j->constraint_damping, h);
        j->frame_q_a = o_qmul(ba->rotation, j->local_rot_a);
        j->frame_q_b = o_qmul(bb->rotation, j->local_rot_b);
        j->frame_p_a = o_rot(ba->rotation, o_sub(j->local_anchor_a, ba->local_center));
        j->frame_p_b = o_rot(bb->rotation, o_sub(j->local_anchor_b, bb->local_center));
        j->delta_center = o_sub(bb->center, ba->center);
        if (j->type == B3_JOINT_WELD) {
            j->angular_mass = o_inv3(isum);
            j->linear_spring = j->linear_hertz == 0.0f ? j->softness
                : o_make_soft(j->linear_hertz, j->linear_damping, h);
            j->angular_spring = j->angular_hertz == 0.0f ? j->softness
                : o_make_soft(j->angular_hertz, j->angular_damping, h);
        } else {
            OV3 axis = o_rot(j->frame_q_a, o_v(0.0f, 0.0f, 1.0f));
            b3r k = o_dot(axis, o_mv(isum, axis));
            b3r one = 1.0f;
            j->axial_mass = k > 0.0f ? one / k : 0.0f;
            j->rotation_axis = axis;
            OQ rel = o_qinv_mul(j->frame_q_a, j->frame_q_b);
            o_hinge_perps(j->frame_q_a, rel, &j->perp_x, &j->perp_y);
            j->spring_softness = o_make_soft(j->hertz, j->damping_ratio, h);
        }
    }
}

static void o_warm_start_joints(OWorld* w) {                                             /* 06:204-239 */
    for (int i = 0; i < w->h->joint_count; i++) {
        OJoint* j = &w->joints[i];
        OBody* ba = &w->bodies[j->body_a];
        OBody* bb = &w->bodies[j->body_b];
        OV3 ra = o_rot(ba->delta_rot, j->frame_p_a);
        OV3 rb = o_rot(bb->delta_rot, j->frame_p_b);
        OV3 ang = j->angular_impulse;
        if (j->type == B3_JOINT_REVOLUTE) {
            b3r axial = j->spring_impulse + j->motor_impulse + j->lower_impulse - j->upper_impulse;
            ang = o_add(o_scale(j->perp_x, j->perp_impulse.x), o_scale(j->perp_y, j->perp_impulse.y));
            ang = o_madd(ang, axial, j->rotation_axis);
        }
        if (ba->flags & B3_FLAG_DYNAMIC) {
            ba->lin_vel = o_msub(ba->lin_vel, j->inv_mass_a, j->linear_impulse);
            ba->ang_vel = o_sub(ba->ang_vel, o_mv(j->inv_i_a, o_add(o_cross(ra, j->linear_impulse), ang)));
        }
        if (bb->flags & B3_FLAG_DYNAMIC) {
            bb->lin_vel = o_madd(bb->lin_vel, j->inv_mass_b, j->linear_impulse);
            bb->ang_vel = o_add(bb->ang_vel, o_mv(j->inv_i_b, o_add(o_cross(rb, j->linear_impulse), ang)));
        }
    }
}

static OM3 o_point_k(b3r ma, b3r mb, OM3 ia, OM3 ib, OV3 ra, OV3 rb) {                  /* 06:241-255 */
    b3r msum = ma + mb;
    OM3 k;
    k.cx = o_v(msum, 0.0f, 0.0f);
    k.cy = o_v(0.0f, msum, 0.0f);
    k.cz = o_v(0.0f, 0.0f, msum);
    k.cx = o_sub(k.cx, o_cross(ra, o_mv(ia, o_v(0.0f, ra.z, -ra.y))));
    k.cy = o_sub(k.cy, o_cross(ra, o_mv(ia, o_v(-ra.z, 0.0f, ra.x))));
    k.cz = o_sub(k.cz, o_cross(ra, o_mv(ia, o_v(ra.y, -ra.x, 0.0f))));
    k.cx = o_sub(k.cx, o_cross(rb, o_mv(ib, o_v(0.0f, rb.z, -rb.y))));
    k.cy = o_sub(k.cy, o_cross(rb, o_mv(ib, o_v(-rb.z, 0.0f, rb.x))));
    k.cz = o_sub(k.cz, o_cross(rb, o_mv(ib, o_v(rb.y, -rb.x, 0.0f))));
    return k;
}

static void o_solve_point(OJoint* j, const OBody* ba, const OBody* bb, OV3* va, OV3* wa, /* 06:257-282 */
        OV3* vb, OV3* wb, OSoft soft, int use_bias) {
    OV3 ra = o_rot(ba->delta_rot, j->frame_p_a);
    OV3 rb = o_rot(bb->delta_rot, j->frame_p_b);
    OV3 cdot = o_sub(o_add(*vb, o_cross(*wb, rb)), o_add(*va, o_cross(*wa, ra)));
    OV3 bias = o_v(0.0f, 0.0f, 0.0f);
    b3r mscale = 1.0f, iscale = 0.0f;
    if (use_bias) {
        OV3 sep = o_add(o_add(o_sub(bb->delta_pos, ba->delta_pos), o_sub(rb, ra)), j->delta_center);
        bias = o_scale(sep, soft.bias_rate);
        mscale = soft.mass_scale;
        iscale = soft.impulse_scale;
    }
    OV3 b = o_solve3(o_point_k(j->inv_mass_a, j->inv_mass_b, j->inv_i_a, j->inv_i_b, ra, rb),
        o_add(cdot, bias));
    OV3 impulse = o_msub(o_scale(b, -mscale), iscale, j->linear_impulse);
    j->linear_impulse = o_add(j->linear_impulse, impulse);
    *va = o_msub(*va, j->inv_mass_a, impulse);
    *wa = o_sub(*wa, o_mv(j->inv_i_a, o_cross(ra, impulse)));
    *vb = o_madd(*vb, j->inv_mass_b, impulse);
    *wb = o_add(*wb, o_mv(j->inv_i_b, o_cross(rb, impulse)));
}

static void o_solve_weld(OJoint* j, OBody* ba, OBody* bb, int use_bias) {                /* 06:285-332 */
    OV3 va = ba->lin_vel, wa = ba->ang_vel, vb = bb->lin_vel, wb = bb->ang_vel;
    OQ qa = o_qmul(ba->delta_rot, j->frame_q_a);
    OQ qb = o_qmul(bb->delta_rot, j->frame_q_b);
    if (o_qdot(qa, qb) < 0.0f) qb = o_qneg(qb);
    OQ rel = o_qinv_mul(qa, qb);
    if (!j->fixed_rotation) {
        OV3 bias = o_v(0.0f, 0.0f, 0.0f);
        b3r mscale = 1.0f, iscale = 0.0f;
        if (use_bias || j->angular_hertz > 0.0f) {
            OQ s = rel;
            if (rel.s < 0.0f) s = o_qneg(rel);
            OQ diff = o_q(-s.v.x, -s.v.y, -s.v.z, 1.0f - s.s);
            OV3 c = o_neg(o_rot(qa, o_scale(o_qmul(diff, o_qconj(s)).v, 2.0f)));
            bias = o_scale(c, j->angular_spring.bias_rate);
            mscale = j->angular_spring.mass_scale;
            iscale = j->angular_spring.impulse_scale;
        }
        OV3 cdot = o_sub(wb, wa);
        OV3 impulse = o_msub(o_scale(o_mv(j->angular_mass, o_add(cdot, bias)), -mscale), iscale, j->angular_impulse);
        j->angular_impulse = o_add(j->angular_impulse, impulse);
        wa = o_sub(wa, o_mv(j->inv_i_a, impulse));
        wb = o_add(wb, o_mv(j->inv_i_b, impulse));
    }
    int lin_bias = use_bias || j->linear_hertz > 0.0f;
    o_solve_point(j, ba, bb, &va, &wa, &vb, &wb, j->linear_spring, lin_bias);
    if (ba->flags & B3_FLAG_DYNAMIC) {
        ba->lin_vel = va;
        ba->ang_vel = wa;
    }
    if (bb->flags & B3_FLAG_DYNAMIC) {
        bb->lin_vel = vb;
        bb->ang_vel = wb;
    }
}

/* One clamped one-sided hinge limit row (06:419-433). */
O_FN b3r o_limit_impulse(b3r c, b3r cdot, b3r inv_h, int use_bias, OSoft softness, b3r axial_mass, b3r old) {
    b3r bias = 0.0f, mscale = 1.0f, iscale = 0.0f;
    if (c > 0.0f) {
        bias = c * inv_h;
    } else if (use_bias) {
        bias = softness.bias_rate * c;
        mscale = softness.mass_scale;
        iscale = softness.impulse_scale;
    }
    b3r dimp = -mscale * axial_mass * (cdot + bias) - iscale * old;
    return o_max(old + dimp, 0.0f);
}

static void o_solve_revolute(OJoint* j, OBody* ba, OBody* bb, b3r h, b3r inv_h, int use_bias) {  /* 06:436-642 */
    OV3 va = ba->lin_vel, wa = ba->ang_vel, vb = bb->lin_vel, wb = bb->ang_vel;
    OQ qa = o_qmul(ba->delta_rot, j->frame_q_a);
    OQ qb = o_qmul(bb->delta_rot, j->frame_q_b);
    if (o_qdot(qa, qb) < 0.0f) qb = o_qneg(qb);
    OQ rel = o_qinv_mul(qa, qb);
    OV3 axis = j->rotation_axis;
    OV3 ia_ax = o_v(0.0f, 0.0f, 0.0f);
    OV3 ib_ax = o_v(0.0f, 0.0f, 0.0f);
    b3r twist = 0.0f;
    int need_twist = (j->enable_spring || j->enable_limit || j->enable_motor) && !j->fixed_rotation;
    if (!j->fixed_rotation) {
        ia_ax = o_mv(j->inv_i_a, axis);
        ib_ax = o_mv(j->inv_i_b, axis);
    }
    if (need_twist) twist = o_twist(rel);
    if (j->enable_spring && !j->fixed_rotation) {                                        /* :480-500 */
        b3r c = twist - j->target_angle;
        b3r bias = j->spring_softness.bias_rate * c;
        b3r mscale = j->spring_softness.mass_scale;
        b3r iscale = j->spring_softness.impulse_scale;
        b3r cdot = o_dot(o_sub(wb, wa), axis);
        b3r dimp = -mscale * j->axial_mass * (cdot + bias) - iscale * j->spring_impulse;
        b3r old = j->spring_impulse;
        b3r nimp = old + dimp;
        if (j->max_motor_torque > 0.0f) {
            b3r maxp = j->max_motor_torque * h;
            nimp = o_clamp(nimp, -maxp, maxp);
        }
        dimp = nimp - old;
        j->spring_impulse = nimp;
        wa = o_msub(wa, dimp, ia_ax);
        wb = o_madd(wb, dimp, ib_ax);
    }
    if (j->enable_motor && !j->fixed_rotation) {                                         /* :501-527 */
        int blocked = 0;
        if (j->enable_limit) {
            if (twist >= j->upper_angle - 0.01f && j->motor_speed > 0.0f) blocked = 1;
            if (twist <= j->lower_angle + 0.01f && j->motor_speed < 0.0f) blocked = 1;
        }
        if (blocked) {
            j->motor_impulse = 0.0f;
        } else {
            b3r cdot = o_dot(o_sub(wb, wa), axis) - j->motor_speed;
            b3r dimp = -j->axial_mass * cdot;
            b3r nimp = j->motor_impulse + dimp;
            b3r maxp = j->max_motor_torque * h;
            nimp = o_clamp(nimp, -maxp, maxp);
            dimp = nimp - j->motor_impulse;
            j->motor_impulse = nimp;
            wa = o_msub(wa, dimp, ia_ax);
            wb = o_madd(wb, dimp, ib_ax);
        }
    }
    if (j->enable_limit && !j->fixed_rotation) {                                         /* :528-550 */
        b3r old = j->lower_impulse;
        j->lower_impulse = o_limit_impulse(twist - j->lower_angle, o_dot(o_sub(wb, wa), axis), inv_h,
            use_bias, j->softness, j->axial_mass, old);
        b3r dimp = j->lower_impulse - old;
        wa = o_msub(wa, dimp, ia_ax);
        wb = o_madd(wb, dimp, ib_ax);
        old = j->upper_impulse;
        j->upper_impulse = o_limit_impulse(j->upper_angle - twist, o_dot(o_sub(wa, wb), axis), inv_h,
            use_bias, j->softness, j->axial_mass, old);
        dimp = j->upper_impulse - old;
        wa = o_madd(wa, dimp, ia_ax);
        wb = o_msub(wb, dimp, ib_ax);
    }
    if (!j->fixed_rotation) {                                                             /* :551-603 */
        OV2 bias;
        bias.x = 0.0f;
        bias.y = 0.0f;
        b3r mscale = 1.0f, iscale = 0.0f;
        if (use_bias) {
            bias.x = j->softness.bias_rate * rel.v.x;
            bias.y = j->softness.bias_rate * rel.v.y;
            mscale = j->softness.mass_scale;
            iscale = j->softness.impulse_scale;
        }
        OV3 px, py;
        o_hinge_perps(qa, rel, &px, &py);
        j->perp_x = px;
        j->perp_y = py;
        OM3 isum = o_madd3(j->inv_i_a, j->inv_i_b);
        OM2 kang;
        kang.cx.x = o_dot(px, o_mv(isum, px));
        kang.cy.y = o_dot(py, o_mv(isum, py));
        kang.cx.y = o_dot(px, o_mv(isum, py));
        kang.cy.x = kang.cx.y;
        OV3 wrel = o_sub(wb, wa);
        OV2 rhs;
        rhs.x = o_dot(wrel, px) + bias.x;
        rhs.y = o_dot(wrel, py) + bias.y;
        OV2 sol = o_solve2(kang, rhs);
        OV2 old = j->perp_impulse;
        OV2 dimp;
        dimp.x = -mscale * sol.x - iscale * old.x;
        dimp.y = -mscale * sol.y - iscale * old.y;
        j->perp_impulse.x += dimp.x;
        j->perp_impulse.y += dimp.y;
        OV3 ang = o_add(o_scale(px, dimp.x), o_scale(py, dimp.y));
        wa = o_sub(wa, o_mv(j->inv_i_a, ang));
        wb = o_add(wb, o_mv(j->inv_i_b, ang));
    }
    o_solve_point(j, ba, bb, &va, &wa, &vb, &wb, j->softness, use_bias);                /* :631 */
    if (ba->flags & B3_FLAG_DYNAMIC) {
        ba->lin_vel = va;
        ba->ang_vel = wa;
    }
    if (bb->flags & B3_FLAG_DYNAMIC) {
        bb->lin_vel = vb;
        bb->ang_vel = wb;
    }
}

static void o_solve_joints(OWorld* w, b3r h, b3r inv_h, int use_bias) {                  /* 07:48-81, 670-679 */
    int iters = use_bias ? B3_JOINT_ITERS : B3_RELAX_ITERS;
    for (int iter = 0; iter < iters; iter++) {
        for (int i = 0; i < w->h->joint_count; i++) {
            OJoint* j = &w->joints[i];
            OBody* ba = &w->bodies[j->body_a];
            OBody* bb = &w->bodies[j->body_b];
            if (j->type == B3_JOINT_WELD) o_solve_weld(j, ba, bb, use_bias);
            else o_solve_revolute(j, ba, bb, h, inv_h, use_bias);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Integration and the step driver: src/puffysics/09_step.inl           */
/* ------------------------------------------------------------------ */

/* A force law in the B3_USER_FORCES hook (01_config.inl:189-198): it adds
 * to the bodies' applied forces and torques of the world it is given. */
typedef struct OForceLaw {
    void (*apply)(const struct OForceLaw* law, OWorld* w, b3r h);
    b3r gravity, softening;   /* o_gravity_law */
    const float* masses;      /* o_gravity_law: this world's masses, or NULL */
} OForceLaw;

/* Plummer-softened gravity between the world's bodies (nbody_rigid.cuh:
 * 15-66: b3_nbody_masses and b3_nbody_accumulate), with the sources at the
 * current centers, center + delta_pos, as the hook reads poses
 * (01_config.inl:189-192). */
static void o_gravity_law(const OForceLaw* f, OWorld* w, b3r h) {
    (void)h;
    int n = w->h->body_count;
    b3r masses[n > 0 ? n : 1];
    for (int i = 0; i < n; i++) {                                                        /* :14-33 */
        OBody* b = &w->bodies[i];
        b3r one = 1.0f;
        masses[i] = f->masses ? f->masses[i] : (b->type == B3_DYNAMIC && b->inv_mass > 0 ? one / b->inv_mass : 0);
    }
    b3r eps2 = f->softening * f->softening;                                              /* :35-66 */
    for (int i = 0; i < n; i++) {
        if (masses[i] == 0) continue;
        OBody* a = &w->bodies[i];
        for (int j = i + 1; j < n; j++) {
            OBody* b = &w->bodies[j];
            if (masses[j] == 0 || (a->type != B3_DYNAMIC && b->type != B3_DYNAMIC)) continue;
            OV3 r = o_sub(o_add(b->center, b->delta_pos), o_add(a->center, a->delta_pos));
            b3r q = o_dot(r, r) + eps2;
            b3r one = 1.0f;
            b3r inv = one / o_sqrt(q);
            OV3 force = o_scale(r, f->gravity * masses[i] * masses[j] * inv * inv * inv);
            if (a->type == B3_DYNAMIC) a->force = o_add(a->force, force);
            if (b->type == B3_DYNAMIC) b->force = o_sub(b->force, force);
        }
    }
}

static void o_integrate_velocities(OWorld* w, b3r h, const OForceLaw* law) {             /* :5-18, 20-53 */
    OV3 saved_force[law ? w->h->body_count + 1 : 1], saved_torque[law ? w->h->body_count + 1 : 1];
    if (law) {                                                                           /* :25-31 */
        for (int i = 0; i < w->h->body_count; i++) {
            saved_force[i] = w->bodies[i].force;
            saved_torque[i] = w->bodies[i].torque;
        }
        law->apply(law, w, h);
    }
    OV3 g = w->h->gravity;
    for (int i = 0; i < w->h->body_count; i++) {
        OBody* b = &w->bodies[i];
        if (b->type != B3_DYNAMIC) continue;
        b3r one = 1.0f;
        b3r ld = one / (1.0f + h * b->linear_damping);
        b3r ad = one / (1.0f + h * b->angular_damping);
        b3r gs = b->inv_mass > 0.0f ? b->gravity_scale : 0.0f;
        OV3 dv = o_add(o_scale(b->force, h * b->inv_mass), o_scale(g, h * gs));
        b->lin_vel = o_madd(dv, ld, b->lin_vel);
        OV3 dw = o_scale(o_mv(b->inv_i_world, b->torque), h);
        b->ang_vel = o_madd(dw, ad, b->ang_vel);
    }
    if (law) {                                                                           /* :33-38 */
        for (int i = 0; i < w->h->body_count; i++) {
            w->bodies[i].force = saved_force[i];
            w->bodies[i].torque = saved_torque[i];
        }
    }
}

/* b3_integrate_position_state (:55-93) on one body. */
static void o_integrate_position_one(OBody* b, b3r h, b3r max_lin2, b3r max_ang2, b3r max_lin, b3r max_ang) {
    if (b->type == B3_STATIC) return;
    OV3 v = b->lin_vel, av = b->ang_vel;
    if (b->flags & B3_LOCK_LIN_X) v.x = 0.0f;
    if (b->flags & B3_LOCK_LIN_Y) v.y = 0.0f;
    if (b->flags & B3_LOCK_LIN_Z) v.z = 0.0f;
    if (b->flags & B3_LOCK_ANG_X) av.x = 0.0f;
    if (b->flags & B3_LOCK_ANG_Y) av.y = 0.0f;
    if (b->flags & B3_LOCK_ANG_Z) av.z = 0.0f;
    b3r v2 = o_len2(v);
    if (v2 > max_lin2 && v2 > 0.0f) v = o_scale(v, o_rsqrt_scale(max_lin, v2));
    b3r w2 = o_len2(av);
    if (w2 > max_ang2 && w2 > 0.0f) av = o_scale(av, o_rsqrt_scale(max_ang, w2));
    b->lin_vel = v;
    b->ang_vel = av;
    b->delta_pos = o_madd(b->delta_pos, h, v);
    b->delta_rot = o_qintegrate(b->delta_rot, o_scale(av, h));
}

static void o_integrate_positions(OWorld* w, b3r h, b3r inv_dt, b3r max_lin) {           /* :95-107 */
    b3r max_ang = B3_MAX_ROTATION * inv_dt;
    b3r max_lin2 = max_lin * max_lin;
    b3r max_ang2 = max_ang * max_ang;
    for (int i = 0; i < w->h->body_count; i++)
        o_integrate_position_one(&w->bodies[i], h, max_lin2, max_ang2, max_lin, max_ang);
}

static void o_finalize(OWorld* w) {                                                      /* :109-130 */
    for (int i = 0; i < w->h->body_count; i++) {
        OBody* b = &w->bodies[i];
        if (b->type == B3_STATIC) continue;
        b->center = o_add(b->center, b->delta_pos);
        b->rotation = o_qnorm(o_qmul(b->delta_rot, b->rotation));
        b->position = o_sub(b->center, o_rot(b->rotation, b->local_center));
        b->delta_pos = o_v(0.0f, 0.0f, 0.0f);
        b->delta_rot = o_qid();
        b->force = o_v(0.0f, 0.0f, 0.0f);
        b->torque = o_v(0.0f, 0.0f, 0.0f);
        if (b->type == B3_DYNAMIC) b->inv_i_world = o_world_inv_i(b->rotation, b->inv_inertia);
    }
}

#include "art.inc"

/* b3_solve_contacts (08_contacts.inl:422-437): with articulated contacts on,
 * a world with joints and contacts whose tree builds takes the articulated
 * sweep. */
static void o_solve_contacts_mode(OWorld* w, b3r inv_h, b3r contact_speed, int use_bias, int art_contacts) {
    if (art_contacts && w->h->joint_count > 0 && w->h->contact_count > 0) {
        OArt art;
        if (o_art_bind(&art, w)) {
            o_art_solve_contacts(&art, w, inv_h, contact_speed, use_bias, 1);
            o_art_free(&art);
            return;
        }
    }
    o_solve_contacts(w, inv_h, contact_speed, use_bias);
}

/* The contacts' share of b3_warm_start (08_contacts.inl:194-232): the
 * articulated sweep when that build option is on and the world has joints
 * and contacts, the independent-body impulses otherwise. */
static void o_warm_contacts(OWorld* w, int art_contacts) {
    if (art_contacts && w->h->joint_count > 0 && w->h->contact_count > 0) {
        OArt art;
        if (o_art_bind(&art, w)) {
            o_art_warm_start(&art, w);
            o_art_free(&art);
            return;
        }
    }
    for (int i = 0; i < w->h->contact_count; i++) {
        OContact* c = &w->contacts[i];
        o_warm_one_contact(c, &w->bodies[c->body_a], &w->bodies[c->body_b]);
    }
}

static void o_step(OWorld* w, b3r dt, int substeps, const OForceLaw* law, int art_contacts) {  /* :148-264 */
    if (dt <= 0.0f) return;
    int subs = substeps < 1 ? 1 : substeps;
    b3r one = 1.0f;
    b3r h = dt / (b3r)(float)subs;
    b3r inv_dt = one / dt;
    b3r inv_h = (b3r)(float)subs * inv_dt;
    b3r hertz = o_min(w->h->contact_hertz, 0.25f * inv_h);
    OSoft cs = o_make_soft(hertz, w->h->contact_damping, h);
    OSoft ss = o_make_soft(2.0f * hertz, 0.5f * w->h->contact_damping, h);
    /* b3_step_begin :159-165 */
    o_find_contacts(w);
    for (int i = 0; i < w->h->contact_count; i++) {
        OContact* c = &w->contacts[i];
        o_prepare_one_contact(c, &w->bodies[c->body_a], &w->bodies[c->body_b], cs, ss);
    }
    o_prepare_joints(w, h);
    o_warm_contacts(w, art_contacts);
    o_warm_start_joints(w);
    /* b3_step_sub :167-181 */
    for (int s = 0; s < subs; s++) {
        o_integrate_velocities(w, h, law);
        o_solve_contacts_mode(w, inv_h, w->h->contact_speed, 1, art_contacts);
        o_solve_joints(w, h, inv_h, 1);
        o_integrate_positions(w, h, inv_dt, w->h->max_linear_speed);
        o_solve_contacts_mode(w, inv_h, w->h->contact_speed, 0, art_contacts);
        o_solve_joints(w, h, inv_h, 0);
        o_apply_restitution(w, w->h->restitution_threshold);
    }
    o_finalize(w);
}

/* ------------------------------------------------------------------ */
/* Exported entry points                                               */
/* ------------------------------------------------------------------ */

size_t ocpu_world_size(unsigned long long sig) {
    B3Layout L;
    return b3_layout_of(sig, &L) ? L.world_size : 0;
}

void ocpu_step(void* world, unsigned long long sig, float dt, int substeps) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    o_step(&w, dt, substeps, NULL, 0);
}

void ocpu_step_art(void* world, unsigned long long sig, float dt, int substeps) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    o_step(&w, dt, substeps, NULL, 1);
}

void ocpu_art_step(void* world, unsigned long long sig, float dt, int substeps) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    o_art_step(&w, dt, substeps);
}

void ocpu_step_gravity(void* world, unsigned long long sig, float dt, int substeps, float gravity,
        float softening, const float* masses) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    OForceLaw law = {o_gravity_law, gravity, softening, masses};
    o_step(&w, dt, substeps, &law, 0);
}

void ocpu_find_contacts(void* world, unsigned long long sig) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    o_find_contacts(&w);
}

static int o_batch_valid(void* data, size_t stride, size_t off, int count, size_t wsize) {  /* b3_batch.cuh:21-27 */
    if (count < 0 || wsize == 0) return 0;
    if (count == 0) return 1;
    return data != NULL && stride >= wsize && off <= stride - wsize && (size_t)count <= SIZE_MAX / stride;
}

int ocpu_batch_step(void* data, size_t stride, size_t world_offset, int count, unsigned long long sig,
        float dt, int substeps, const unsigned char* active) {                          /* b3_batch.cuh:39-48 */
    size_t wsize = ocpu_world_size(sig);
    if (!o_batch_valid(data, stride, world_offset, count, wsize) || !isfinite(dt) || dt < 0 || substeps < 1)
        return 0;
    if (dt == 0) return 1;
    for (int i = 0; i < count; i++)
        if (!active || active[i])
            ocpu_step((unsigned char*)data + (size_t)i * stride + world_offset, sig, dt, substeps);
    return 1;
}

int ocpu_batch_restore(void* data, size_t stride, size_t world_offset, int count, unsigned long long sig,
        const void* initial, const unsigned char* reset) {                              /* b3_batch.cuh:53-60 */
    size_t wsize = ocpu_world_size(sig);
    if (!o_batch_valid(data, stride, world_offset, count, wsize) || (count && !initial)) return 0;
    for (int i = 0; i < count; i++)
        if (!reset || reset[i])
            memcpy((unsigned char*)data + (size_t)i * stride + world_offset,
                (const unsigned char*)initial + (size_t)i * wsize, wsize);
    return 1;
}

void ocpu_apply_force(void* world, unsigned long long sig, int body, float x, float y, float z) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    w.bodies[body].force = o_add(w.bodies[body].force, o_v(x, y, z));
}

void ocpu_apply_torque(void* world, unsigned long long sig, int body, float x, float y, float z) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    w.bodies[body].torque = o_add(w.bodies[body].torque, o_v(x, y, z));
}

void ocpu_apply_linear_impulse(void* world, unsigned long long sig, int body, float x, float y, float z) {
    OWorld w;
    if (!o_view(&w, world, sig)) return;
    OBody* b = &w.bodies[body];
    if (b->type == B3_DYNAMIC) b->lin_vel = o_madd(b->lin_vel, b->inv_mass, o_v(x, y, z));
}
