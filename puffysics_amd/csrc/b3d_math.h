/*
 * b3d_math.h - fp32 vector / quaternion / matrix helpers for the stepping
 * kernels.
 *
 * Every helper evaluates its terms in the same order as the reference math
 * (src/puffysics/03_math.inl), and the kernels are compiled with
 * -ffp-contract=off, so a product or sum rounds exactly where the reference
 * rounds.  That is what lets contact indices come out bit-identical: the
 * narrowphase thresholds (dist2 > r^2, s > 0.02, det <= 1e-12 ...) see the
 * same bits on both sides.
 *
 * The same header compiles for gfx950 (hipcc) and for the host (g++), so the
 * per-lane step can also be built as a host library for logic tests.
 */
#ifndef PUFFYSICS_AMD_B3D_MATH_H
#define PUFFYSICS_AMD_B3D_MATH_H

#include <float.h>
#include <math.h>
#include <stdint.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define B3D_FN __host__ __device__ static inline __attribute__((always_inline))
#define B3D_MFN __host__ __device__ inline __attribute__((always_inline))
#else
#define B3D_FN static inline __attribute__((always_inline))
#define B3D_MFN inline __attribute__((always_inline))
#endif
/* B3D_FN for free functions, B3D_MFN for member functions. */

namespace b3d {

struct V3 { float x, y, z; };
struct V2 { float x, y; };
struct Q { V3 v; float s; };        /* vector part first, like B3Quat */
struct M3 { V3 cx, cy, cz; };       /* column major, like B3Mat3 */
struct M2 { V2 cx, cy; };
struct Soft { float bias_rate, mass_scale, impulse_scale; };

/* ---- vectors (03_math.inl:5-90) ---- */
B3D_FN V3 v3(float x, float y, float z) { V3 r; r.x = x; r.y = y; r.z = z; return r; }
B3D_FN V3 zero3() { return v3(0.0f, 0.0f, 0.0f); }
B3D_FN V3 add(V3 a, V3 b) { return v3(a.x + b.x, a.y + b.y, a.z + b.z); }
B3D_FN V3 sub(V3 a, V3 b) { return v3(a.x - b.x, a.y - b.y, a.z - b.z); }
B3D_FN V3 neg(V3 a) { return v3(-a.x, -a.y, -a.z); }
B3D_FN V3 scale(V3 a, float s) { return v3(a.x * s, a.y * s, a.z * s); }
/* a + s b and a - s b, the product rounded before the sum */
B3D_FN V3 madd(V3 a, float s, V3 b) { return v3(a.x + s * b.x, a.y + s * b.y, a.z + s * b.z); }
B3D_FN V3 msub(V3 a, float s, V3 b) { return v3(a.x - s * b.x, a.y - s * b.y, a.z - s * b.z); }
B3D_FN float dot(V3 a, V3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
B3D_FN V3 cross(V3 a, V3 b) {
    return v3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
B3D_FN float len2(V3 a) { return dot(a, a); }
B3D_FN float len(V3 a) { return sqrtf(len2(a)); }
/* The library's reciprocal square roots are true divisions by sqrtf
 * (03_math.inl:57-71), not hardware rsq approximations. */
B3D_FN float rsqrt(float x) { return 1.0f / sqrtf(x); }
B3D_FN float rsqrt_scale(float a, float x) { return a / sqrtf(x); }
B3D_FN V3 norm(V3 a) {
    float l2 = len2(a);
    if (l2 > 0.0f) return scale(a, rsqrt(l2));
    return v3(0.0f, 1.0f, 0.0f);
}
B3D_FN float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }
B3D_FN float maxf(float a, float b) { return a > b ? a : b; }
B3D_FN float minf(float a, float b) { return a < b ? a : b; }

/* ---- quaternions (03_math.inl:92-158, 265-309) ---- */
B3D_FN Q q4(float x, float y, float z, float s) { Q q; q.v = v3(x, y, z); q.s = s; return q; }
B3D_FN Q qid() { return q4(0.0f, 0.0f, 0.0f, 1.0f); }
B3D_FN float qdot(Q a, Q b) { return dot(a.v, b.v) + a.s * b.s; }
B3D_FN Q qnorm(Q q) {
    float d2 = qdot(q, q);
    if (d2 <= 0.0f) return qid();
    float k = rsqrt(d2);
    return q4(q.v.x * k, q.v.y * k, q.v.z * k, q.s * k);
}
B3D_FN Q qmul(Q a, Q b) {
    Q r;
    r.v = add(add(scale(b.v, a.s), scale(a.v, b.s)), cross(a.v, b.v));
    r.s = a.s * b.s - dot(a.v, b.v);
    return r;
}
B3D_FN Q qneg(Q q) { return q4(-q.v.x, -q.v.y, -q.v.z, -q.s); }
B3D_FN Q qconj(Q q) { return q4(-q.v.x, -q.v.y, -q.v.z, q.s); }
/* conj(a) * b */
B3D_FN Q qinv_mul(Q a, Q b) {
    V3 t = cross(b.v, a.v);
    t = madd(t, a.s, b.v);
    t = msub(t, b.s, a.v);
    return q4(t.x, t.y, t.z, a.s * b.s + dot(a.v, b.v));
}
B3D_FN V3 rot(Q q, V3 v) {
    V3 t = scale(cross(q.v, v), 2.0f);
    return add(v, add(scale(t, q.s), cross(q.v, t)));
}
B3D_FN V3 invrot(Q q, V3 v) { return rot(q4(-q.v.x, -q.v.y, -q.v.z, q.s), v); }
B3D_FN V3 xf(V3 p, Q q, V3 local) { return add(p, rot(q, local)); }
/* Normalised first-order quaternion update (03_math.inl:152-157). */
B3D_FN Q qintegrate(Q q, V3 dw) {
    Q qd = q4(0.5f * dw.x, 0.5f * dw.y, 0.5f * dw.z, 0.0f);
    qd = qmul(qd, q);
    return qnorm(q4(q.v.x + qd.v.x, q.v.y + qd.v.y, q.v.z + qd.v.z, q.s + qd.s));
}
B3D_FN void axes(Q q, V3* x, V3* y, V3* z) {
    *x = rot(q, v3(1.0f, 0.0f, 0.0f));
    *y = rot(q, v3(0.0f, 1.0f, 0.0f));
    *z = rot(q, v3(0.0f, 0.0f, 1.0f));
}
/* Angle of the twist about local Z (03_math.inl:293-309, libm atan2f). */
B3D_FN float twist(Q q) {
    float t = q.s < 0.0f ? atan2f(-q.v.z, -q.s) : atan2f(q.v.z, q.s);
    return 2.0f * t;
}
/* Hinge perpendicular rows 0.5 R(qa) (e s + rel.v x e), e = x, y (03_math.inl:311-319). */
B3D_FN void hinge_perps(Q qa, Q rel, V3* px, V3* py) {
    V3 ex = v3(1.0f, 0.0f, 0.0f);
    V3 ey = v3(0.0f, 1.0f, 0.0f);
    *px = scale(rot(qa, add(scale(ex, rel.s), cross(rel.v, ex))), 0.5f);
    *py = scale(rot(qa, add(scale(ey, rel.s), cross(rel.v, ey))), 0.5f);
}

/* ---- matrices (03_math.inl:166-238, 343-359) ---- */
B3D_FN M3 m3zero() { M3 m; m.cx = zero3(); m.cy = m.cx; m.cz = m.cx; return m; }
B3D_FN V3 mv(M3 m, V3 v) { return add(add(scale(m.cx, v.x), scale(m.cy, v.y)), scale(m.cz, v.z)); }
B3D_FN M3 madd3(M3 a, M3 b) {
    M3 r;
    r.cx = add(a.cx, b.cx);
    r.cy = add(a.cy, b.cy);
    r.cz = add(a.cz, b.cz);
    return r;
}
/* R diag(inv) R^T, one column at a time. */
B3D_FN M3 world_inv_i(Q q, V3 inv) {
    V3 ax, ay, az;
    axes(q, &ax, &ay, &az);
    M3 r;
    r.cx = add(add(scale(ax, inv.x * ax.x), scale(ay, inv.y * ay.x)), scale(az, inv.z * az.x));
    r.cy = add(add(scale(ax, inv.x * ax.y), scale(ay, inv.y * ay.y)), scale(az, inv.z * az.y));
    r.cz = add(add(scale(ax, inv.x * ax.z), scale(ay, inv.y * ay.z)), scale(az, inv.z * az.z));
    return r;
}
/* Cofactor inverse; zero matrix when |det| < 1e-12. */
B3D_FN M3 inv3(M3 m) {
    V3 c0 = cross(m.cy, m.cz);
    float det = dot(m.cx, c0);
    M3 r = m3zero();
    if (fabsf(det) < 1.0e-12f) return r;
    float inv = 1.0f / det;
    V3 r0 = scale(c0, inv);
    V3 r1 = scale(cross(m.cz, m.cx), inv);
    V3 r2 = scale(cross(m.cx, m.cy), inv);
    r.cx = v3(r0.x, r1.x, r2.x);
    r.cy = v3(r0.y, r1.y, r2.y);
    r.cz = v3(r0.z, r1.z, r2.z);
    return r;
}
B3D_FN M2 inv2(M2 k) {
    float det = k.cx.x * k.cy.y - k.cx.y * k.cy.x;
    M2 r;
    r.cx.x = 0.0f; r.cx.y = 0.0f; r.cy.x = 0.0f; r.cy.y = 0.0f;
    if (fabsf(det) < 1.0e-12f) return r;
    float inv = 1.0f / det;
    r.cx.x = k.cy.y * inv;
    r.cx.y = -k.cx.y * inv;
    r.cy.x = -k.cy.x * inv;
    r.cy.y = k.cx.x * inv;
    return r;
}
B3D_FN V2 mv2(M2 m, V2 v) {
    V2 r;
    r.x = m.cx.x * v.x + m.cy.x * v.y;
    r.y = m.cx.y * v.x + m.cy.y * v.y;
    return r;
}
/* 2x2 solve that treats a non-positive determinant as singular. */
B3D_FN V2 solve2(M2 m, V2 b) {
    float det = m.cx.x * m.cy.y - m.cx.y * m.cy.x;
    V2 r;
    r.x = 0.0f; r.y = 0.0f;
    if (det <= 1.0e-12f) return r;
    float inv = 1.0f / det;
    r.x = inv * (m.cy.y * b.x - m.cy.x * b.y);
    r.y = inv * (-m.cx.y * b.x + m.cx.x * b.y);
    return r;
}
B3D_FN V3 solve3(M3 a, V3 b) { return mv(inv3(a), b); }
/* Unit vector orthogonal to n; the branch point is 1/sqrt(3). */
B3D_FN V3 perp(V3 n) {
    if (fabsf(n.x) >= 0.57735027f) return norm(v3(-n.y, n.x, 0.0f));
    return norm(v3(0.0f, -n.z, n.y));
}
/* Soft-constraint coefficients for a spring of `hertz` and damping ratio
 * `zeta` over a substep h (03_math.inl:247-263). */
B3D_FN Soft make_soft(float hertz, float zeta, float h) {
    Soft s;
    s.bias_rate = 0.0f; s.mass_scale = 0.0f; s.impulse_scale = 0.0f;
    if (hertz == 0.0f) return s;
    float omega = (2.0f * 3.14159265359f) * hertz;
    float a1 = 2.0f * zeta + h * omega;
    float a2 = h * omega * a1;
    float a3 = 1.0f / (1.0f + a2);
    s.bias_rate = omega / a1;
    s.mass_scale = a2 * a3;
    s.impulse_scale = a3;
    return s;
}

}  // namespace b3d

#endif
