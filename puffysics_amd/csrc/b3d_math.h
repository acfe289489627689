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

/* Worlds per tile, and the stride between consecutive words of one world
 * in the tiles, scratch and LDS rows: 64 (one wave) on the GPU.  A host
 * build with B3D_LANES 1 steps plain B3World structs in place (the
 * library's CPU b3_step). */
#ifndef B3D_LANES
#define B3D_LANES 64
#endif

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
/* ---- atan2f with the host C library's bits ----
 *
 * The reference's twist calls libm atan2f (03_math.inl:305-306); its CPU
 * path runs glibc 2.35, whose float atan2 is Sun's fdlibm method (fdlibm
 * 5.3, e_atan2.c and s_atan.c) in the single-precision form by Ian Lance
 * Taylor (Cygnus Support) that newlib and glibc carry:
 *   atan(x): reduce |x| to t on one of five intervals, with breakpoints at
 *   7/16, 11/16, 19/16 and 39/16 and the reductions t = x,
 *   (2x-1)/(2+x), (x-1)/(x+1), (x-1.5)/(1+1.5x) and -1/x, which are
 *   exact shifts by atan(0), atan(1/2), atan(1), atan(3/2) and atan(inf);
 *   then atan(t) = t - t (s1 + s2), an 11-term odd polynomial in t^2
 *   split into even and odd powers of t^4; the shift is added as a
 *   hi + lo pair.
 *   atan2(y, x): IEEE special cases, then atan(|y/x|) with |y/x| rounded
 *   once, signed and moved to the quadrant of (x, y) with pi as hi + lo.
 * The constants are that source's single-precision decimals, as a C
 * compiler rounds them (the first coefficient's decimal 3.3333334327e-01
 * is 0x3eaaaaab).  Every operation is a single fp32 add, multiply or
 * correctly rounded divide in the source's order, and nothing is
 * contracted (-ffp-contract=off), so device and host give the same bits.
 * This was checked against glibc's atanf on all 2^32 inputs and against
 * its atan2f on 5e9 sampled pairs, edge values included.  The host-side
 * test is in tests/test_atan2.py; the device test in
 * tests/test_gpu_atan2.py. */
B3D_FN uint32_t fbits_(float f) { return __builtin_bit_cast(uint32_t, f); }
B3D_FN float fd_atanf(float x) {
    const int32_t hx = (int32_t)fbits_(x);
    const int32_t ix = hx & 0x7fffffff;
    if (ix >= 0x4c000000) {                         /* |x| >= 2^25, or NaN */
        if (ix > 0x7f800000) return x + x;
        const float r = 0x1.921fb4p+0f + 0x1.4442d0p-24f;   /* atan(inf) hi + lo */
        return hx > 0 ? r : -0x1.921fb4p+0f - 0x1.4442d0p-24f;
    }
    int id;
    float hi = 0.0f, lo = 0.0f;
    if (ix < 0x3ee00000) {                          /* |x| < 7/16 */
        if (ix < 0x31000000) return x;              /* |x| < 2^-29 */
        id = -1;
    } else {
        x = fabsf(x);
        if (ix < 0x3f980000) {                      /* |x| < 19/16 */
            if (ix < 0x3f300000) {                  /* |x| < 11/16 */
                id = 0; x = (2.0f * x - 1.0f) / (2.0f + x);
                hi = 0x1.dac670p-2f; lo = 0x1.586ed2p-28f;      /* atan(1/2) */
            } else {
                id = 1; x = (x - 1.0f) / (x + 1.0f);
                hi = 0x1.921fb4p-1f; lo = 0x1.4442d0p-25f;      /* atan(1) */
            }
        } else {
            if (ix < 0x401c0000) {                  /* |x| < 39/16 */
                id = 2; x = (x - 1.5f) / (1.0f + 1.5f * x);
                hi = 0x1.f730bcp-1f; lo = 0x1.281f68p-25f;      /* atan(3/2) */
            } else {
                id = 3; x = -1.0f / x;
                hi = 0x1.921fb4p+0f; lo = 0x1.4442d0p-24f;      /* atan(inf) */
            }
        }
    }
    const float z = x * x;
    const float w = z * z;
    const float s1 = z * (0x1.555556p-2f + w * (0x1.24924ap-3f + w * (0x1.745cdcp-4f
        + w * (0x1.10d66ap-4f + w * (0x1.97b4b2p-5f + w * 0x1.0ad3aep-6f)))));
    const float s2 = w * (-0x1.99999ap-3f + w * (-0x1.c71c70p-4f + w * (-0x1.3b0f2ap-4f
        + w * (-0x1.dde2d6p-5f + w * -0x1.2b4442p-5f))));
    if (id < 0) return x - x * (s1 + s2);
    const float r = hi - ((x * (s1 + s2) - lo) - x);
    return hx < 0 ? -r : r;
}
B3D_FN float fd_atan2f(float y, float x) {
    const float pi_o_4 = 0x1.921fb6p-1f, pi_o_2 = 0x1.921fb6p+0f;
    const float pi = 0x1.921fb6p+1f, pi_lo = -0x1.777a5cp-24f, tiny = 1.0e-30f;
    const int32_t hx = (int32_t)fbits_(x), ix = hx & 0x7fffffff;
    const int32_t hy = (int32_t)fbits_(y), iy = hy & 0x7fffffff;
    if (ix > 0x7f800000 || iy > 0x7f800000) return x + y;      /* NaN */
    if (hx == 0x3f800000) return fd_atanf(y);                   /* x == 1 */
    const int m = ((hy >> 31) & 1) | ((hx >> 30) & 2);          /* 2 sign(x) + sign(y) */
    if (iy == 0) {
        if (m < 2) return y;
        return m == 2 ? pi + tiny : -pi - tiny;
    }
    if (ix == 0) return hy < 0 ? -pi_o_2 - tiny : pi_o_2 + tiny;
    if (ix == 0x7f800000) {
        if (iy == 0x7f800000) {
            switch (m) {
            case 0: return pi_o_4 + tiny;
            case 1: return -pi_o_4 - tiny;
            case 2: return 3.0f * pi_o_4 + tiny;
            default: return -3.0f * pi_o_4 - tiny;
            }
        }
        switch (m) {
        case 0: return 0.0f;
        case 1: return -0.0f;
        case 2: return pi + tiny;
        default: return -pi - tiny;
        }
    }
    if (iy == 0x7f800000) return hy < 0 ? -pi_o_2 - tiny : pi_o_2 + tiny;
    const int32_t k = (iy - ix) >> 23;
    float z;
    if (k > 60) z = pi_o_2 + 0.5f * pi_lo;                      /* |y/x| > 2^60 */
    else if (hx < 0 && k < -60) z = 0.0f;
    else z = fd_atanf(fabsf(y / x));
    switch (m) {
    case 0: return z;
    case 1: return -z;
    case 2: return pi - (z - pi_lo);
    default: return (z - pi_lo) - pi;
    }
}

/* Angle of the twist about local Z (03_math.inl:293-309), with the host
 * library's atan2f bits (fd_atan2f above). */
B3D_FN float twist(Q q) {
    float t = q.s < 0.0f ? fd_atan2f(-q.v.z, -q.s) : fd_atan2f(q.v.z, q.s);
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
