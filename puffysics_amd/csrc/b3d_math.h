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

/* ---- sinf and cosf with the host C library's bits ----
 *
 * b3_q_axis_angle calls libm sinf and cosf (03_math.inl:321-326); on its CPU
 * path glibc 2.35 evaluates them by the method of Arm's optimized-routines
 * (Szabolcs Nagy, 2018, sincosf.h, which glibc carries as
 * sysdeps/ieee754/flt-32):
 *   - the argument goes to double; |x| < pi/4 is evaluated directly (and
 *     |x| < 2^-12 returns x, or 1 for the cosine);
 *   - |x| < 120 is reduced by n = round(x 2/pi) as x - n pi/2, with n taken
 *     from the integer part of x (2/pi) 2^24 plus 2^23, shifted;
 *   - larger |x| is reduced with 2/pi as a table of 32-bit windows of its
 *     bits, three products of the 24-bit mantissa giving a 62-bit fixed
 *     point fraction (Payne and Hanek);
 *   - n mod 4 picks the sign and whether the sine or the cosine polynomial
 *     runs on the reduced argument: x + x^3 (s1 + x^2 s2 + x^4 s3), or
 *     c0 + c1 x^2 + c2 x^4 + c3 x^6 + c4 x^8, in double, rounded once to
 *     float.
 * The coefficients are that source's hex doubles.  glibc on an x86-64 host
 * with FMA runs its FMA build, in which the compiler contracts every
 * a + b c of the polynomials and the reduction's x - n pi/2 into one fused
 * operation; the functions below make exactly those fma calls (and nothing
 * else is contracted: -ffp-contract=off).  Checked on all 2^32 floats
 * against this host's sinf and cosf (tests/test_sincos.py), and on the
 * device against the host's (tests/test_gpu_sincos.py). */
struct SinCosTab { double sign[4], hpi_inv, hpi, c0, c1, c2, c3, c4, s1, s2, s3; };
B3D_FN const SinCosTab& sincos_tab(int k) {
    /* k = 1: the quadrants where the cosine polynomial's sign is flipped */
    static constexpr SinCosTab t[2] = {
        {{1.0, -1.0, -1.0, 1.0}, 0x1.45f306dc9c883p+23, 0x1.921fb54442d18p+0, 0x1p+0, -0x1.ffffffd0c621cp-2,
         0x1.55553e1068f19p-5, -0x1.6c087e89a359dp-10, 0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
         0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13},
        {{1.0, -1.0, -1.0, 1.0}, 0x1.45f306dc9c883p+23, 0x1.921fb54442d18p+0, -0x1p+0, 0x1.ffffffd0c621cp-2,
         -0x1.55553e1068f19p-5, 0x1.6c087e89a359dp-10, -0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
         0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13}};
    return t[k];
}
/* 2/pi: window i (i >= 3) holds bits 8 (i - 3) .. 8 (i - 3) + 31 of its
 * binary fraction, windows 0-2 its first 8, 16 and 24 bits. */
B3D_FN uint32_t two_over_pi_window(int i) {
    static constexpr uint32_t w[24] = {
        0x000000a2, 0x0000a2f9, 0x00a2f983, 0xa2f9836e, 0xf9836e4e, 0x836e4e44, 0x6e4e4415, 0x4e441529,
        0x441529fc, 0x1529fc27, 0x29fc2757, 0xfc2757d1, 0x2757d1f5, 0x57d1f534, 0xd1f534dd, 0xf534ddc0,
        0x34ddc0db, 0xddc0db62, 0xc0db6295, 0xdb629599, 0x6295993c, 0x95993c43, 0x993c4390, 0x3c439041};
    return w[i];
}
/* the exponent and top mantissa bits that the range tests compare */
B3D_FN uint32_t top12_(float x) { return (fbits_(x) >> 20) & 0x7ffu; }
/* The sine (odd n) or cosine (even n) polynomial of the reduced argument. */
B3D_FN float sincos_poly(double x, double x2, const SinCosTab& p, int n) {
    if ((n & 1) == 0) {
        double x3 = x * x2;
        double s1 = fma(x2, p.s3, p.s2);
        double x7 = x3 * x2;
        double s = fma(x3, p.s1, x);
        return (float)fma(x7, s1, s);
    }
    double x4 = x2 * x2;
    double c2 = fma(x2, p.c4, p.c3);
    double c1 = fma(x2, p.c1, p.c0);
    double x6 = x4 * x2;
    double c = fma(x4, p.c2, c1);
    return (float)fma(x6, c2, c);
}
/* x - n pi/2 for |x| < 120, n the nearest integer to x 2/pi. */
B3D_FN double sincos_reduce_small(double x, const SinCosTab& p, int* np) {
    double r = x * p.hpi_inv;
    int n = ((int32_t)r + 0x800000) >> 24;
    *np = n;
    return fma(-(double)n, p.hpi, x);
}
/* The same for finite |x| >= 120, from the float's bits. */
B3D_FN double sincos_reduce_large(uint32_t xi, int* np) {
    int i = (int)((xi >> 26) & 15u);
    int shift = (int)((xi >> 23) & 7u);
    uint32_t m = ((xi & 0xffffffu) | 0x800000u) << shift;
    uint64_t r0 = (uint64_t)(uint32_t)(m * two_over_pi_window(i));
    uint64_t r1 = (uint64_t)m * two_over_pi_window(i + 4);
    uint64_t r2 = (uint64_t)m * two_over_pi_window(i + 8);
    r0 = (r2 >> 32) | (r0 << 32);
    r0 += r1;
    uint64_t n = (r0 + (1ull << 61)) >> 62;
    r0 -= n << 62;
    *np = (int)n;
    return (double)(int64_t)r0 * 0x1.921fb54442d18p-62;
}
/* cos when want_cos, else sin, with glibc's bits for every non-NaN float. */
B3D_FN float or_sincosf(float y, bool want_cos) {
    double x = y;
    int n;
    if (top12_(y) < top12_(0x1.921fb6p-1f)) {                   /* |y| < pi/4 */
        if (top12_(y) < top12_(0x1p-12f)) return want_cos ? 1.0f : y;
        return sincos_poly(x, x * x, sincos_tab(0), want_cos ? 1 : 0);
    }
    int q;
    if (top12_(y) < top12_(120.0f)) {
        x = sincos_reduce_small(x, sincos_tab(0), &n);
        q = n;
    } else if (top12_(y) < top12_(__builtin_inff())) {
        uint32_t xi = fbits_(y);
        x = sincos_reduce_large(xi, &n);
        q = n + (int)(xi >> 31);                                /* the original sign */
    } else {
        return (y - y) / (y - y);                               /* inf or NaN: NaN */
    }
    const SinCosTab& p = sincos_tab((q & 2) ? 1 : 0);
    double s = p.sign[q & 3];
    return sincos_poly(x * s, x * x, p, want_cos ? (n ^ 1) : n);
}
B3D_FN float or_sinf(float y) { return or_sincosf(y, false); }
B3D_FN float or_cosf(float y) { return or_sincosf(y, true); }

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
