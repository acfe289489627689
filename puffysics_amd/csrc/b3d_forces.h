/*
 * b3d_forces.h - built-in per-substep force laws for the B3_USER_FORCES
 * hook (01_config.inl:189-198, 09_step.inl:20-53), run by
 * step_world(L, dt, substeps, law) of b3d_lane.h.  Host and device code,
 * like the lane code.
 */
#ifndef PUFFYSICS_AMD_B3D_FORCES_H
#define PUFFYSICS_AMD_B3D_FORCES_H

#include "b3d_lane.h"

namespace b3d {

/* Plummer-softened gravity between the bodies of one world
 * (nbody_rigid.cuh:15-66), as a force law: the sources sit at the current
 * centers (center + delta_pos), and the masses are the caller's
 * gravitational masses or, without them, 1 / inv_mass of the dynamic bodies
 * (0 for the rest, which then neither feel nor source gravity).  Pairs run
 * i < j in body order; each pair adds its force to a dynamic i and
 * subtracts it from a dynamic j, so body i's sum takes the pairs (k, i),
 * k < i, first and then (i, j), j > i, as the reference's loop does. */
struct GravityLaw {
    static constexpr bool kActive = true;
    float gravity;
    float softening;
    const float* masses;  /* this world's gravitational masses, or null */

    B3D_MFN float mass(const ForceView& v, int b) const {
        if (masses) return masses[b];
        float im = v.inv_mass(b);
        return v.type(b) == kDynamic && im > 0.0f ? 1.0f / im : 0.0f;
    }
    B3D_MFN void operator()(const ForceView& v) const {
        float eps2 = softening * softening;
        int nb = v.body_count();
        for (int i = 0; i < nb; i++) {
            float mi = mass(v, i);
            if (mi == 0.0f) continue;
            int ti = v.type(i);
            V3 ci = add(v.center(i), v.delta_pos(i));
            V3 fi = v.force(i);
            for (int j = i + 1; j < nb; j++) {
                float mj = mass(v, j);
                int tj = v.type(j);
                if (mj == 0.0f || (ti != kDynamic && tj != kDynamic)) continue;
                V3 r = sub(add(v.center(j), v.delta_pos(j)), ci);
                float q = dot(r, r) + eps2;
                float inv = 1.0f / sqrtf(q);
                V3 f = scale(r, gravity * mi * mj * inv * inv * inv);
                if (ti == kDynamic) fi = add(fi, f);
                if (tj == kDynamic) v.set_force(j, sub(v.force(j), f));
            }
            v.set_force(i, fi);
        }
    }
};

/* ---- ambient fluid (ambient.h:76-370) ----
 * Buoyancy, dynamic pressure, Blasius skin friction and a lagged added-mass
 * reaction on every dynamic body, from surface samples of its shapes:
 * b3_fluid_step run as the hook's law.  As in the reference's hook, it
 * reads the start-of-step position, rotation and center and the current
 * velocities.  The sample directions use cosf / sinf of golden-angle
 * multiples, which the host tabulates (kFluidTrig entries, cos then sin) so
 * the device sees the host library's values; skin friction calls the
 * device's powf. */
constexpr float kPi = 3.14159265359f;                 /* B3_PI, 01_config.inl:140 */
constexpr float kFluidGolden = 2.39996322972865332f;  /* ambient.h:25 */
constexpr int kFluidAlphaN = 32;                      /* B3_FLUID_ALPHA_N */
constexpr int kFluidTrig = 1024;                      /* largest sample index tabulated, + 1 */

/* B3Fluid (ambient.h:24-35). */
struct FluidParams {
    float density, separation_cos, mu, drag_scale, fric_scale, added_scale;
    int sphere_samples, box_face_samples, capsule_rings, buoyancy;
};

B3D_FN float fcomp(V3 v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : v.z); }
B3D_FN V3 fset(V3 v, int i, float x) {
    if (i == 0) v.x = x;
    else if (i == 1) v.y = x;
    else v.z = x;
    return v;
}

/* Simpson rule for the ellipsoid added-mass integral (ambient.h:94-126). */
B3D_FN float fluid_alpha(float s2, float a, float b, float c) {
    float l2 = a * a;
    if (b * b > l2) l2 = b * b;
    if (c * c > l2) l2 = c * c;
    if (l2 <= 1.0e-12f) return 0.0f;
    float abc = a * b * c;
    const int n = kFluidAlphaN;
    float hstep = 1.0f / (float)n;
    float sum = 0.0f;
    for (int i = 0; i <= n; i++) {
        float t = (float)i * hstep;
        float inv = 1.0f - t * t;
        float gv = 0.0f;
        if (inv > 1.0e-12f) {
            float u = l2 * t * t / inv;
            float du = 2.0f * l2 * t / (inv * inv);
            float d = sqrtf((a * a + u) * (b * b + u) * (c * c + u));
            gv = abc * du / ((s2 + u) * d);
        }
        float wgt = (i == 0 || i == n) ? 1.0f : ((i & 1) ? 4.0f : 2.0f);
        sum += wgt * gv;
    }
    return sum * hstep / 3.0f;
}

/* One shape as the fluid law reads it. */
struct FluidShape {
    int type;
    V3 local_pos, half;
    Q local_rot;
    float radius;
};

struct FluidLaw {
    static constexpr bool kActive = true;
    FluidParams f;
    float* state;        /* this world's 6 * max_bodies + 1 words */
    const float* trig;   /* cos(kFluidGolden * k), then sin, k < kFluidTrig */

    /* Sample k of a shape in its frame (ambient.h:177-256); false past the last. */
    B3D_MFN bool sample(const FluidShape& s, int k, V3* pos, V3* nrm, float* area) const {
        if (s.type == kSphere) {
            int n = f.sphere_samples > 0 ? f.sphere_samples : 16;
            if (k >= n) return false;
            float y = 1.0f - 2.0f * ((float)k + 0.5f) / (float)n;
            float r = sqrtf(maxf(0.0f, 1.0f - y * y));
            *pos = v3(s.radius * r * trig[k], s.radius * y, s.radius * r * trig[kFluidTrig + k]);
            *nrm = norm(*pos);
            *area = 4.0f * kPi * s.radius * s.radius / (float)n;
            return true;
        }
        if (s.type == kBox) {
            int kx = f.box_face_samples > 0 ? f.box_face_samples : 1;
            int per_face = kx * kx;
            int face = k / per_face;
            int cell = k - face * per_face;
            if (face >= 6) return false;
            int axis = face >> 1;
            float sign = (face & 1) ? -1.0f : 1.0f;
            int ua = (axis + 1) % 3, va = (axis + 2) % 3;
            int iu = cell / kx, iv = cell - iu * kx;
            float hu = fcomp(s.half, ua), hv = fcomp(s.half, va);
            float u = -hu + 2.0f * hu * ((float)iu + 0.5f) / (float)kx;
            float vv = -hv + 2.0f * hv * ((float)iv + 0.5f) / (float)kx;
            V3 p = zero3();
            p = fset(p, axis, sign * fcomp(s.half, axis));
            p = fset(p, ua, u);
            p = fset(p, va, vv);
            *pos = p;
            *nrm = fset(zero3(), axis, sign);
            *area = (2.0f * hu) * (2.0f * hv) / (float)per_face;
            return true;
        }
        if (s.type == kCapsule) {
            int m = f.capsule_rings > 0 ? f.capsule_rings : 2;
            const int ka = 8;
            int cyl = m * ka;
            if (k < cyl) {
                int ring = k / ka, around = k - ring * ka;
                float y = -s.half.y + 2.0f * s.half.y * ((float)ring + 0.5f) / (float)m;
                float c = trig[around], sn = trig[kFluidTrig + around];
                *pos = v3(s.radius * c, y, s.radius * sn);
                *nrm = v3(c, 0.0f, sn);
                *area = (2.0f * kPi * s.radius) * (2.0f * s.half.y) / (float)(m * ka);
                return true;
            }
            int cn = f.sphere_samples > 0 ? f.sphere_samples : 16;
            int kc = k - cyl;
            int per_cap = cn >> 1;
            if (kc >= 2 * per_cap) return false;
            int sg = kc >= per_cap ? -1 : 1;
            int j = kc - (sg < 0 ? per_cap : 0);
            float y = 1.0f - 2.0f * ((float)j + 0.5f) / (float)cn;
            float r = sqrtf(maxf(0.0f, 1.0f - y * y));
            *pos = v3(s.radius * r * trig[j], (float)sg * s.half.y + s.radius * y, s.radius * r * trig[kFluidTrig + j]);
            *nrm = norm(*pos);
            *area = 2.0f * kPi * s.radius * s.radius / (float)per_cap;
            return true;
        }
        return false;
    }

    /* b3_fluid_body (ambient.h:258-359). */
    B3D_MFN void body(const ForceView& v, int bi, bool have_prev) const {
        if (v.type(bi) != kDynamic) return;
        const Lane& L = v.L;
        float* st = state + 6 * bi;
        V3 lin = v.lin_vel(bi), ang = v.ang_vel(bi);
        V3 position = v.position(bi), center = v.center(bi);
        Q rotation = v.rotation(bi);
        V3 g = ld3(L.w, H_GRAVITY);
        V3 f_acc = zero3(), t_acc = zero3(), a_est = zero3();
        bool use_added = have_prev && f.added_scale > 0.0f && v.h > 0.0f;
        if (use_added) a_est = scale(sub(lin, v3(st[0], st[1], st[2])), 1.0f / v.h);
        int ns = clampi(ldi(L.w, H_SHAPE_COUNT), 0, L.g.max_s);
        for (int si = 0; si < ns; si++) {
            if (ldi(L.w, sw(L, si, S_BODY)) != bi) continue;
            FluidShape s;
            s.type = ldi(L.w, sw(L, si, S_TYPE));
            s.local_pos = ld3(L.w, sw(L, si, S_LOCAL_POS));
            s.local_rot = ldq(L.w, sw(L, si, S_LOCAL_ROT));
            s.radius = ldf(L.w, sw(L, si, S_RADIUS));
            s.half = ld3(L.w, sw(L, si, S_HALF));
            V3 sp = xf(position, rotation, s.local_pos);
            Q sq = qmul(rotation, s.local_rot);
            float vol;
            if (s.type == kSphere) vol = (4.0f / 3.0f) * kPi * s.radius * s.radius * s.radius;
            else if (s.type == kBox) vol = 8.0f * s.half.x * s.half.y * s.half.z;
            else vol = kPi * s.radius * s.radius * (2.0f * s.half.y) + (4.0f / 3.0f) * kPi * s.radius * s.radius * s.radius;
            if (f.buoyancy) {
                V3 cw = xf(sp, sq, s.local_pos);   /* the centroid is local_pos for every type (:141-157) */
                V3 fb = scale(g, -f.density * vol);
                f_acc = add(f_acc, fb);
                t_acc = add(t_acc, cross(sub(cw, center), fb));
            }
            if (use_added) {
                float ax, ay, az;
                if (s.type == kSphere) {
                    ax = ay = az = s.radius;
                } else if (s.type == kBox) {
                    ax = s.half.x;
                    ay = s.half.y;
                    az = s.half.z;
                } else {
                    ax = s.radius;
                    az = s.radius;
                    ay = 1.5f * s.half.y + s.radius;
                }
                float alx = fluid_alpha(ax * ax, ax, ay, az);
                float aly = fluid_alpha(ay * ay, ax, ay, az);
                float alz = fluid_alpha(az * az, ax, ay, az);
                V3 ma = v3(f.density * vol * alx / (2.0f - alx), f.density * vol * aly / (2.0f - aly),
                    f.density * vol * alz / (2.0f - alz));
                ma = scale(ma, f.added_scale);
                for (int i = 0; i < 3; i++) {
                    V3 axis = rot(sq, fset(zero3(), i, 1.0f));
                    float proj = dot(axis, a_est);
                    f_acc = msub(f_acc, fcomp(ma, i) * proj, axis);
                }
            }
            const bool fric = f.mu > 0.0f && f.fric_scale > 0.0f;
            float Lc = 0.0f;
            if (fric) {
                if (s.type == kSphere) {
                    Lc = 2.0f * s.radius * sqrtf(kPi);
                } else if (s.type == kBox) {
                    Lc = sqrtf(8.0f * (s.half.x * s.half.y + s.half.y * s.half.z + s.half.x * s.half.z));
                } else {
                    float rr = s.radius;
                    Lc = sqrtf(2.0f * kPi * rr * (2.0f * s.half.y) + 4.0f * kPi * rr * rr);
                }
            }
            V3 lp, ln;
            float area;
            for (int k = 0; sample(s, k, &lp, &ln, &area); k++) {
                V3 p = xf(sp, sq, lp);
                V3 n = rot(sq, ln);
                V3 r = sub(p, center);
                V3 rdot = add(lin, cross(ang, r));
                float spd = len(rdot);
                if (spd <= 1.0e-9f) continue;
                float nd = dot(n, rdot);
                if (nd / spd < f.separation_cos) continue;
                float u2 = len2(rdot) - nd * nd;
                float pdyn = -0.5f * f.density * u2 * f.drag_scale;
                V3 df = scale(n, pdyn * area);
                f_acc = add(f_acc, df);
                t_acc = add(t_acc, cross(r, df));
                if (fric) {
                    V3 ut = msub(rdot, nd, n);
                    float us = len(ut);
                    if (us > 1.0e-9f) {
                        float re = f.density * us * Lc / f.mu;
                        float cf = 0.0576f * powf(re, -0.2f);
                        V3 ff = scale(ut, (-0.5f * cf * f.density * us * area) * f.fric_scale);
                        f_acc = add(f_acc, ff);
                        t_acc = add(t_acc, cross(r, ff));
                    }
                }
            }
        }
        v.set_force(bi, add(v.force(bi), f_acc));
        v.set_torque(bi, add(v.torque(bi), t_acc));
        st[0] = lin.x;
        st[1] = lin.y;
        st[2] = lin.z;
        st[3] = ang.x;
        st[4] = ang.y;
        st[5] = ang.z;
    }

    /* b3_fluid_step (ambient.h:361-370). */
    B3D_MFN void operator()(const ForceView& v) const {
        int nb = v.body_count();
        int* have = (int*)(state + 6 * v.L.g.max_b);
        bool have_prev = *have != 0;
        for (int bi = 0; bi < nb; bi++) body(v, bi, have_prev);
        *have = 1;
    }
};

/* The host table of cosf / sinf of golden-angle multiples the fluid law
 * samples with (cos in [0, kFluidTrig), sin after). */
inline void fluid_trig_table(float* out) {
    for (int k = 0; k < kFluidTrig; k++) {
        float th = kFluidGolden * (float)k;
        out[k] = cosf(th);
        out[kFluidTrig + k] = sinf(th);
    }
}

}  // namespace b3d

#endif
