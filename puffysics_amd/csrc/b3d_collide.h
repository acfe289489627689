/*
 * b3d_collide.h - shape-pair narrowphase for the stepping kernels.
 *
 * Pure functions of two posed shapes that produce a manifold of up to four
 * points (src/puffysics/05_collision.inl).  Feature ids, the normal
 * orientation (A -> B) and the point order are the reference's, since the
 * warm start matches points by feature id and contact order is part of the
 * Gauss-Seidel order:
 *   sphere-sphere 1, capsule-capsule 2, sphere-box 3, sphere-capsule 4,
 *   capsule-box 5, box-box SAT axis 0..14 (edge axes give one support
 *   point), clipped incident-face points 16+i (reference face on A) or
 *   20+i (reference face on B).
 * The manifold lives in registers; the two 8-vertex clip polygons of the
 * box-box path live in a caller-provided per-lane buffer (LDS on the GPU).
 */
#ifndef PUFFYSICS_AMD_B3D_COLLIDE_H
#define PUFFYSICS_AMD_B3D_COLLIDE_H

#include "b3d_math.h"

namespace b3d {

constexpr float kSpeculative = 0.020f;  /* B3_SPECULATIVE, 01_config.inl:140-146 */
constexpr int kMaxManifold = 4;
constexpr int kSphere = 0, kCapsule = 1, kBox = 2;

struct Mani {
    int count;
    V3 normal;
    V3 p_a[kMaxManifold];
    V3 p_b[kMaxManifold];
    float sep[kMaxManifold];
    uint32_t feature[kMaxManifold];
};

/* A shape in world space. */
struct Posed {
    int type;
    V3 p;
    Q q;
    float radius;
    V3 half;
};

B3D_FN void mani_clear(Mani* m) { m->count = 0; m->normal = v3(0.0f, 1.0f, 0.0f); }
/* Append a point.  Slots are selected with constant indices so that the
 * manifold stays in registers. */
B3D_FN void mani_push(Mani* m, V3 pa, V3 pb, float sep, uint32_t feat) {
    if (m->count >= kMaxManifold) return;
#pragma unroll
    for (int k = 0; k < kMaxManifold; k++) {
        if (k == m->count) {
            m->p_a[k] = pa;
            m->p_b[k] = pb;
            m->sep[k] = sep;
            m->feature[k] = feat;
        }
    }
    m->count++;
}

/* Closest point to p on segment ab (05_collision.inl:5-13). */
B3D_FN V3 closest_seg(V3 a, V3 b, V3 p) {
    V3 ab = sub(b, a);
    float d = len2(ab);
    if (d <= 1.0e-12f) return a;
    float t = clampf(dot(sub(p, a), ab) / d, 0.0f, 1.0f);
    return madd(a, t, ab);
}

/* Closest points between segments a1a2 and b1b2 (05_collision.inl:15-55). */
B3D_FN void closest_segs(V3 a1, V3 a2, V3 b1, V3 b2, V3* pa, V3* pb) {
    V3 d1 = sub(a2, a1);
    V3 d2 = sub(b2, b1);
    V3 r = sub(a1, b1);
    float a = len2(d1);
    float e = len2(d2);
    float f = dot(d2, r);
    float s, t;
    if (a <= 1.0e-12f && e <= 1.0e-12f) {
        *pa = a1;
        *pb = b1;
        return;
    }
    if (a <= 1.0e-12f) {
        s = 0.0f;
        t = clampf(f / e, 0.0f, 1.0f);
    } else {
        float c = dot(d1, r);
        if (e <= 1.0e-12f) {
            t = 0.0f;
            s = clampf(-c / a, 0.0f, 1.0f);
        } else {
            float b = dot(d1, d2);
            float den = a * e - b * b;
            s = den != 0.0f ? clampf((b * f - c * e) / den, 0.0f, 1.0f) : 0.0f;
            t = (b * s + f) / e;
            if (t < 0.0f) {
                t = 0.0f;
                s = clampf(-c / a, 0.0f, 1.0f);
            } else if (t > 1.0f) {
                t = 1.0f;
                s = clampf((b - c) / a, 0.0f, 1.0f);
            }
        }
    }
    *pa = madd(a1, s, d1);
    *pb = madd(b1, t, d2);
}

/* Two spheres (05_collision.inl:83-98). */
B3D_FN void collide_balls(Mani* m, V3 ca, float ra, V3 cb, float rb, uint32_t feat) {
    mani_clear(m);
    V3 d = sub(cb, ca);
    float dist2 = len2(d);
    float rad = ra + rb;
    if (dist2 > rad * rad) return;
    float dist = sqrtf(dist2);
    V3 n = dist > 1.0e-8f ? scale(d, rsqrt(dist2)) : v3(0.0f, 1.0f, 0.0f);
    m->normal = n;
    mani_push(m, madd(ca, ra, n), msub(cb, rb, n), dist - rad, feat);
}

/* Closest point of an oriented box to p; inside points go to the nearest
 * face (05_collision.inl:100-129). */
B3D_FN V3 closest_obb(V3 c, Q q, V3 half, V3 p, int* inside, int* face) {
    V3 local = invrot(q, sub(p, c));
    V3 cl = v3(clampf(local.x, -half.x, half.x), clampf(local.y, -half.y, half.y),
        clampf(local.z, -half.z, half.z));
    int in = fabsf(local.x) <= half.x && fabsf(local.y) <= half.y && fabsf(local.z) <= half.z;
    *inside = in;
    *face = -1;
    if (in) {
        float dx = half.x - fabsf(local.x);
        float dy = half.y - fabsf(local.y);
        float dz = half.z - fabsf(local.z);
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
    }
    return xf(c, q, cl);
}

/* Sphere of radius r at p against a surface point q (05_collision.inl:131-150). */
B3D_FN void collide_ball_point(Mani* m, V3 p, float r, V3 q, int inside, V3 n_fb, uint32_t feat) {
    V3 d = sub(p, q);
    float dist2 = len2(d);
    if (!inside && dist2 > r * r) return;
    V3 n;
    float sep;
    if (inside) {
        n = dist2 > 1.0e-12f ? norm(d) : n_fb;
        sep = -len(d) - r;
    } else {
        float dist = sqrtf(dist2);
        n = scale(d, rsqrt(dist2));
        sep = dist - r;
    }
    m->normal = n;
    mani_push(m, msub(p, r, n), q, sep, feat);
}

B3D_FN void collide_sphere_box(Mani* m, V3 sc, float r, V3 bc, Q bq, V3 half) {
    mani_clear(m);
    int inside, face;
    V3 q = closest_obb(bc, bq, half, sc, &inside, &face);
    V3 ax, ay, az;
    axes(bq, &ax, &ay, &az);
    V3 n_fb = face == 0 ? ax : (face == 1 ? ay : az);
    collide_ball_point(m, sc, r, q, inside, n_fb, 3u);
}

/* Capsule segment c1c2 against a box: two rounds of closest-point
 * alternation from the segment midpoint (05_collision.inl:164-175). */
B3D_FN void collide_capsule_box(Mani* m, V3 c1, V3 c2, float r, V3 bc, Q bq, V3 half) {
    mani_clear(m);
    V3 mid = scale(add(c1, c2), 0.5f);
    int inside, face;
    V3 q = closest_obb(bc, bq, half, mid, &inside, &face);
    V3 p = closest_seg(c1, c2, q);
    q = closest_obb(bc, bq, half, p, &inside, &face);
    p = closest_seg(c1, c2, q);
    collide_ball_point(m, p, r, q, inside, v3(0.0f, 1.0f, 0.0f), 5u);
}

struct Obb { V3 c; V3 ax[3]; V3 h; };

B3D_FN Obb make_obb(V3 c, Q q, V3 h) {
    Obb o;
    o.c = c;
    o.h = h;
    axes(q, &o.ax[0], &o.ax[1], &o.ax[2]);
    return o;
}
/* Component or axis i of a box, chosen among values: the empty asm fixes
 * the loaded components as values first, since a choice among the fields'
 * addresses (what the optimiser makes of a choice among loads) keeps the
 * box in private memory. */
B3D_FN void opaque3(V3& v) {
#ifdef __HIP_DEVICE_COMPILE__
    asm("" : "+v"(v.x), "+v"(v.y), "+v"(v.z));
#else
    (void)v;
#endif
}
B3D_FN float half_i(V3 h, int i) {
    opaque3(h);
    return i == 0 ? h.x : (i == 1 ? h.y : h.z);
}
/* Field-wise choice between two boxes (a pointer select would force both
 * into memory). */
B3D_FN V3 vsel(bool c, V3 x, V3 y) { return v3(c ? x.x : y.x, c ? x.y : y.y, c ? x.z : y.z); }
B3D_FN Obb obb_sel(bool c, const Obb* x, const Obb* y) {
    Obb o;
    o.c = vsel(c, x->c, y->c);
    o.ax[0] = vsel(c, x->ax[0], y->ax[0]);
    o.ax[1] = vsel(c, x->ax[1], y->ax[1]);
    o.ax[2] = vsel(c, x->ax[2], y->ax[2]);
    o.h = vsel(c, x->h, y->h);
    return o;
}
/* Axis i of a box, selected without indexing so the box stays in registers. */
B3D_FN V3 axis_i(const Obb* o, int i) {
    V3 a0 = o->ax[0], a1 = o->ax[1], a2 = o->ax[2];
    opaque3(a0);
    opaque3(a1);
    opaque3(a2);
    return i == 0 ? a0 : (i == 1 ? a1 : a2);
}
B3D_FN V3 support(const Obb* o, V3 dir) {
    float sx = dot(o->ax[0], dir) < 0.0f ? -o->h.x : o->h.x;
    float sy = dot(o->ax[1], dir) < 0.0f ? -o->h.y : o->h.y;
    float sz = dot(o->ax[2], dir) < 0.0f ? -o->h.z : o->h.z;
    return add(o->c, add(scale(o->ax[0], sx), add(scale(o->ax[1], sy), scale(o->ax[2], sz))));
}
/* Clip polygons live in a per-lane buffer with a stride of B3D_LANES
 * floats between consecutive words (LDS on the GPU): vertex i of a polygon
 * at words 3i..3i+2.  Two polygons of kClipVerts vertices are used. */
constexpr int kClipVerts = 8;
constexpr int kClipStride = B3D_LANES;
constexpr int kClipWords = 2 * 3 * kClipVerts;
B3D_FN V3 clip_get(const float* poly, int i) {
    const float* v = poly + 3 * i * kClipStride;
    return v3(v[0], v[kClipStride], v[2 * kClipStride]);
}
B3D_FN void clip_put(float* poly, int i, V3 x) {
    float* v = poly + 3 * i * kClipStride;
    v[0] = x.x;
    v[kClipStride] = x.y;
    v[2 * kClipStride] = x.z;
}
/* Sutherland-Hodgman against one plane, at most 8 output vertices. */
B3D_FN int clip_plane(const float* in, int n, float* out, V3 pn, float po) {
    if (n <= 0) return 0;
    int c = 0;
    V3 prev = clip_get(in, n - 1);
    float pd = dot(prev, pn) - po;
    int pin = pd <= 0.0f;
    /* every input vertex is read before the first is used (unrolled over
     * the polygon's at most kClipVerts vertices) */
    V3 vin[kClipVerts];
#pragma unroll
    for (int i = 0; i < kClipVerts; i++)
        if (i < n) vin[i] = clip_get(in, i);
#pragma unroll
    for (int i = 0; i < kClipVerts; i++) {
        if (i >= n) break;
        V3 cur = vin[i];
        float cd = dot(cur, pn) - po;
        int cin = cd <= 0.0f;
        if (cin != pin && c < kClipVerts) {
            float t = pd / (pd - cd);
            clip_put(out, c++, madd(prev, t, sub(cur, prev)));
        }
        if (cin && c < kClipVerts) clip_put(out, c++, cur);
        prev = cur;
        pd = cd;
        pin = cin;
    }
    return c;
}
B3D_FN void face_pts(const Obb* o, int axis, float sign, float* out) {
    int ta = (axis + 1) % 3;
    int tb = (axis + 2) % 3;
    V3 c = madd(o->c, sign * half_i(o->h, axis), axis_i(o, axis));
    V3 a = scale(axis_i(o, ta), half_i(o->h, ta));
    V3 b = scale(axis_i(o, tb), half_i(o->h, tb));
    clip_put(out, 0, sub(sub(c, a), b));
    clip_put(out, 1, add(sub(c, a), b));
    clip_put(out, 2, add(add(c, a), b));
    clip_put(out, 3, sub(add(c, a), b));
}
B3D_FN int best_axis(const Obb* o, V3 n) {
    float b0 = fabsf(dot(o->ax[0], n));
    float b1 = fabsf(dot(o->ax[1], n));
    float b2 = fabsf(dot(o->ax[2], n));
    if (b0 >= b1 && b0 >= b2) return 0;
    return b1 >= b2 ? 1 : 2;
}
B3D_FN void mani_support(Mani* m, const Obb* a, const Obb* b, V3 n, int feat) {
    V3 pa = support(a, n);
    V3 pb = support(b, neg(n));
    mani_push(m, pa, pb, dot(sub(pb, pa), n), (uint32_t)feat);
}
/* Face axis: -1 when separated beyond the speculative margin. */
B3D_FN int try_face(float s, V3 axis, float side, float* best, V3* n, int feat, int* out_feat) {
    if (s > kSpeculative) return -1;
    if (s > *best) {
        *best = s;
        *n = side < 0.0f ? neg(axis) : axis;
        *out_feat = feat;
    }
    return 0;
}
/* Edge-edge axis, preferred only when deeper than the best by 0.002. */
B3D_FN int try_edge(float e, float ra, float rb, V3 cr, float* best, V3* n, int feat, int* out_feat) {
    float cl2 = len2(cr);
    if (cl2 <= 1.0e-3f) return 0;
    float inv = rsqrt(cl2);
    float s = (fabsf(e) - ra - rb) * inv;
    if (s > kSpeculative && cl2 > 0.05f) return -1;
    if (s > kSpeculative) return 0;
    if (s > *best + 0.002f) {
        *best = s;
        *n = e < 0.0f ? scale(cr, -inv) : scale(cr, inv);
        *out_feat = feat;
    }
    return 0;
}

/* 15-axis SAT, then reference-face clipping or a support-point pair
 * (05_collision.inl:295-461).  `clip` is the two-polygon buffer. */
B3D_FN void collide_boxes(Mani* m, const Obb* a, const Obb* b, float* clip) {
    mani_clear(m);
    V3 d = sub(b->c, a->c);
    float t0 = dot(d, a->ax[0]), t1 = dot(d, a->ax[1]), t2 = dot(d, a->ax[2]);
    float r00 = dot(a->ax[0], b->ax[0]), r01 = dot(a->ax[0], b->ax[1]), r02 = dot(a->ax[0], b->ax[2]);
    float r10 = dot(a->ax[1], b->ax[0]), r11 = dot(a->ax[1], b->ax[1]), r12 = dot(a->ax[1], b->ax[2]);
    float r20 = dot(a->ax[2], b->ax[0]), r21 = dot(a->ax[2], b->ax[1]), r22 = dot(a->ax[2], b->ax[2]);
    float ar00 = fabsf(r00), ar01 = fabsf(r01), ar02 = fabsf(r02);
    float ar10 = fabsf(r10), ar11 = fabsf(r11), ar12 = fabsf(r12);
    float ar20 = fabsf(r20), ar21 = fabsf(r21), ar22 = fabsf(r22);
    float hax = a->h.x, hay = a->h.y, haz = a->h.z;
    float hbx = b->h.x, hby = b->h.y, hbz = b->h.z;
    float best = -FLT_MAX;
    V3 n = a->ax[0];
    int feat = 0;

    if (try_face(fabsf(t0) - hax - (hbx * ar00 + hby * ar01 + hbz * ar02), a->ax[0], t0, &best, &n, 0, &feat) < 0) return;
    if (try_face(fabsf(t1) - hay - (hbx * ar10 + hby * ar11 + hbz * ar12), a->ax[1], t1, &best, &n, 1, &feat) < 0) return;
    if (try_face(fabsf(t2) - haz - (hbx * ar20 + hby * ar21 + hbz * ar22), a->ax[2], t2, &best, &n, 2, &feat) < 0) return;
    float u0 = t0 * r00 + t1 * r10 + t2 * r20;
    float u1 = t0 * r01 + t1 * r11 + t2 * r21;
    float u2 = t0 * r02 + t1 * r12 + t2 * r22;
    if (try_face(fabsf(u0) - hbx - (hax * ar00 + hay * ar10 + haz * ar20), b->ax[0], u0, &best, &n, 3, &feat) < 0) return;
    if (try_face(fabsf(u1) - hby - (hax * ar01 + hay * ar11 + haz * ar21), b->ax[1], u1, &best, &n, 4, &feat) < 0) return;
    if (try_face(fabsf(u2) - hbz - (hax * ar02 + hay * ar12 + haz * ar22), b->ax[2], u2, &best, &n, 5, &feat) < 0) return;

    if (try_edge(t2 * r10 - t1 * r20, hay * ar20 + haz * ar10, hby * ar02 + hbz * ar01, cross(a->ax[0], b->ax[0]), &best, &n, 6, &feat) < 0) return;
    if (try_edge(t2 * r11 - t1 * r21, hay * ar21 + haz * ar11, hbz * ar00 + hbx * ar02, cross(a->ax[0], b->ax[1]), &best, &n, 7, &feat) < 0) return;
    if (try_edge(t2 * r12 - t1 * r22, hay * ar22 + haz * ar12, hbx * ar01 + hby * ar00, cross(a->ax[0], b->ax[2]), &best, &n, 8, &feat) < 0) return;
    if (try_edge(t0 * r20 - t2 * r00, haz * ar00 + hax * ar20, hby * ar12 + hbz * ar11, cross(a->ax[1], b->ax[0]), &best, &n, 9, &feat) < 0) return;
    if (try_edge(t0 * r21 - t2 * r01, haz * ar01 + hax * ar21, hbz * ar10 + hbx * ar12, cross(a->ax[1], b->ax[1]), &best, &n, 10, &feat) < 0) return;
    if (try_edge(t0 * r22 - t2 * r02, haz * ar02 + hax * ar22, hbx * ar11 + hby * ar10, cross(a->ax[1], b->ax[2]), &best, &n, 11, &feat) < 0) return;
    if (try_edge(t1 * r00 - t0 * r10, hax * ar10 + hay * ar00, hby * ar22 + hbz * ar21, cross(a->ax[2], b->ax[0]), &best, &n, 12, &feat) < 0) return;
    if (try_edge(t1 * r01 - t0 * r11, hax * ar11 + hay * ar01, hbz * ar20 + hbx * ar22, cross(a->ax[2], b->ax[1]), &best, &n, 13, &feat) < 0) return;
    if (try_edge(t1 * r02 - t0 * r12, hax * ar12 + hay * ar02, hbx * ar21 + hby * ar20, cross(a->ax[2], b->ax[2]), &best, &n, 14, &feat) < 0) return;

    if (dot(n, d) < 0.0f) n = neg(n);
    m->normal = n;
    if (feat >= 6) {
        mani_support(m, a, b, n, feat);
        return;
    }
    Obb ref = obb_sel(feat < 3, a, b);
    Obb inc = obb_sel(feat < 3, b, a);
    int ref_axis = feat < 3 ? feat : feat - 3;
    V3 ref_ax = axis_i(&ref, ref_axis);
    float rd = dot(ref_ax, n);
    float ref_sign = (feat < 3 ? rd < 0.0f : rd > 0.0f) ? -1.0f : 1.0f;
    V3 rn = scale(ref_ax, ref_sign);
    int inc_axis = best_axis(&inc, rn);
    float inc_sign = dot(axis_i(&inc, inc_axis), rn) > 0.0f ? -1.0f : 1.0f;
    float* poly = clip;
    float* tmp = clip + 3 * kClipVerts * kClipStride;
    face_pts(&inc, inc_axis, inc_sign, poly);
    int count = 4;
    int ta = (ref_axis + 1) % 3;
    int tb = (ref_axis + 2) % 3;
    V3 face_c = madd(ref.c, ref_sign * half_i(ref.h, ref_axis), ref_ax);
    for (int i = 0; i < 4; i++) {
        int t = i < 2 ? ta : tb;
        float s = (i & 1) ? 1.0f : -1.0f;
        V3 cn = scale(axis_i(&ref, t), s);
        float co = dot(cn, ref.c) + half_i(ref.h, t);
        count = clip_plane(poly, count, tmp, cn, co);
        float* t2 = poly;
        poly = tmp;
        tmp = t2;
        if (count == 0) {
            mani_support(m, a, b, n, feat);
            return;
        }
    }
    float ro = dot(rn, face_c);
    for (int i = 0; i < count && m->count < kMaxManifold; i++) {
        V3 pv = clip_get(poly, i);
        float plane_s = dot(pv, rn) - ro;
        if (plane_s <= kSpeculative) {
            V3 on_ref = msub(pv, plane_s, rn);
            V3 pa = feat < 3 ? on_ref : pv;
            V3 pb = feat < 3 ? pv : on_ref;
            float sep = dot(sub(pb, pa), n);
            mani_push(m, pa, pb, sep, (feat < 3 ? 16u : 20u) + (uint32_t)i);
        }
    }
    if (m->count == 0) mani_support(m, a, b, n, feat);
}

B3D_FN void mani_flip(Mani* m) {
    m->normal = neg(m->normal);
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) {
        if (i < m->count) {
            V3 t = m->p_a[i];
            m->p_a[i] = m->p_b[i];
            m->p_b[i] = t;
        }
    }
}

/* Type-ordered dispatch; the manifold comes back oriented A -> B with every
 * separation recomputed along the final normal (05_collision.inl:472-534). */
B3D_FN void collide_pair(Mani* m, Posed A, Posed B, float* clip) {
    V3 center_a = A.p, center_b = B.p;
    int flip = 0;
    if (A.type > B.type) {
        Posed t = A;
        A = B;
        B = t;
        flip = 1;
    }
    if (A.type == kSphere && B.type == kSphere) {
        collide_balls(m, A.p, A.radius, B.p, B.radius, 1u);
    } else if (A.type == kSphere && B.type == kCapsule) {
        V3 y = rot(B.q, v3(0.0f, B.half.y, 0.0f));
        collide_balls(m, closest_seg(sub(B.p, y), add(B.p, y), A.p), B.radius, A.p, A.radius, 4u);
        mani_flip(m);
    } else if (A.type == kSphere && B.type == kBox) {
        collide_sphere_box(m, A.p, A.radius, B.p, B.q, B.half);
    } else if (A.type == kCapsule && B.type == kCapsule) {
        V3 ya = rot(A.q, v3(0.0f, A.half.y, 0.0f));
        V3 yb = rot(B.q, v3(0.0f, B.half.y, 0.0f));
        V3 ca, cb;
        closest_segs(sub(A.p, ya), add(A.p, ya), sub(B.p, yb), add(B.p, yb), &ca, &cb);
        collide_balls(m, ca, A.radius, cb, B.radius, 2u);
    } else if (A.type == kCapsule && B.type == kBox) {
        V3 y = rot(A.q, v3(0.0f, A.half.y, 0.0f));
        collide_capsule_box(m, sub(A.p, y), add(A.p, y), A.radius, B.p, B.q, B.half);
    } else {
        Obb oa = make_obb(A.p, A.q, A.half);
        Obb ob = make_obb(B.p, B.q, B.half);
        collide_boxes(m, &oa, &ob, clip);
    }
    if (flip && m->count > 0) mani_flip(m);
    if (m->count > 0) {
        if (dot(m->normal, sub(center_b, center_a)) < 0.0f) m->normal = neg(m->normal);
#pragma unroll
        for (int i = 0; i < kMaxManifold; i++)
            if (i < m->count) m->sep[i] = dot(sub(m->p_b[i], m->p_a[i]), m->normal);
    }
}

}  // namespace b3d

#endif
