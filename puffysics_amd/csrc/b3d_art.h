/*
 * b3d_art.h - the step with articulation-aware contacts (the reference's
 * B3_ART_CONTACTS=1, 01_config.inl:176-187): per-lane lane code, host and
 * device, like b3d_lane.h.
 *
 * In a world with revolute joints and contacts whose joint tree builds
 * (b3_art_bind, b3_art.cuh:488-490), the contact warm start and both
 * contact sweeps apply every impulse through the tree's Delassus operator
 * J M^-1 J^T (Featherstone's articulated-body algorithm, b3_art.cuh:
 * 607-749) instead of the independent-body masses; other worlds take the
 * ordinary path.  This step keeps contacts in the world's own rows (the
 * reference's layout) rather than in packed records: the articulated
 * solve reads and writes the same fields as the reference, and no lane's
 * record slot depends on which other lanes are articulated.
 *
 * Per-lane workspace (ArtWs): one block of kArtLinkWords words per link of
 * the tree, word-transposed across the tile's lanes like the worlds, then
 * the breadth-first search's temporaries.  The tree depends only on the
 * joints and the bodies' types and masses, which a step does not change,
 * so it is built once per step; the reference rebuilds an identical one on
 * every call.  The joint angles and rates that b3_art_refresh also
 * computes (b3_art.cuh:563-568) feed only b3_art_step's integrator, never
 * the Delassus operator: art_refresh leaves them out, art_refresh_q (the
 * integrator's) adds them.
 *
 * The second half is b3_art_step (09_step.inl:266-323), the reduced-
 * coordinate integrator: passive revolute trees move by their joint angles
 * (articulated-body dynamics, then forward kinematics), loop-closing joints
 * ("cuts") are solved as 5x5 Delassus blocks, and contacts take four
 * articulated sweeps per solve.
 */
#ifndef PUFFYSICS_AMD_B3D_ART_H
#define PUFFYSICS_AMD_B3D_ART_H

#include "b3d_lane.h"

namespace b3d {

constexpr int kArtMaxDeg = 8;        /* B3_ART_MAX_DEG, b3_art.cuh:31-33 */
constexpr int kArtMaxCuts = 8;       /* B3_ART_MAX_CUTS, :34-36 */
constexpr int kArtCutIters = 4;      /* B3_ART_CUT_ITERS, :37-39 */
constexpr int kArtContactIters = 4;  /* B3_ART_CONTACT_ITERS, :1281-1283 */
constexpr float kArtDmin = 1.0e-8f;  /* B3_ART_DMIN, :40-42 */

/* Link block words.  AL_C (bias acceleration), AL_Q / AL_QD (joint angle
 * and rate) and the child-side joint frame AL_ANCHOR_B / AL_ROT_B serve the
 * reduced integrator only.  AL_IA, AL_U, AL_DINV, AL_IC and AL_GJ are the
 * pose-only half of the Delassus operator (art_pose_pass). */
constexpr int AL_PARENT = 0, AL_BODY = 1, AL_FIXED = 2, AL_FLOATING = 3, AL_ANCHOR_A = 4, AL_ROT_A = 7,
              AL_LC = 11, AL_ILOCAL = 14, AL_MASS = 17, AL_COM = 18, AL_POS = 21, AL_ROT = 24, AL_R = 28,
              AL_SW = 31, AL_SV = 34, AL_IWW = 37, AL_IA = 46, AL_U = 82, AL_PA = 88, AL_DINV = 94, AL_A = 95,
              AL_C = 101, AL_Q = 107, AL_QD = 108, AL_ANCHOR_B = 109, AL_ROT_B = 112, AL_IC = 116, AL_GJ = 122,
              kArtLinkWords = 171;
/* A floating root's elimination record (AL_GJ + ...): pivot rows, reciprocal
 * pivots, the other rows' multipliers [k][r], and whether it completed. */
constexpr int GJ_PIV = 0, GJ_INV = 6, GJ_MUL = 12, GJ_OK = 48;
/* Search temporaries per body: degree, neighbours and joints, link of the
 * body, seen flag, queue, parent body and joint. */
constexpr int kArtBodyTmp = 2 * kArtMaxDeg + 6;

/* Words of one lane's workspace for a body capacity: the link blocks, the
 * search temporaries, then the cut count and the cut joints. */
B3D_FN int art_ws_words(int max_b) { return max_b * (kArtLinkWords + kArtBodyTmp) + 1 + kArtMaxCuts * (1 + 25); }

struct M6 { M3 ww, wv, vw, vv; };   /* spatial inertia, angular first (b3_art.cuh:54-59) */
struct S6 { V3 w, v; };             /* motion or force: (angular, linear) */
struct ArtRow { int link_a, link_b, torque; V3 ra, rb, n; };

struct ArtWs {
    float* p;   /* lane base; word k at p[k * kLanes] */
    int max_b;
    int n_links;
    B3D_MFN int li(int link, int f) const { return link * kArtLinkWords + f; }
    B3D_MFN float gf(int link, int f) const { return p[li(link, f) * kLanes]; }
    B3D_MFN int gi(int link, int f) const { return __builtin_bit_cast(int, gf(link, f)); }
    B3D_MFN V3 g3(int link, int f) const { return v3(gf(link, f), gf(link, f + 1), gf(link, f + 2)); }
    B3D_MFN Q gq(int link, int f) const { Q q; q.v = g3(link, f); q.s = gf(link, f + 3); return q; }
    B3D_MFN M3 gm3(int link, int f) const { M3 m; m.cx = g3(link, f); m.cy = g3(link, f + 3); m.cz = g3(link, f + 6); return m; }
    B3D_MFN S6 g6(int link, int f) const { S6 s; s.w = g3(link, f); s.v = g3(link, f + 3); return s; }
    B3D_MFN M6 gI(int link, int f) const { M6 m; m.ww = gm3(link, f); m.wv = gm3(link, f + 9); m.vw = gm3(link, f + 18); m.vv = gm3(link, f + 27); return m; }
    B3D_MFN void sf(int link, int f, float x) const { p[li(link, f) * kLanes] = x; }
    B3D_MFN void si(int link, int f, int x) const { sf(link, f, __builtin_bit_cast(float, x)); }
    B3D_MFN void s3(int link, int f, V3 x) const { sf(link, f, x.x); sf(link, f + 1, x.y); sf(link, f + 2, x.z); }
    B3D_MFN void sq(int link, int f, Q x) const { s3(link, f, x.v); sf(link, f + 3, x.s); }
    B3D_MFN void sm3(int link, int f, M3 m) const { s3(link, f, m.cx); s3(link, f + 3, m.cy); s3(link, f + 6, m.cz); }
    B3D_MFN void s6(int link, int f, S6 s) const { s3(link, f, s.w); s3(link, f + 3, s.v); }
    B3D_MFN void sI(int link, int f, M6 m) const { sm3(link, f, m.ww); sm3(link, f + 9, m.wv); sm3(link, f + 18, m.vw); sm3(link, f + 27, m.vv); }
    /* search temporaries of body b */
    B3D_MFN int ti(int b, int f) const { return __builtin_bit_cast(int, p[(max_b * kArtLinkWords + b * kArtBodyTmp + f) * kLanes]); }
    B3D_MFN void tsi(int b, int f, int x) const { p[(max_b * kArtLinkWords + b * kArtBodyTmp + f) * kLanes] = __builtin_bit_cast(float, x); }
    /* loop cuts: count, then joint indices */
    B3D_MFN int cut_word(int k) const { return max_b * (kArtLinkWords + kArtBodyTmp) + k; }
    B3D_MFN int n_cuts() const { return __builtin_bit_cast(int, p[cut_word(0) * kLanes]); }
    B3D_MFN int cut(int c) const { return __builtin_bit_cast(int, p[cut_word(1 + c) * kLanes]); }
    B3D_MFN void set_n_cuts(int n) const { p[cut_word(0) * kLanes] = __builtin_bit_cast(float, n); }
    B3D_MFN void set_cut(int c, int j) const { p[cut_word(1 + c) * kLanes] = __builtin_bit_cast(float, j); }
    /* each cut's regularised 5x5 Delassus block, for the iterations of one pass */
    B3D_MFN float gd(int c, int k) const { return p[cut_word(1 + kArtMaxCuts + c * 25 + k) * kLanes]; }
    B3D_MFN void sd(int c, int k, float v) const { p[cut_word(1 + kArtMaxCuts + c * 25 + k) * kLanes] = v; }
};
constexpr int AT_DEG = 0, AT_ADJ_B = 1, AT_ADJ_J = 1 + kArtMaxDeg, AT_LINK = 1 + 2 * kArtMaxDeg, AT_SEEN = AT_LINK + 1,
              AT_QUEUE = AT_SEEN + 1, AT_PARENT_B = AT_QUEUE + 1, AT_PARENT_J = AT_PARENT_B + 1;

B3D_FN S6 s6zero() { S6 s; s.w = zero3(); s.v = zero3(); return s; }
B3D_FN M6 m6zero() { M6 m; m.ww = m3zero(); m.wv = m.ww; m.vw = m.ww; m.vv = m.ww; return m; }
B3D_FN M3 m3sub(M3 a, M3 b) { M3 r; r.cx = sub(a.cx, b.cx); r.cy = sub(a.cy, b.cy); r.cz = sub(a.cz, b.cz); return r; }
B3D_FN M3 m3scale(M3 a, float s) { M3 r; r.cx = scale(a.cx, s); r.cy = scale(a.cy, s); r.cz = scale(a.cz, s); return r; }
B3D_FN M3 outer(V3 a, V3 b) { M3 r; r.cx = scale(a, b.x); r.cy = scale(a, b.y); r.cz = scale(a, b.z); return r; }
/* I m (b3_I_mul, :173-178) */
B3D_FN S6 imul(const M6& I, S6 m) {
    S6 f;
    f.w = add(mv(I.ww, m.w), mv(I.wv, m.v));
    f.v = add(mv(I.vw, m.w), mv(I.vv, m.v));
    return f;
}
B3D_FN float sdot(S6 s, S6 f) { return dot(s.w, f.w) + dot(s.v, f.v); }
B3D_FN M6 iadd(const M6& a, const M6& b) {
    M6 r;
    r.ww = madd3(a.ww, b.ww);
    r.wv = madd3(a.wv, b.wv);
    r.vw = madd3(a.vw, b.vw);
    r.vv = madd3(a.vv, b.vv);
    return r;
}
/* b3_I_shift (:189-209) */
B3D_FN M6 ishift(const M6& I, V3 r) {
    M6 O = m6zero();
    V3 cols_n[6], cols_f[6];
#pragma unroll
    for (int k = 0; k < 6; k++) {
        S6 m = s6zero();
        if (k < 3) m.w = v3(k == 0 ? 1.0f : 0.0f, k == 1 ? 1.0f : 0.0f, k == 2 ? 1.0f : 0.0f);
        else m.v = v3(k == 3 ? 1.0f : 0.0f, k == 4 ? 1.0f : 0.0f, k == 5 ? 1.0f : 0.0f);
        m.v = add(m.v, cross(m.w, r));
        S6 f = imul(I, m);
        cols_n[k] = add(f.w, cross(r, f.v));
        cols_f[k] = f.v;
    }
    O.ww.cx = cols_n[0]; O.ww.cy = cols_n[1]; O.ww.cz = cols_n[2];
    O.vw.cx = cols_f[0]; O.vw.cy = cols_f[1]; O.vw.cz = cols_f[2];
    O.wv.cx = cols_n[3]; O.wv.cy = cols_n[4]; O.wv.cz = cols_n[5];
    O.vv.cx = cols_f[3]; O.vv.cy = cols_f[4]; O.vv.cz = cols_f[5];
    return O;
}
/* b3_I_rank1 (:211-217) */
B3D_FN M6 irank1(M6 I, S6 U, float dinv) {
    I.ww = m3sub(I.ww, m3scale(outer(U.w, U.w), dinv));
    I.wv = m3sub(I.wv, m3scale(outer(U.w, U.v), dinv));
    I.vw = m3sub(I.vw, m3scale(outer(U.v, U.w), dinv));
    I.vv = m3sub(I.vv, m3scale(outer(U.v, U.v), dinv));
    return I;
}
/* a = I^-1 rhs by Gauss-Jordan with partial pivoting on the packed 6x6
 * (b3_solve6 / b3_I_pack / b3_I_solve, :230-318); false if singular. */
B3D_FN bool isolve(const M6& I, S6 rhs, S6* a) {
    float M[6][7];
    V3 cn[3] = {I.ww.cx, I.ww.cy, I.ww.cz}, cf[3] = {I.vw.cx, I.vw.cy, I.vw.cz};
    V3 dn[3] = {I.wv.cx, I.wv.cy, I.wv.cz}, df[3] = {I.vv.cx, I.vv.cy, I.vv.cz};
    for (int c = 0; c < 3; c++) {
        M[0][c] = cn[c].x; M[1][c] = cn[c].y; M[2][c] = cn[c].z;
        M[3][c] = cf[c].x; M[4][c] = cf[c].y; M[5][c] = cf[c].z;
        M[0][3 + c] = dn[c].x; M[1][3 + c] = dn[c].y; M[2][3 + c] = dn[c].z;
        M[3][3 + c] = df[c].x; M[4][3 + c] = df[c].y; M[5][3 + c] = df[c].z;
    }
    M[0][6] = rhs.w.x; M[1][6] = rhs.w.y; M[2][6] = rhs.w.z;
    M[3][6] = rhs.v.x; M[4][6] = rhs.v.y; M[5][6] = rhs.v.z;
    for (int k = 0; k < 6; k++) {
        int piv = k;
        float best = fabsf(M[k][k]);
        for (int r = k + 1; r < 6; r++) {
            float v = fabsf(M[r][k]);
            if (v > best) {
                best = v;
                piv = r;
            }
        }
        if (best < 1.0e-12f) {
            *a = s6zero();
            return false;
        }
        if (piv != k) {
            for (int c = k; c < 7; c++) {
                float t = M[k][c];
                M[k][c] = M[piv][c];
                M[piv][c] = t;
            }
        }
        float inv = 1.0f / M[k][k];
        for (int c = k; c < 7; c++) M[k][c] *= inv;
        for (int r = 0; r < 6; r++) {
            if (r == k) continue;
            float s = M[r][k];
            for (int c = k; c < 7; c++) M[r][c] -= s * M[k][c];
        }
    }
    a->w = v3(M[0][6], M[1][6], M[2][6]);
    a->v = v3(M[3][6], M[4][6], M[5][6]);
    return true;
}

/* The same elimination split in two: isolve_record runs it on I alone and
 * keeps what the right-hand side's column sees (row swaps, reciprocal
 * pivots, multipliers); isolve_replay applies those to a right-hand side.
 * Together they give isolve's result bit for bit: the column's operations
 * and their order are unchanged. */
B3D_FN void isolve_record(const ArtWs& A, int li, const M6& I) {
    float M[6][6];
    V3 cn[3] = {I.ww.cx, I.ww.cy, I.ww.cz}, cf[3] = {I.vw.cx, I.vw.cy, I.vw.cz};
    V3 dn[3] = {I.wv.cx, I.wv.cy, I.wv.cz}, df[3] = {I.vv.cx, I.vv.cy, I.vv.cz};
    for (int c = 0; c < 3; c++) {
        M[0][c] = cn[c].x; M[1][c] = cn[c].y; M[2][c] = cn[c].z;
        M[3][c] = cf[c].x; M[4][c] = cf[c].y; M[5][c] = cf[c].z;
        M[0][3 + c] = dn[c].x; M[1][3 + c] = dn[c].y; M[2][3 + c] = dn[c].z;
        M[3][3 + c] = df[c].x; M[4][3 + c] = df[c].y; M[5][3 + c] = df[c].z;
    }
    const int g = AL_GJ;
    for (int k = 0; k < 6; k++) {
        int piv = k;
        float best = fabsf(M[k][k]);
        for (int r = k + 1; r < 6; r++) {
            float v = fabsf(M[r][k]);
            if (v > best) {
                best = v;
                piv = r;
            }
        }
        if (best < 1.0e-12f) {
            A.si(li, g + GJ_OK, 0);
            return;
        }
        A.si(li, g + GJ_PIV + k, piv);
        if (piv != k) {
            for (int c = k; c < 6; c++) {
                float t = M[k][c];
                M[k][c] = M[piv][c];
                M[piv][c] = t;
            }
        }
        float inv = 1.0f / M[k][k];
        A.sf(li, g + GJ_INV + k, inv);
        for (int c = k; c < 6; c++) M[k][c] *= inv;
        for (int r = 0; r < 6; r++) {
            if (r == k) continue;
            float sr = M[r][k];
            A.sf(li, g + GJ_MUL + k * 6 + r, sr);
            for (int c = k; c < 6; c++) M[r][c] -= sr * M[k][c];
        }
    }
    A.si(li, g + GJ_OK, 1);
}
B3D_FN bool isolve_replay(const ArtWs& A, int li, S6 rhs, S6* a) {
    const int g = AL_GJ;
    if (!A.gi(li, g + GJ_OK)) {
        *a = s6zero();
        return false;
    }
    float b[6] = {rhs.w.x, rhs.w.y, rhs.w.z, rhs.v.x, rhs.v.y, rhs.v.z};
    for (int k = 0; k < 6; k++) {
        int piv = A.gi(li, g + GJ_PIV + k);
        if (piv != k) {
            float t = b[k];
            b[k] = b[piv];
            b[piv] = t;
        }
        b[k] *= A.gf(li, g + GJ_INV + k);
        for (int r = 0; r < 6; r++) {
            if (r == k) continue;
            b[r] -= A.gf(li, g + GJ_MUL + k * 6 + r) * b[k];
        }
    }
    a->w = v3(b[0], b[1], b[2]);
    a->v = v3(b[3], b[4], b[5]);
    return true;
}

/* b3_art_from_world (:340-486): the spanning forest of the revolute joints,
 * breadth first from the static bodies, then from dynamic ones; dynamic
 * bodies outside it float alone; joints that close a loop are recorded as
 * cuts (used by the reduced integrator only).  False when the tree cannot
 * be built (self-joint, a degree above kArtMaxDeg, more than kArtMaxCuts
 * cuts, or no link). */
B3D_FN bool art_build(const Lane& L, ArtWs& A) {
    const uint32_t* w = L.w;
    int nb = body_count(L);
    int nj = clampi(ldi(w, H_JOINT_COUNT), 0, L.g.max_j);
    A.n_links = 0;
    for (int i = 0; i < nb; i++) {
        A.tsi(i, AT_DEG, 0);
        A.tsi(i, AT_LINK, -1);
        A.tsi(i, AT_SEEN, 0);
        A.tsi(i, AT_PARENT_B, -1);
        A.tsi(i, AT_PARENT_J, -1);
    }
    for (int k = 0; k < nj; k++) {
        if (ldi(w, jw(L, k, J_TYPE)) != kJointRevolute) continue;
        int a = ldi(w, jw(L, k, J_BODY_A)), b = ldi(w, jw(L, k, J_BODY_B));
        if (a == b) return false;
        int da = A.ti(a, AT_DEG), db = A.ti(b, AT_DEG);
        if (da >= kArtMaxDeg || db >= kArtMaxDeg) return false;
        A.tsi(a, AT_ADJ_B + da, b);
        A.tsi(a, AT_ADJ_J + da, k);
        A.tsi(a, AT_DEG, da + 1);
        A.tsi(b, AT_ADJ_B + db, a);
        A.tsi(b, AT_ADJ_J + db, k);
        A.tsi(b, AT_DEG, db + 1);
    }
    int n_cuts = 0;
    A.set_n_cuts(0);
    for (int pass = 0; pass < 2; pass++) {
        for (int s = 0; s < nb; s++) {
            int is_static = ldi(w, bw(L, s, B_TYPE)) != kDynamic;
            if (A.ti(s, AT_DEG) == 0 || A.ti(s, AT_SEEN) || is_static != (pass == 0)) continue;
            /* the queue holds bodies in visiting order; its i-th entry is AT_QUEUE of body slot i */
            int qh = 0, qt = 0;
            A.tsi(qt++, AT_QUEUE, s);
            A.tsi(s, AT_SEEN, 1);
            A.tsi(s, AT_PARENT_B, -1);
            while (qh < qt) {
                int u = A.ti(qh++, AT_QUEUE);
                int du = A.ti(u, AT_DEG);
                for (int e = 0; e < du; e++) {
                    int v = A.ti(u, AT_ADJ_B + e);
                    if (A.ti(v, AT_SEEN)) {
                        if (A.ti(u, AT_PARENT_B) != v && A.ti(v, AT_PARENT_B) != u) {
                            int jk = A.ti(u, AT_ADJ_J + e), dup = 0;
                            for (int c = 0; c < n_cuts; c++) dup |= A.cut(c) == jk;
                            if (!dup) {
                                if (n_cuts >= kArtMaxCuts) return false;
                                A.set_cut(n_cuts++, jk);
                                A.set_n_cuts(n_cuts);
                            }
                        }
                        continue;
                    }
                    A.tsi(v, AT_SEEN, 1);
                    A.tsi(v, AT_PARENT_B, u);
                    A.tsi(v, AT_PARENT_J, A.ti(u, AT_ADJ_J + e));
                    A.tsi(qt++, AT_QUEUE, v);
                }
            }
            for (int t = 0; t < qt; t++) {
                int b = A.ti(t, AT_QUEUE);
                if (A.n_links >= A.max_b) return false;
                int li = A.n_links++;
                A.tsi(b, AT_LINK, li);
                int type = ldi(w, bw(L, b, B_TYPE));
                int pb = A.ti(b, AT_PARENT_B);
                A.si(li, AL_BODY, b);
                A.si(li, AL_FIXED, type != kDynamic);
                A.si(li, AL_FLOATING, pb < 0 && type == kDynamic);
                if (pb < 0) {
                    A.si(li, AL_PARENT, -1);
                } else {
                    A.si(li, AL_PARENT, A.ti(pb, AT_LINK));
                    int jk = A.ti(b, AT_PARENT_J);
                    int side_b = ldi(w, jw(L, jk, J_BODY_B)) == b;
                    A.s3(li, AL_ANCHOR_A, ld3(w, jw(L, jk, side_b ? J_LOCAL_ANCHOR_A : J_LOCAL_ANCHOR_B)));
                    A.sq(li, AL_ROT_A, ldq(w, jw(L, jk, side_b ? J_LOCAL_ROT_A : J_LOCAL_ROT_B)));
                    A.s3(li, AL_ANCHOR_B, ld3(w, jw(L, jk, side_b ? J_LOCAL_ANCHOR_B : J_LOCAL_ANCHOR_A)));
                    A.sq(li, AL_ROT_B, ldq(w, jw(L, jk, side_b ? J_LOCAL_ROT_B : J_LOCAL_ROT_A)));
                }
            }
        }
    }
    for (int s = 0; s < nb; s++) {
        if (A.ti(s, AT_SEEN) || ldi(w, bw(L, s, B_TYPE)) != kDynamic) continue;
        if (A.n_links >= A.max_b) return false;
        int li = A.n_links++;
        A.si(li, AL_BODY, s);
        A.si(li, AL_FIXED, 0);
        A.si(li, AL_FLOATING, 1);
        A.si(li, AL_PARENT, -1);
    }
    /* b3_art_link_from_body (:329-338) */
    for (int i = 0; i < A.n_links; i++) {
        int b = A.gi(i, AL_BODY);
        float im = ldf(w, bw(L, b, B_INV_MASS));
        V3 ii = ld3(w, bw(L, b, B_INV_INERTIA));
        A.sf(i, AL_MASS, im > 0.0f ? 1.0f / im : 0.0f);
        A.s3(i, AL_ILOCAL, v3(ii.x > 0.0f ? 1.0f / ii.x : 0.0f, ii.y > 0.0f ? 1.0f / ii.y : 0.0f,
            ii.z > 0.0f ? 1.0f / ii.z : 0.0f));
        A.s3(i, AL_LC, ld3(w, bw(L, b, B_LOCAL_CENTER)));
    }
    return A.n_links > 0;
}

/* The links' poses, inertias and joint axes at the bodies' current delta
 * poses (b3_art_refresh, :527-570, and b3_art_lived_pose, :492-497); the
 * delta poses are the step's, in the delta records. */
B3D_FN void art_refresh(const Lane& L, const ArtWs& A) {
    const uint32_t* w = L.w;
    for (int i = 0; i < A.n_links; i++) {
        int b = A.gi(i, AL_BODY);
        const uint32_t* d = delta_rec(L, b);
        Q rq = qnorm(qmul(rq4(d, BD_DQ), ldq(w, bw(L, b, B_ROTATION))));
        V3 com = add(ld3(w, bw(L, b, B_CENTER)), r3(d, BD_DP));
        A.sq(i, AL_ROT, rq);
        A.s3(i, AL_COM, com);
        A.s3(i, AL_POS, sub(com, rot(rq, A.g3(i, AL_LC))));
        if (A.gi(i, AL_FIXED)) {
            A.sm3(i, AL_IWW, m3zero());
            A.sf(i, AL_MASS, 0.0f);
        } else {
            A.sm3(i, AL_IWW, world_inv_i(rq, A.g3(i, AL_ILOCAL)));
        }
        A.s3(i, AL_SW, zero3());
        A.s3(i, AL_SV, zero3());
        A.s3(i, AL_R, zero3());
        int p = A.gi(i, AL_PARENT);
        if (p < 0) continue;
        V3 anchor = xf(A.g3(p, AL_POS), A.gq(p, AL_ROT), A.g3(i, AL_ANCHOR_A));
        V3 axis_local = rot(A.gq(i, AL_ROT_A), v3(0.0f, 0.0f, 1.0f));
        V3 u = norm(rot(A.gq(p, AL_ROT), axis_local));
        A.s3(i, AL_R, sub(com, A.g3(p, AL_COM)));
        A.s3(i, AL_SW, u);
        A.s3(i, AL_SV, cross(u, sub(com, anchor)));
    }
}

/* The link's spatial inertia: world inertia, then mass on the diagonal. */
B3D_FN M6 art_inertia(const ArtWs& A, int i) {
    M6 I = m6zero();
    I.ww = A.gm3(i, AL_IWW);
    float m = A.gf(i, AL_MASS);
    if (!A.gi(i, AL_FIXED)) {
        I.vv.cx = v3(m, 0.0f, 0.0f);
        I.vv.cy = v3(0.0f, m, 0.0f);
        I.vv.cz = v3(0.0f, 0.0f, m);
    }
    return I;
}

B3D_FN S6 art_wrench(V3 r, V3 n, float x, int torque) {                 /* :675-686 */
    S6 f;
    if (torque == 1) {
        f.w = scale(n, x);
        f.v = zero3();
    } else {
        f.v = scale(n, x);
        f.w = cross(r, f.v);
    }
    return f;
}

/* The pose-only half of b3_art_delassus_apply (:722-749): the refresh, the
 * links' own inertias (b3_art_seed_bias's linear form, :572-605) and, of the
 * backward sweep (:607-633), the articulated inertias, U = I^A S, 1/D, the
 * zero-bias term I^A c (c = 0) and each floating root's elimination.  None
 * of it depends on the impulses, and nothing a sweep does between two
 * operator calls changes the poses it is built from (only velocities), so a
 * pass runs it once and art_delassus reuses it for every call: the values
 * are the ones each call of the reference recomputes. */
B3D_FN void art_pose_pass(const Lane& L, const ArtWs& A) {
    art_refresh(L, A);
    for (int i = 0; i < A.n_links; i++) A.sI(i, AL_IA, art_inertia(A, i));
    for (int i = A.n_links - 1; i >= 0; i--) {
        int p = A.gi(i, AL_PARENT);
        if (p < 0) {
            if (!A.gi(i, AL_FIXED) && A.gi(i, AL_FLOATING)) isolve_record(A, i, A.gI(i, AL_IA));
            continue;
        }
        S6 S;
        S.w = A.g3(i, AL_SW);
        S.v = A.g3(i, AL_SV);
        M6 IA = A.gI(i, AL_IA);
        S6 U = imul(IA, S);
        A.s6(i, AL_U, U);
        float D = sdot(S, U);
        if (D < kArtDmin) D = kArtDmin;
        float Dinv = 1.0f / D;
        A.sf(i, AL_DINV, Dinv);
        A.s6(i, AL_IC, imul(IA, s6zero()));
        if (!A.gi(p, AL_FIXED))
            A.sI(p, AL_IA, iadd(A.gI(p, AL_IA), ishift(irank1(IA, U, Dinv), A.g3(i, AL_R))));
    }
}

/* y = J M^-1 J^T x for n rows: the impulse half of b3_art_delassus_apply
 * (:722-749) on the last art_pose_pass, with the zero link velocities and
 * joint rates it sets (the row wrenches, the bias-force half of the
 * backward sweep, the forward sweep :635-666); the accelerations stay in
 * the links' AL_A words. */
B3D_FN void art_delassus(const Lane& L, const ArtWs& A, const ArtRow* rows, const float* x, float* y, int n) {
    (void)L;
    for (int i = 0; i < A.n_links; i++) {
        S6 pa;
        pa.w = sub(zero3(), zero3());
        pa.v = pa.w;
        A.s6(i, AL_PA, pa);
    }
    for (int e = 0; e < n; e++) {
        const ArtRow& row = rows[e];
        if (row.link_a >= 0 && !A.gi(row.link_a, AL_FIXED)) {
            S6 f = art_wrench(row.ra, row.n, x[e], row.torque);
            S6 pa = A.g6(row.link_a, AL_PA);
            pa.w = sub(pa.w, f.w);
            pa.v = sub(pa.v, f.v);
            A.s6(row.link_a, AL_PA, pa);
        }
        if (row.link_b >= 0 && !A.gi(row.link_b, AL_FIXED)) {
            S6 f = art_wrench(row.rb, row.n, x[e], row.torque);
            S6 pa = A.g6(row.link_b, AL_PA);
            pa.w = add(pa.w, f.w);
            pa.v = add(pa.v, f.v);
            A.s6(row.link_b, AL_PA, pa);
        }
    }
    /* backward sweep, bias forces only (zero joint torques) */
    for (int i = A.n_links - 1; i >= 0; i--) {
        int p = A.gi(i, AL_PARENT);
        if (p < 0) continue;
        S6 S;
        S.w = A.g3(i, AL_SW);
        S.v = A.g3(i, AL_SV);
        S6 U = A.g6(i, AL_U);
        float Dinv = A.gf(i, AL_DINV);
        S6 pA = A.g6(i, AL_PA);
        float u = 0.0f - sdot(S, pA);
        S6 Ic = A.g6(i, AL_IC);
        pA.w = add(add(pA.w, Ic.w), scale(U.w, u * Dinv));
        pA.v = add(add(pA.v, Ic.v), scale(U.v, u * Dinv));
        if (!A.gi(p, AL_FIXED)) {
            V3 r = A.g3(i, AL_R);
            S6 pp = A.g6(p, AL_PA);
            pp.w = add(pp.w, add(pA.w, cross(r, pA.v)));
            pp.v = add(pp.v, pA.v);
            A.s6(p, AL_PA, pp);
        }
    }
    /* forward sweep */
    for (int i = 0; i < A.n_links; i++) {
        int p = A.gi(i, AL_PARENT);
        if (p < 0) {
            S6 a = s6zero();
            if (!A.gi(i, AL_FIXED) && A.gi(i, AL_FLOATING)) {
                S6 pA = A.g6(i, AL_PA), rhs;
                rhs.w = neg(pA.w);
                rhs.v = neg(pA.v);
                if (!isolve_replay(A, i, rhs, &a)) a = s6zero();
            }
            A.s6(i, AL_A, a);
            continue;
        }
        S6 ap = A.g6(p, AL_A), rhs;
        V3 r = A.g3(i, AL_R);
        rhs.w = ap.w;
        rhs.v = add(ap.v, cross(ap.w, r));
        rhs.w = add(rhs.w, zero3());
        rhs.v = add(rhs.v, zero3());
        S6 S;
        S.w = A.g3(i, AL_SW);
        S.v = A.g3(i, AL_SV);
        float u = 0.0f - sdot(S, A.g6(i, AL_PA));
        u -= sdot(S, imul(A.gI(i, AL_IA), rhs));
        float qdd = A.gf(i, AL_DINV) * u;
        S6 a;
        a.w = add(rhs.w, scale(S.w, qdd));
        a.v = add(rhs.v, scale(S.v, qdd));
        A.s6(i, AL_A, a);
    }
    /* row accelerations (b3_art_row_eval with accel, :688-720; the link
     * velocities are zero) */
    for (int e = 0; e < n; e++) {
        const ArtRow& row = rows[e];
        float yy = 0.0f;
        if (row.torque == 1) {
            if (row.link_a >= 0) yy += dot(A.g3(row.link_a, AL_A), row.n);
            if (row.link_b >= 0) yy -= dot(A.g3(row.link_b, AL_A), row.n);
        } else {
            V3 z = zero3();
            if (row.link_a >= 0) {
                S6 a = A.g6(row.link_a, AL_A);
                V3 ac = add(a.v, cross(a.w, row.ra));
                ac = add(ac, cross(z, cross(z, row.ra)));
                yy += dot(ac, row.n);
            }
            if (row.link_b >= 0) {
                S6 a = A.g6(row.link_b, AL_A);
                V3 ac = add(a.v, cross(a.w, row.rb));
                ac = add(ac, cross(z, cross(z, row.rb)));
                yy -= dot(ac, row.n);
            }
        }
        y[e] = yy;
    }
}

B3D_FN int art_link_of(const ArtWs& A, int body) {                      /* :751-758 */
    for (int i = 0; i < A.n_links; i++)
        if (A.gi(i, AL_BODY) == body) return i;
    return -1;
}
B3D_FN bool art_make_row(const ArtWs& A, int a, int b, V3 ra, V3 rb, V3 n, ArtRow* row) {   /* :769-779 */
    row->link_a = a >= 0 ? art_link_of(A, a) : -1;
    row->link_b = b >= 0 ? art_link_of(A, b) : -1;
    row->torque = 0;
    row->ra = ra;
    row->rb = rb;
    row->n = n;
    return row->link_a >= 0 || row->link_b >= 0;
}
B3D_FN float art_response(const Lane& L, const ArtWs& A, const ArtRow& row) {   /* :781-787 */
    float x = 1.0f, y = 0.0f;
    art_delassus(L, A, &row, &x, &y, 1);
    return y;
}
/* Impulse lambda along a row: the velocity change of every link
 * (b3_art_apply_impulse and b3_art_add_delta_vel, :789-808). */
B3D_FN void art_apply(const Lane& L, const ArtWs& A, const ArtRow& row, float lambda) {
    float x = -lambda, y = 0.0f;
    art_delassus(L, A, &row, &x, &y, 1);
    for (int i = 0; i < A.n_links; i++) {
        if (A.gi(i, AL_FIXED)) continue;
        int b = A.gi(i, AL_BODY);
        S6 a = A.g6(i, AL_A);
        set_vlin(L, b, add(vlin(L, b), a.v));
        set_vang(L, b, add(vang(L, b), a.w));
    }
}

/* ---- the contact rows in the world (the reference's layout) ---- */

struct WContact {
    int a, b, pc;
    V3 n;
};
B3D_FN WContact wc_load(const Lane& L, int c) {
    WContact k;
    k.a = ldi(L.w, cw(L, c, C_BODY_A));
    k.b = ldi(L.w, cw(L, c, C_BODY_B));
    k.pc = clampi(ldi(L.w, cw(L, c, C_POINT_COUNT)), 0, kMaxManifold);
    k.n = ld3(L.w, cw(L, c, C_NORMAL));
    return k;
}

/* b3_art_solve_rolling_fields (:810-867) */
B3D_FN void art_rolling(const Lane& L, const ArtWs& A, int ba, int bb, V3 t1, V3 t2, float rolling, float total_n,
        V3* impulse) {
    float max_r = rolling * total_n;
    if (!(max_r > 0.0f)) return;
    ArtRow rows[2];
    if (!art_make_row(A, ba, bb, zero3(), zero3(), t1, &rows[0])) return;
    rows[0].torque = 1;
    art_make_row(A, ba, bb, zero3(), zero3(), t2, &rows[1]);
    rows[1].torque = 1;
    float e0[2] = {1.0f, 0.0f}, e1[2] = {0.0f, 1.0f}, col0[2], col1[2];
    art_delassus(L, A, rows, e0, col0, 2);
    art_delassus(L, A, rows, e1, col1, 2);
    M2 K;
    K.cx.x = col0[0];
    K.cx.y = col0[1];
    K.cy.x = col1[0];
    K.cy.y = col1[1];
    M2 Minv = inv2(K);
    V3 dw = sub(vang(L, bb), vang(L, ba));
    V2 vt;
    vt.x = dot(dw, t1);
    vt.y = dot(dw, t2);
    V2 tm = mv2(Minv, vt);
    V3 old = *impulse;
    V2 oi, ni, df;
    oi.x = dot(old, t1);
    oi.y = dot(old, t2);
    ni.x = oi.x - tm.x;
    ni.y = oi.y - tm.y;
    float fl2 = ni.x * ni.x + ni.y * ni.y;
    if (fl2 > max_r * max_r && fl2 > 0.0f) {
        float sc = rsqrt_scale(max_r, fl2);
        ni.x *= sc;
        ni.y *= sc;
    }
    df.x = ni.x - oi.x;
    df.y = ni.y - oi.y;
    *impulse = add(scale(t1, ni.x), scale(t2, ni.y));
    if (df.x != 0.0f) art_apply(L, A, rows[0], df.x);
    if (df.y != 0.0f) art_apply(L, A, rows[1], df.y);
}

/* b3_art_solve_friction (:1034-1121) on world contact c. */
B3D_FN void art_friction(const Lane& L, const ArtWs& A, int c, const WContact& k) {
    uint32_t* w = L.w;
    float total_n = 0.0f, twist_lim = 0.0f;
    for (int p = 0; p < k.pc; p++) {
        float ni = ldf(w, pw(L, c, p, P_NORMAL_IMPULSE));
        total_n += ni;
        twist_lim += ldf(w, pw(L, c, p, P_LEVER)) * ni;
    }
    float friction = ldf(w, cw(L, c, C_FRICTION));
    float max_t = friction * twist_lim;
    if (max_t > 0.0f) {
        ArtRow tw;
        if (art_make_row(A, k.a, k.b, zero3(), zero3(), k.n, &tw)) {
            tw.torque = 1;
            float ww = art_response(L, A, tw);
            float twist_mass = ww > 0.0f ? 1.0f / ww : 0.0f;
            stf(w, cw(L, c, C_TWIST_MASS), twist_mass);
            float twist_s = dot(k.n, sub(vang(L, k.b), vang(L, k.a)));
            float dtw = -twist_mass * twist_s;
            float old_t = ldf(w, cw(L, c, C_TWIST_IMPULSE));
            float nt = old_t + dtw;
            if (nt > max_t) nt = max_t;
            else if (nt < -max_t) nt = -max_t;
            dtw = nt - old_t;
            stf(w, cw(L, c, C_TWIST_IMPULSE), nt);
            if (dtw != 0.0f) art_apply(L, A, tw, dtw);
        }
    }
    float max_f = friction * total_n;
    V3 t1 = ld3(w, cw(L, c, C_TANGENT1)), t2 = ld3(w, cw(L, c, C_TANGENT2));
    if (max_f > 0.0f) {
        V3 ca = ld3(w, cw(L, c, C_CENTER_A)), cb = ld3(w, cw(L, c, C_CENTER_B));
        ArtRow rows[2];
        if (art_make_row(A, k.a, k.b, ca, cb, t1, &rows[0])) {
            art_make_row(A, k.a, k.b, ca, cb, t2, &rows[1]);
            float e0[2] = {1.0f, 0.0f}, e1[2] = {0.0f, 1.0f}, col0[2], col1[2];
            art_delassus(L, A, rows, e0, col0, 2);
            art_delassus(L, A, rows, e1, col1, 2);
            M2 K;
            K.cx.x = col0[0];
            K.cx.y = col0[1];
            K.cy.x = col1[0];
            K.cy.y = col1[1];
            M2 Minv = inv2(K);
            stf(w, cw(L, c, C_TANGENT_MASS), Minv.cx.x);
            stf(w, cw(L, c, C_TANGENT_MASS + 1), Minv.cx.y);
            stf(w, cw(L, c, C_TANGENT_MASS + 2), Minv.cy.x);
            stf(w, cw(L, c, C_TANGENT_MASS + 3), Minv.cy.y);
            V3 vra = add(vlin(L, k.a), cross(vang(L, k.a), ca));
            V3 vrb = add(vlin(L, k.b), cross(vang(L, k.b), cb));
            V3 vr = sub(vrb, vra);
            V2 vt, ni, df, fi;
            vt.x = dot(vr, t1);
            vt.y = dot(vr, t2);
            V2 tm = mv2(Minv, vt);
            fi.x = ldf(w, cw(L, c, C_FRICTION_IMPULSE));
            fi.y = ldf(w, cw(L, c, C_FRICTION_IMPULSE + 1));
            ni.x = fi.x - tm.x;
            ni.y = fi.y - tm.y;
            float fl2 = ni.x * ni.x + ni.y * ni.y;
            if (fl2 > max_f * max_f && fl2 > 0.0f) {
                float sc = rsqrt_scale(max_f, fl2);
                ni.x *= sc;
                ni.y *= sc;
            }
            df.x = ni.x - fi.x;
            df.y = ni.y - fi.y;
            stf(w, cw(L, c, C_FRICTION_IMPULSE), ni.x);
            stf(w, cw(L, c, C_FRICTION_IMPULSE + 1), ni.y);
            if (df.x != 0.0f) art_apply(L, A, rows[0], df.x);
            if (df.y != 0.0f) art_apply(L, A, rows[1], df.y);
        }
    }
    V3 roll = ld3(w, cw(L, c, C_ROLLING_IMPULSE));
    art_rolling(L, A, k.a, k.b, t1, t2, ldf(w, cw(L, c, C_ROLLING)), total_n, &roll);
    st3(w, cw(L, c, C_ROLLING_IMPULSE), roll);
}

/* b3_art_solve_contacts (b3_art.cuh:1220-1279): one iteration from the
 * contact sweeps (08_contacts.inl:425-432), kArtContactIters from the
 * reduced integrator; the normal masses are computed on the first. */
B3D_FN void art_solve_contacts(const Lane& L, const ArtWs& A, float inv_h, float contact_speed, int use_bias,
        int iters = 1) {
    uint32_t* w = L.w;
    int cc = ldi(w, H_CONTACT_COUNT);
    if (cc > 0) art_pose_pass(L, A);
    for (int it = 0; it < iters; it++)
    for (int c = 0; c < cc; c++) {
        WContact k = wc_load(L, c);
        const uint32_t* da = delta_rec(L, k.a);
        const uint32_t* db = delta_rec(L, k.b);
        V3 dp = sub(r3(db, BD_DP), r3(da, BD_DP));
        Q dqa = rq4(da, BD_DQ), dqb = rq4(db, BD_DQ);
        Soft soft = ldsoft(w, cw(L, c, C_SOFTNESS));
        for (int p = 0; p < k.pc; p++) {
            V3 ra = ld3(w, pw(L, c, p, P_R_A)), rb = ld3(w, pw(L, c, p, P_R_B));
            ArtRow row;
            if (!art_make_row(A, k.a, k.b, ra, rb, k.n, &row)) continue;
            float nmass;
            if (it == 0) {
                float ww = art_response(L, A, row);
                nmass = ww > 0.0f ? 1.0f / ww : 0.0f;
                stf(w, pw(L, c, p, P_NORMAL_MASS), nmass);
            } else {
                nmass = ldf(w, pw(L, c, p, P_NORMAL_MASS));
            }
            V3 ds = add(dp, sub(rot(dqb, rb), rot(dqa, ra)));
            float sep = dot(ds, k.n) + ldf(w, pw(L, c, p, P_BASE_SEP));
            float vbias = 0.0f, mscale = 1.0f, iscale = 0.0f;
            if (sep > 0.0f) {
                vbias = sep * inv_h;
            } else if (use_bias) {
                vbias = maxf(soft.mass_scale * soft.bias_rate * sep, -contact_speed);
                mscale = soft.mass_scale;
                iscale = soft.impulse_scale;
            }
            V3 vra = add(vlin(L, k.a), cross(vang(L, k.a), ra));
            V3 vrb = add(vlin(L, k.b), cross(vang(L, k.b), rb));
            float vn = dot(sub(vrb, vra), k.n);
            float old = ldf(w, pw(L, c, p, P_NORMAL_IMPULSE));
            float dimp = -nmass * (mscale * vn + vbias) - iscale * old;
            float nimp = maxf(old + dimp, 0.0f);
            dimp = nimp - old;
            stf(w, pw(L, c, p, P_NORMAL_IMPULSE), nimp);
            stf(w, pw(L, c, p, P_TOTAL_NORMAL), ldf(w, pw(L, c, p, P_TOTAL_NORMAL)) + dimp);
            if (dimp != 0.0f) art_apply(L, A, row, dimp);
        }
        if (!use_bias) art_friction(L, A, c, k);
    }
}

/* b3_warm_start's articulated branch (08_contacts.inl:195-226). */
B3D_FN void art_warm_start(const Lane& L, const ArtWs& A) {
    uint32_t* w = L.w;
    int cc = ldi(w, H_CONTACT_COUNT);
    if (cc > 0) art_pose_pass(L, A);
    for (int c = 0; c < cc; c++) {
        WContact k = wc_load(L, c);
        ArtRow row;
        for (int p = 0; p < k.pc; p++) {
            if (art_make_row(A, k.a, k.b, ld3(w, pw(L, c, p, P_R_A)), ld3(w, pw(L, c, p, P_R_B)), k.n, &row))
                art_apply(L, A, row, ldf(w, pw(L, c, p, P_NORMAL_IMPULSE)));
        }
        V3 t[2] = {ld3(w, cw(L, c, C_TANGENT1)), ld3(w, cw(L, c, C_TANGENT2))};
        float f[2] = {ldf(w, cw(L, c, C_FRICTION_IMPULSE)), ldf(w, cw(L, c, C_FRICTION_IMPULSE + 1))};
        V3 ca = ld3(w, cw(L, c, C_CENTER_A)), cb = ld3(w, cw(L, c, C_CENTER_B));
        V3 roll = ld3(w, cw(L, c, C_ROLLING_IMPULSE));
        for (int q = 0; q < 2; q++) {
            if (art_make_row(A, k.a, k.b, ca, cb, t[q], &row)) art_apply(L, A, row, f[q]);
            row.torque = 1;
            art_apply(L, A, row, dot(roll, t[q]));
        }
        if (art_make_row(A, k.a, k.b, zero3(), zero3(), k.n, &row)) {
            row.torque = 1;
            art_apply(L, A, row, ldf(w, cw(L, c, C_TWIST_IMPULSE)));
        }
    }
}

/* ---- the ordinary contact path on the world rows (independent bodies) ---- */

/* b3_prepare_one_contact (08_contacts.inl:234-291) for every contact. */
B3D_FN void wrow_prepare(const Lane& L, Soft cs, Soft ss) {
    uint32_t* w = L.w;
    int cc = ldi(w, H_CONTACT_COUNT);
    const float inv_tau = 1.0f / kSpeculative;
    for (int c = 0; c < cc; c++) {
        WContact k = wc_load(L, c);
        bool dyn_a = ldi(w, bw(L, k.a, B_TYPE)) == kDynamic, dyn_b = ldi(w, bw(L, k.b, B_TYPE)) == kDynamic;
        float ma = dyn_a ? ldf(w, bw(L, k.a, B_INV_MASS)) : 0.0f;
        float mb = dyn_b ? ldf(w, bw(L, k.b, B_INV_MASS)) : 0.0f;
        M3 ia = dyn_a ? ldm3(w, bw(L, k.a, B_INV_I_WORLD)) : m3zero();
        M3 ib = dyn_b ? ldm3(w, bw(L, k.b, B_INV_I_WORLD)) : m3zero();
        stf(w, cw(L, c, C_INV_MASS_A), ma);
        stf(w, cw(L, c, C_INV_MASS_B), mb);
        stm3(w, cw(L, c, C_INV_I_A), ia);
        stm3(w, cw(L, c, C_INV_I_B), ib);
        stm3(w, cw(L, c, C_ROLLING_MASS), inv3(madd3(ia, ib)));
        stsoft(w, cw(L, c, C_SOFTNESS), ldi(w, cw(L, c, C_STATIC)) ? ss : cs);
        V3 n = k.n;
        V3 center_a = zero3(), center_b = zero3();
        float wsum = 0.0f;
        V3 va = vlin(L, k.a), wa = vang(L, k.a), vb = vlin(L, k.b), wb = vang(L, k.b);
        for (int p = 0; p < k.pc; p++) {
            V3 ra = ld3(w, pw(L, c, p, P_R_A)), rb = ld3(w, pw(L, c, p, P_R_B));
            V3 rn_a = cross(ra, n), rn_b = cross(rb, n);
            float kn = ma + mb + dot(rn_a, mv(ia, rn_a)) + dot(rn_b, mv(ib, rn_b));
            stf(w, pw(L, c, p, P_NORMAL_MASS), kn > 0.0f ? 1.0f / kn : 0.0f);
            V3 vra = add(va, cross(wa, ra)), vrb = add(vb, cross(wb, rb));
            stf(w, pw(L, c, p, P_REL_VEL), dot(n, sub(vrb, vra)));
            stf(w, pw(L, c, p, P_TOTAL_NORMAL), 0.0f);
            float sep = ldf(w, pw(L, c, p, P_BASE_SEP)) + dot(sub(rb, ra), n);
            float weight = clampf(2.0f - sep * inv_tau, kMinFrictionW, 1.0f);
            center_a = madd(center_a, weight, ra);
            center_b = madd(center_b, weight, rb);
            wsum += weight;
        }
        float invw = wsum > 0.0f ? 1.0f / wsum : 0.0f;
        center_a = scale(center_a, invw);
        center_b = scale(center_b, invw);
        st3(w, cw(L, c, C_CENTER_A), center_a);
        st3(w, cw(L, c, C_CENTER_B), center_b);
        for (int p = 0; p < k.pc; p++)
            stf(w, pw(L, c, p, P_LEVER), len(sub(ld3(w, pw(L, c, p, P_R_A)), center_a)));
        V3 t1 = ld3(w, cw(L, c, C_TANGENT1)), t2 = ld3(w, cw(L, c, C_TANGENT2));
        V3 rt_a1 = cross(center_a, t1), rt_a2 = cross(center_a, t2);
        V3 rt_b1 = cross(center_b, t1), rt_b2 = cross(center_b, t2);
        M2 k2;
        k2.cx.x = ma + mb + dot(rt_a1, mv(ia, rt_a1)) + dot(rt_b1, mv(ib, rt_b1));
        k2.cy.y = ma + mb + dot(rt_a2, mv(ia, rt_a2)) + dot(rt_b2, mv(ib, rt_b2));
        k2.cx.y = dot(rt_a1, mv(ia, rt_a2)) + dot(rt_b1, mv(ib, rt_b2));
        k2.cy.x = k2.cx.y;
        M2 tm = inv2(k2);
        stf(w, cw(L, c, C_TANGENT_MASS), tm.cx.x);
        stf(w, cw(L, c, C_TANGENT_MASS + 1), tm.cx.y);
        stf(w, cw(L, c, C_TANGENT_MASS + 2), tm.cy.x);
        stf(w, cw(L, c, C_TANGENT_MASS + 3), tm.cy.y);
        float kt = dot(n, mv(madd3(ia, ib), n));
        stf(w, cw(L, c, C_TWIST_MASS), kt > 0.0f ? 1.0f / kt : 0.0f);
    }
}

struct WMass { float ma, mb; M3 ia, ib; };
B3D_FN WMass wc_masses(const Lane& L, int c) {
    WMass m;
    m.ma = ldf(L.w, cw(L, c, C_INV_MASS_A));
    m.mb = ldf(L.w, cw(L, c, C_INV_MASS_B));
    m.ia = ldm3(L.w, cw(L, c, C_INV_I_A));
    m.ib = ldm3(L.w, cw(L, c, C_INV_I_B));
    return m;
}

/* b3_warm_one_contact (08_contacts.inl:293-313) for every contact. */
B3D_FN void wrow_warm(const Lane& L) {
    uint32_t* w = L.w;
    int cc = ldi(w, H_CONTACT_COUNT);
    for (int c = 0; c < cc; c++) {
        WContact k = wc_load(L, c);
        WMass m = wc_masses(L, c);
        for (int p = 0; p < k.pc; p++) {
            V3 P = scale(k.n, ldf(w, pw(L, c, p, P_NORMAL_IMPULSE)));
            apply_impulse(L, k.a, m.ma, m.ia, ld3(w, pw(L, c, p, P_R_A)), P, -1.0f);
            apply_impulse(L, k.b, m.mb, m.ib, ld3(w, pw(L, c, p, P_R_B)), P, 1.0f);
        }
        V3 f = add(scale(ld3(w, cw(L, c, C_TANGENT1)), ldf(w, cw(L, c, C_FRICTION_IMPULSE))),
            scale(ld3(w, cw(L, c, C_TANGENT2)), ldf(w, cw(L, c, C_FRICTION_IMPULSE + 1))));
        apply_impulse(L, k.a, m.ma, m.ia, ld3(w, cw(L, c, C_CENTER_A)), f, -1.0f);
        apply_impulse(L, k.b, m.mb, m.ib, ld3(w, cw(L, c, C_CENTER_B)), f, 1.0f);
        V3 tr = add(scale(k.n, ldf(w, cw(L, c, C_TWIST_IMPULSE))), ld3(w, cw(L, c, C_ROLLING_IMPULSE)));
        if (is_dyn_flag(L, k.a)) set_vang(L, k.a, sub(vang(L, k.a), mv(m.ia, tr)));
        if (is_dyn_flag(L, k.b)) set_vang(L, k.b, add(vang(L, k.b), mv(m.ib, tr)));
    }
}

/* b3_solve_one_contact (08_contacts.inl:315-413) over every contact. */
B3D_FN void wrow_solve(const Lane& L, float inv_h, float contact_speed, int use_bias) {
    uint32_t* w = L.w;
    int cc = ldi(w, H_CONTACT_COUNT);
    for (int c = 0; c < cc; c++) {
        WContact k = wc_load(L, c);
        WMass m = wc_masses(L, c);
        Soft soft = ldsoft(w, cw(L, c, C_SOFTNESS));
        V3 va = vlin(L, k.a), wa = vang(L, k.a), vb = vlin(L, k.b), wb = vang(L, k.b);
        const uint32_t* da = delta_rec(L, k.a);
        const uint32_t* db = delta_rec(L, k.b);
        V3 dp = sub(r3(db, BD_DP), r3(da, BD_DP));
        Q dqa = rq4(da, BD_DQ), dqb = rq4(db, BD_DQ);
        float total_n = 0.0f, twist_lim = 0.0f;
        for (int p = 0; p < k.pc; p++) {
            V3 ra = ld3(w, pw(L, c, p, P_R_A)), rb = ld3(w, pw(L, c, p, P_R_B));
            V3 ds = add(dp, sub(rot(dqb, rb), rot(dqa, ra)));
            float sep = dot(ds, k.n) + ldf(w, pw(L, c, p, P_BASE_SEP));
            float vbias = 0.0f, mscale = 1.0f, iscale = 0.0f;
            if (sep > 0.0f) {
                vbias = sep * inv_h;
            } else if (use_bias) {
                vbias = maxf(soft.mass_scale * soft.bias_rate * sep, -contact_speed);
                mscale = soft.mass_scale;
                iscale = soft.impulse_scale;
            }
            V3 vra = add(va, cross(wa, ra)), vrb = add(vb, cross(wb, rb));
            float vn = dot(sub(vrb, vra), k.n);
            float old = ldf(w, pw(L, c, p, P_NORMAL_IMPULSE));
            float dimp = -ldf(w, pw(L, c, p, P_NORMAL_MASS)) * (mscale * vn + vbias) - iscale * old;
            float nimp = maxf(old + dimp, 0.0f);
            dimp = nimp - old;
            stf(w, pw(L, c, p, P_NORMAL_IMPULSE), nimp);
            stf(w, pw(L, c, p, P_TOTAL_NORMAL), ldf(w, pw(L, c, p, P_TOTAL_NORMAL)) + nimp);
            total_n += nimp;
            twist_lim += ldf(w, pw(L, c, p, P_LEVER)) * nimp;
            V3 P = scale(k.n, dimp);
            va = msub(va, m.ma, P);
            wa = sub(wa, mv(m.ia, cross(ra, P)));
            vb = madd(vb, m.mb, P);
            wb = add(wb, mv(m.ib, cross(rb, P)));
        }
        if (!use_bias) {
            float friction = ldf(w, cw(L, c, C_FRICTION));
            float twist_s = dot(k.n, sub(wb, wa));
            float max_t = friction * twist_lim;
            float dtw = -ldf(w, cw(L, c, C_TWIST_MASS)) * twist_s;
            float old_t = ldf(w, cw(L, c, C_TWIST_IMPULSE));
            float nt = clampf(old_t + dtw, -max_t, max_t);
            stf(w, cw(L, c, C_TWIST_IMPULSE), nt);
            dtw = nt - old_t;
            wa = sub(wa, mv(m.ia, scale(k.n, dtw)));
            wb = add(wb, mv(m.ib, scale(k.n, dtw)));
            V3 t1 = ld3(w, cw(L, c, C_TANGENT1)), t2 = ld3(w, cw(L, c, C_TANGENT2));
            V3 ca = ld3(w, cw(L, c, C_CENTER_A)), cb = ld3(w, cw(L, c, C_CENTER_B));
            V3 vr = sub(add(vb, cross(wb, cb)), add(va, cross(wa, ca)));
            V2 vt;
            vt.x = dot(vr, t1);
            vt.y = dot(vr, t2);
            M2 tmass;
            tmass.cx.x = ldf(w, cw(L, c, C_TANGENT_MASS));
            tmass.cx.y = ldf(w, cw(L, c, C_TANGENT_MASS + 1));
            tmass.cy.x = ldf(w, cw(L, c, C_TANGENT_MASS + 2));
            tmass.cy.y = ldf(w, cw(L, c, C_TANGENT_MASS + 3));
            V2 tm = mv2(tmass, vt);
            V2 fi, ni;
            fi.x = ldf(w, cw(L, c, C_FRICTION_IMPULSE));
            fi.y = ldf(w, cw(L, c, C_FRICTION_IMPULSE + 1));
            ni.x = fi.x - tm.x;
            ni.y = fi.y - tm.y;
            float max_f = friction * total_n;
            float fl2 = ni.x * ni.x + ni.y * ni.y;
            if (fl2 > max_f * max_f && fl2 > 0.0f) {
                float sc = rsqrt_scale(max_f, fl2);
                ni.x *= sc;
                ni.y *= sc;
            }
            V2 df;
            df.x = ni.x - fi.x;
            df.y = ni.y - fi.y;
            stf(w, cw(L, c, C_FRICTION_IMPULSE), ni.x);
            stf(w, cw(L, c, C_FRICTION_IMPULSE + 1), ni.y);
            V3 P = add(scale(t1, df.x), scale(t2, df.y));
            va = msub(va, m.ma, P);
            wa = sub(wa, mv(m.ia, cross(ca, P)));
            vb = madd(vb, m.mb, P);
            wb = add(wb, mv(m.ib, cross(cb, P)));
            V3 roll = ld3(w, cw(L, c, C_ROLLING_IMPULSE));
            solve_rolling(t1, t2, ldf(w, cw(L, c, C_ROLLING)), total_n, m.ia, m.ib, &roll, &wa, &wb);
            st3(w, cw(L, c, C_ROLLING_IMPULSE), roll);
        }
        if (is_dyn_flag(L, k.a)) {
            set_vlin(L, k.a, va);
            set_vang(L, k.a, wa);
        }
        if (is_dyn_flag(L, k.b)) {
            set_vlin(L, k.b, vb);
            set_vang(L, k.b, wb);
        }
    }
}

/* b3_apply_restitution (08_contacts.inl:439-480) on the world rows. */
B3D_FN void wrow_restitution(const Lane& L, float threshold) {
    uint32_t* w = L.w;
    int cc = ldi(w, H_CONTACT_COUNT);
    for (int c = 0; c < cc; c++) {
        float e = ldf(w, cw(L, c, C_RESTITUTION));
        if (e == 0.0f) continue;
        WContact k = wc_load(L, c);
        WMass m = wc_masses(L, c);
        V3 va = vlin(L, k.a), wa = vang(L, k.a), vb = vlin(L, k.b), wb = vang(L, k.b);
        for (int p = 0; p < k.pc; p++) {
            float rv = ldf(w, pw(L, c, p, P_REL_VEL));
            if (rv > -threshold || ldf(w, pw(L, c, p, P_TOTAL_NORMAL)) == 0.0f) continue;
            V3 ra = ld3(w, pw(L, c, p, P_R_A)), rb = ld3(w, pw(L, c, p, P_R_B));
            V3 vra = add(va, cross(wa, ra)), vrb = add(vb, cross(wb, rb));
            float vn = dot(sub(vrb, vra), k.n);
            float old = ldf(w, pw(L, c, p, P_NORMAL_IMPULSE));
            float imp = -ldf(w, pw(L, c, p, P_NORMAL_MASS)) * (vn + e * rv);
            float nimp = maxf(old + imp, 0.0f);
            imp = nimp - old;
            stf(w, pw(L, c, p, P_NORMAL_IMPULSE), nimp);
            V3 P = scale(k.n, imp);
            va = msub(va, m.ma, P);
            wa = sub(wa, mv(m.ia, cross(ra, P)));
            vb = madd(vb, m.mb, P);
            wb = add(wb, mv(m.ib, cross(rb, P)));
        }
        if (is_dyn_flag(L, k.a)) {
            set_vlin(L, k.a, va);
            set_vang(L, k.a, wa);
        }
        if (is_dyn_flag(L, k.b)) {
            set_vlin(L, k.b, vb);
            set_vang(L, k.b, wb);
        }
    }
}

/* The step's constants (b3_soft_step_params). */
struct ArtParams {
    int subs;
    float h, inv_h, inv_dt, contact_speed, rest_threshold;
    Soft cs, ss;
};
B3D_FN ArtParams art_params(const Lane& L, float dt, int substeps) {
    ArtParams P;
    P.subs = substeps < 1 ? 1 : substeps;
    P.h = dt / (float)P.subs;
    P.inv_dt = 1.0f / dt;
    P.inv_h = (float)P.subs * P.inv_dt;
    float hertz = minf(ldf(L.w, H_CONTACT_HERTZ), 0.25f * P.inv_h);
    float damping = ldf(L.w, H_CONTACT_DAMPING);
    P.cs = make_soft(hertz, damping, P.h);
    P.ss = make_soft(2.0f * hertz, 0.5f * damping, P.h);
    P.contact_speed = ldf(L.w, H_CONTACT_SPEED);
    P.rest_threshold = ldf(L.w, H_RESTITUTION_THRESHOLD);
    return P;
}

/* The opening both integrators share: contacts found and prepared in the
 * world rows, velocities staged, per-step body records. */
B3D_FN void art_open(const Lane& L, const ArtParams& P) {
    find_contacts(L);
    body_prepass(L, P.h);   /* with the velocity rows */
    wrow_prepare(L, P.cs, P.ss);
}

/* The rest of b3_step with articulated contacts (09_step.inl:148-264 with
 * 08_contacts.inl:194-232, 422-437).  Joints, integration and finalize are
 * the ordinary step's.  `built` is 1 when the caller has already built the
 * lane's tree, 0 when it has not tried. */
B3D_FN void art_indep_rest(const Lane& L, ArtWs& A, const ArtParams& P, int built) {
    prepare_joints(L, P.h);
    bool art = ldi(L.w, H_JOINT_COUNT) > 0 && ldi(L.w, H_CONTACT_COUNT) > 0 && (built || art_build(L, A));
    if (art) art_warm_start(L, A);
    else wrow_warm(L);
    warm_start_joints(L);
    joint_geometry(L);
    for (int s = 0; s < P.subs; s++) {
        integrate_velocities(L);
        if (art) art_solve_contacts(L, A, P.inv_h, P.contact_speed, 1);
        else wrow_solve(L, P.inv_h, P.contact_speed, 1);
        solve_joints(L, P.h, P.inv_h, 1);
        integrate_positions(L, P.h, P.inv_dt);
        delta_geometry(L);
        if (art) art_solve_contacts(L, A, P.inv_h, P.contact_speed, 0);
        else wrow_solve(L, P.inv_h, P.contact_speed, 0);
        solve_joints(L, P.h, P.inv_h, 0);
        wrow_restitution(L, P.rest_threshold);
    }
    finalize(L);
    vel_store(L);
}

B3D_FN ArtWs art_ws_of(const Lane& L, float* ws) {
    ArtWs A;
    A.p = ws;
    A.max_b = L.g.max_b;
    A.n_links = 0;
    return A;
}

/* One world's b3_step built with articulated contacts.  `ws` is the lane's
 * workspace. */
B3D_FN void step_world_art(const Lane& L0, float* ws, float dt, int substeps) {
    if (!(dt > 0.0f)) return;
    Lane L = L0;
    L.sslot = wave_slot(L);
    ArtParams P = art_params(L, dt, substeps);
    art_open(L, P);
    ArtWs A = art_ws_of(L, ws);
    art_indep_rest(L, A, P, 0);
}

/* ---- the reduced-coordinate integrator (b3_art_step) ---- */

/* 03_math.inl:321-326, with the host C library's sinf and cosf bits
 * (or_sinf, or_cosf in b3d_math.h). */
B3D_FN Q qaxis_angle(V3 axis, float radians) {
    axis = norm(axis);
    float h = 0.5f * radians;
    float s = or_sinf(h);
    return q4(s * axis.x, s * axis.y, s * axis.z, or_cosf(h));
}

/* art_refresh with each joint's rate about its axis and its angle, the
 * twist of the child frame relative to the parent frame (b3_art.cuh:
 * 499-507, 563-568). */
B3D_FN void art_refresh_q(const Lane& L, const ArtWs& A) {
    art_refresh(L, A);
    for (int i = 0; i < A.n_links; i++) {
        int p = A.gi(i, AL_PARENT);
        float q = 0.0f, qd = 0.0f;
        if (p >= 0) {
            V3 wrel = sub(vang(L, A.gi(i, AL_BODY)), vang(L, A.gi(p, AL_BODY)));
            qd = dot(wrel, A.g3(i, AL_SW));
            Q qa = qmul(A.gq(p, AL_ROT), A.gq(i, AL_ROT_A));
            Q qb = qmul(A.gq(i, AL_ROT), A.gq(i, AL_ROT_B));
            if (qdot(qa, qb) < 0.0f) qb = qneg(qb);
            q = twist(qinv_mul(qa, qb));
        }
        A.sf(i, AL_Q, q);
        A.sf(i, AL_QD, qd);
    }
}

/* Link accelerations under gravity, applied loads and velocity products
 * with zero joint torques (b3_art_aba, :668-673: the refresh, the full
 * b3_art_seed_bias, :572-605, and both sweeps, :607-666). */
B3D_FN void art_aba(const Lane& L, const ArtWs& A) {
    art_refresh_q(L, A);
    V3 g = ld3(L.w, H_GRAVITY);
    for (int i = 0; i < A.n_links; i++) {
        M6 I = art_inertia(A, i);
        A.sI(i, AL_IA, I);
        S6 pa = s6zero(), c = s6zero();
        if (!A.gi(i, AL_FIXED)) {
            int b = A.gi(i, AL_BODY);
            S6 v;
            v.w = vang(L, b);
            v.v = vlin(L, b);
            S6 ext;
            ext.v = add(ld3(L.w, bw(L, b, B_FORCE)),
                scale(g, A.gf(i, AL_MASS) * ldf(L.w, bw(L, b, B_GRAVITY_SCALE))));
            ext.w = ld3(L.w, bw(L, b, B_TORQUE));
            S6 Iw = imul(I, v);
            pa.w = sub(cross(v.w, Iw.w), ext.w);
            pa.v = sub(cross(v.w, Iw.v), ext.v);
            int p = A.gi(i, AL_PARENT);
            if (p >= 0) {
                float qd = A.gf(i, AL_QD);
                V3 wp = vang(L, A.gi(p, AL_BODY));
                c.w = cross(v.w, scale(A.g3(i, AL_SW), qd));
                c.v = add(cross(v.w, scale(A.g3(i, AL_SV), qd)), cross(wp, cross(wp, A.g3(i, AL_R))));
            }
        }
        A.s6(i, AL_PA, pa);
        A.s6(i, AL_C, c);
    }
    for (int i = A.n_links - 1; i >= 0; i--) {
        int p = A.gi(i, AL_PARENT);
        if (p < 0) continue;
        S6 S;
        S.w = A.g3(i, AL_SW);
        S.v = A.g3(i, AL_SV);
        M6 IA = A.gI(i, AL_IA);
        S6 U = imul(IA, S);
        A.s6(i, AL_U, U);
        float D = sdot(S, U);
        if (D < kArtDmin) D = kArtDmin;
        float Dinv = 1.0f / D;
        A.sf(i, AL_DINV, Dinv);
        S6 pA = A.g6(i, AL_PA);
        float u = 0.0f - sdot(S, pA);
        M6 IAp = irank1(IA, U, Dinv);
        S6 Ic = imul(IA, A.g6(i, AL_C));
        pA.w = add(add(pA.w, Ic.w), scale(U.w, u * Dinv));
        pA.v = add(add(pA.v, Ic.v), scale(U.v, u * Dinv));
        if (!A.gi(p, AL_FIXED)) {
            V3 r = A.g3(i, AL_R);
            A.sI(p, AL_IA, iadd(A.gI(p, AL_IA), ishift(IAp, r)));
            S6 pp = A.g6(p, AL_PA);
            pp.w = add(pp.w, add(pA.w, cross(r, pA.v)));
            pp.v = add(pp.v, pA.v);
            A.s6(p, AL_PA, pp);
        }
    }
    for (int i = 0; i < A.n_links; i++) {
        int p = A.gi(i, AL_PARENT);
        if (p < 0) {
            S6 a = s6zero();
            if (!A.gi(i, AL_FIXED) && A.gi(i, AL_FLOATING)) {
                S6 pA = A.g6(i, AL_PA), rhs;
                rhs.w = neg(pA.w);
                rhs.v = neg(pA.v);
                if (!isolve(A.gI(i, AL_IA), rhs, &a)) a = s6zero();
            }
            A.s6(i, AL_A, a);
            continue;
        }
        S6 ap = A.g6(p, AL_A), rhs, c = A.g6(i, AL_C);
        V3 r = A.g3(i, AL_R);
        rhs.w = ap.w;
        rhs.v = add(ap.v, cross(ap.w, r));
        rhs.w = add(rhs.w, c.w);
        rhs.v = add(rhs.v, c.v);
        S6 S;
        S.w = A.g3(i, AL_SW);
        S.v = A.g3(i, AL_SV);
        float u = 0.0f - sdot(S, A.g6(i, AL_PA));
        u -= sdot(S, imul(A.gI(i, AL_IA), rhs));
        float qdd = A.gf(i, AL_DINV) * u;
        S6 a;
        a.w = add(rhs.w, scale(S.w, qdd));
        a.v = add(rhs.v, scale(S.v, qdd));
        A.s6(i, AL_A, a);
    }
}

/* b3_art_integrate_vel (:990-1000). */
B3D_FN void art_integrate_vel(const Lane& L, const ArtWs& A, float h) {
    art_aba(L, A);
    for (int i = 0; i < A.n_links; i++) {
        if (A.gi(i, AL_FIXED)) continue;
        int b = A.gi(i, AL_BODY);
        S6 a = A.g6(i, AL_A);
        set_vlin(L, b, madd(vlin(L, b), h, a.v));
        set_vang(L, b, madd(vang(L, b), h, a.w));
    }
}

/* Link i's pose from its parent's and its joint angle q (b3_art_fk_link,
 * :509-525). */
B3D_FN void art_fk_link(const ArtWs& A, int i, float q) {
    int p = A.gi(i, AL_PARENT);
    Q rz = qaxis_angle(v3(0.0f, 0.0f, 1.0f), q);
    Q rp = A.gq(p, AL_ROT);
    Q rq = qnorm(qmul(rp, qmul(A.gq(i, AL_ROT_A), qmul(rz, qconj(A.gq(i, AL_ROT_B))))));
    V3 anchor = xf(A.g3(p, AL_POS), rp, A.g3(i, AL_ANCHOR_A));
    V3 com = add(anchor, rot(rq, sub(A.g3(i, AL_LC), A.g3(i, AL_ANCHOR_B))));
    A.sq(i, AL_ROT, rq);
    A.s3(i, AL_COM, com);
    A.s3(i, AL_POS, sub(com, rot(rq, A.g3(i, AL_LC))));
}

/* Roots move as free bodies (b3_integrate_position_state, 09_step.inl:
 * 55-93, without axis locks: locked worlds never get here); joints advance
 * by h qd, the rate clamped to the rotation limit, and the tree's poses
 * follow, written to the delta records (b3_art_integrate_pos, :1002-1032;
 * b3_art_write_delta, :981-988). */
B3D_FN void art_integrate_pos(const Lane& L, const ArtWs& A, float h, float inv_dt) {
    float max_lin = ldf(L.w, H_MAX_LINEAR_SPEED);
    float max_ang = kMaxRotation * inv_dt;
    float max_lin2 = max_lin * max_lin;
    float max_ang2 = max_ang * max_ang;
    art_refresh_q(L, A);
    for (int i = 0; i < A.n_links; i++) {
        int p = A.gi(i, AL_PARENT);
        int b = A.gi(i, AL_BODY);
        if (p < 0) {
            if (A.gi(i, AL_FIXED)) continue;
            V3 v = vlin(L, b), av = vang(L, b);
            float v2 = len2(v);
            if (v2 > max_lin2 && v2 > 0.0f) v = scale(v, rsqrt_scale(max_lin, v2));
            float w2 = len2(av);
            if (w2 > max_ang2 && w2 > 0.0f) av = scale(av, rsqrt_scale(max_ang, w2));
            set_vlin(L, b, v);
            set_vang(L, b, av);
            uint32_t* d = delta_rec(L, b);
            V3 dp = madd(r3(d, BD_DP), h, v);
            Q dq = qintegrate(rq4(d, BD_DQ), scale(av, h));
            rs3(d, BD_DP, dp);
            rsq(d, BD_DQ, dq);
            Q rq = qnorm(qmul(dq, ldq(L.w, bw(L, b, B_ROTATION))));
            V3 com = add(ld3(L.w, bw(L, b, B_CENTER)), dp);
            A.sq(i, AL_ROT, rq);
            A.s3(i, AL_COM, com);
            A.s3(i, AL_POS, sub(com, rot(rq, A.g3(i, AL_LC))));
            continue;
        }
        float qd = A.gf(i, AL_QD);
        if (qd * qd > max_ang2 && max_ang2 > 0.0f) qd = copysignf(max_ang, qd);
        art_fk_link(A, i, A.gf(i, AL_Q) + h * qd);
        if (A.gi(i, AL_FIXED)) continue;
        uint32_t* d = delta_rec(L, b);
        rs3(d, BD_DP, sub(A.g3(i, AL_COM), ld3(L.w, bw(L, b, B_CENTER))));
        rsq(d, BD_DQ, qnorm(qmul(A.gq(i, AL_ROT), qconj(ldq(L.w, bw(L, b, B_ROTATION))))));
    }
}

/* The velocity along a row (b3_art_row_eval without accelerations,
 * :688-720); the link velocities are the bodies'. */
B3D_FN float art_row_vel(const Lane& L, const ArtWs& A, const ArtRow& row) {
    float y = 0.0f;
    int ba = row.link_a >= 0 ? A.gi(row.link_a, AL_BODY) : -1;
    int bb = row.link_b >= 0 ? A.gi(row.link_b, AL_BODY) : -1;
    if (row.torque == 1) {
        if (ba >= 0) y += dot(vang(L, ba), row.n);
        if (bb >= 0) y -= dot(vang(L, bb), row.n);
        return y;
    }
    if (ba >= 0) y += dot(add(vlin(L, ba), cross(vang(L, ba), row.ra)), row.n);
    if (bb >= 0) y -= dot(add(vlin(L, bb), cross(vang(L, bb), row.rb)), row.n);
    return y;
}

/* The five rows of cut c, three linear and two angular, with their errors
 * (b3_art_cut_rows, :1123-1175); false when a side has no link. */
B3D_FN bool art_cut_rows(const Lane& L, const ArtWs& A, int c, ArtRow rows[5], float err[5]) {
    const uint32_t* w = L.w;
    int jk = A.cut(c);
    int la = art_link_of(A, ldi(w, jw(L, jk, J_BODY_A))), lb = art_link_of(A, ldi(w, jw(L, jk, J_BODY_B)));
    if (la < 0 || lb < 0) return false;
    Q rla = A.gq(la, AL_ROT), rlb = A.gq(lb, AL_ROT);
    V3 pa = xf(A.g3(la, AL_POS), rla, ld3(w, jw(L, jk, J_LOCAL_ANCHOR_A)));
    V3 pb = xf(A.g3(lb, AL_POS), rlb, ld3(w, jw(L, jk, J_LOCAL_ANCHOR_B)));
    V3 ra = sub(pa, A.g3(la, AL_COM)), rb = sub(pb, A.g3(lb, AL_COM)), d = sub(pb, pa);
    for (int k = 0; k < 3; k++) {
        V3 ax = v3(k == 0 ? 1.0f : 0.0f, k == 1 ? 1.0f : 0.0f, k == 2 ? 1.0f : 0.0f);
        rows[k].link_a = la;
        rows[k].link_b = lb;
        rows[k].torque = 0;
        rows[k].ra = ra;
        rows[k].rb = rb;
        rows[k].n = ax;
        err[k] = dot(d, ax);
    }
    Q qa = qmul(rla, ldq(w, jw(L, jk, J_LOCAL_ROT_A))), qb = qmul(rlb, ldq(w, jw(L, jk, J_LOCAL_ROT_B)));
    if (qdot(qa, qb) < 0.0f) qb = qneg(qb);
    Q rel = qinv_mul(qa, qb);
    for (int k = 3; k < 5; k++) {
        rows[k].link_a = la;
        rows[k].link_b = lb;
        rows[k].torque = 1;
        rows[k].ra = zero3();
        rows[k].rb = zero3();
        rows[k].n = rot(qa, k == 3 ? v3(1.0f, 0.0f, 0.0f) : v3(0.0f, 1.0f, 0.0f));
    }
    err[3] = 2.0f * rel.v.x;
    err[4] = 2.0f * rel.v.y;
    return true;
}

/* x = D^-1 b for a 5x5 block by Gauss-Jordan with partial pivoting
 * (b3_solve_n, :869-923); false if a pivot is below 1e-12. */
B3D_FN bool solve5(const float* D, const float* b, float* x) {
    float M[5][6];
    for (int r = 0; r < 5; r++) {
        for (int c = 0; c < 5; c++) M[r][c] = D[r * 5 + c];
        M[r][5] = b[r];
    }
    for (int k = 0; k < 5; k++) {
        int piv = k;
        float best = fabsf(M[k][k]);
        for (int r = k + 1; r < 5; r++) {
            float v = fabsf(M[r][k]);
            if (v > best) {
                best = v;
                piv = r;
            }
        }
        if (best < 1.0e-12f) return false;
        if (piv != k) {
            for (int c = k; c < 6; c++) {
                float t = M[k][c];
                M[k][c] = M[piv][c];
                M[piv][c] = t;
            }
        }
        float inv = 1.0f / M[k][k];
        for (int c = k; c < 6; c++) M[k][c] *= inv;
        for (int r = 0; r < 5; r++) {
            if (r == k) continue;
            float s = M[r][k];
            for (int c = k; c < 6; c++) M[r][c] -= s * M[k][c];
        }
    }
    for (int r = 0; r < 5; r++) x[r] = M[r][5];
    return true;
}

/* Each cut's five rows solved together against its 5x5 Delassus block,
 * Baumgarte-biased by 0.2 / h of the joint error on the biased pass
 * (b3_art_solve_cuts, :1177-1218, with b3_art_delassus_matrix, :925-940,
 * and b3_art_apply_impulses, :942-959). */
B3D_FN void art_solve_cuts(const Lane& L, const ArtWs& A, float inv_h, int use_bias, int iters) {
    int nc = A.n_cuts();
    if (nc < 1) return;
    /* the reference refreshes again before each cut's rows are evaluated;
     * the poses are unchanged within the pass and the velocities are read
     * from the bodies */
    art_pose_pass(L, A);
    for (int it = 0; it < iters; it++) {
        for (int c = 0; c < nc; c++) {
            ArtRow rows[5];
            float err[5];
            if (!art_cut_rows(L, A, c, rows, err)) continue;
            float rhs[5];
            for (int k = 0; k < 5; k++) {
                float vbias = 0.0f;
                if (use_bias) vbias = 0.2f * inv_h * err[k];
                rhs[k] = art_row_vel(L, A, rows[k]) - vbias;
            }
            /* the block depends only on the poses, which the pass does not
             * change: built on the first iteration, the same bits reused */
            float D[25], x[5], y[5];
            if (it == 0) {
                for (int k = 0; k < 5; k++) x[k] = 0.0f;
                for (int col = 0; col < 5; col++) {
                    x[col] = 1.0f;
                    art_delassus(L, A, rows, x, y, 5);
                    for (int r = 0; r < 5; r++) D[r * 5 + col] = y[r];
                    x[col] = 0.0f;
                }
                for (int k = 0; k < 5; k++) D[k * 5 + k] += 1.0e-8f;
                for (int k = 0; k < 25; k++) A.sd(c, k, D[k]);
            } else {
                for (int k = 0; k < 25; k++) D[k] = A.gd(c, k);
            }
            float lam[5];
            if (!solve5(D, rhs, lam)) {
                for (int k = 0; k < 5; k++) {
                    float ww = D[k * 5 + k];
                    lam[k] = ww > 1.0e-10f ? rhs[k] / ww : 0.0f;
                }
            }
            int any = 0;
            for (int k = 0; k < 5; k++) {
                x[k] = -lam[k];
                any |= lam[k] != 0.0f;
            }
            if (!any) continue;
            art_delassus(L, A, rows, x, y, 5);
            for (int i = 0; i < A.n_links; i++) {
                if (A.gi(i, AL_FIXED)) continue;
                int b = A.gi(i, AL_BODY);
                S6 a = A.g6(i, AL_A);
                set_vlin(L, b, add(vlin(L, b), a.v));
                set_vang(L, b, add(vang(L, b), a.w));
            }
        }
    }
}

/* What the reduced integrator cannot honour sends a world to the ordinary
 * step (09_step.inl:271-291): a weld, a motor, spring or limit, a joint
 * with fixed rotation, a kinematic body or an axis lock. */
B3D_FN bool art_reduced_supported(const Lane& L) {
    const uint32_t* w = L.w;
    int nj = clampi(ldi(w, H_JOINT_COUNT), 0, L.g.max_j);
    for (int j = 0; j < nj; j++) {
        if (ldi(w, jw(L, j, J_FIXED_ROTATION)) || ldi(w, jw(L, j, J_ENABLE_SPRING)) || ldi(w, jw(L, j, J_ENABLE_LIMIT))
                || ldi(w, jw(L, j, J_TYPE)) != kJointRevolute || ldi(w, jw(L, j, J_ENABLE_MOTOR)))
            return false;
    }
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        if (ldi(w, bw(L, b, B_TYPE)) == kKinematic || (ldu(w, bw(L, b, B_FLAGS)) & 0x3fu)) return false;
    }
    return true;
}

/* One world's b3_art_step (09_step.inl:266-323): worlds it cannot take, and
 * worlds without joints or whose tree does not build, take the step with
 * articulated contacts.  The opening is shared so that every stepping lane
 * ranks its records together. */
B3D_FN void step_world_art_reduced(const Lane& L0, float* ws, float dt, int substeps) {
    if (!(dt > 0.0f)) return;
    Lane L = L0;
    L.sslot = wave_slot(L);
    ArtParams P = art_params(L, dt, substeps);
    bool supported = art_reduced_supported(L);
    art_open(L, P);
    ArtWs A = art_ws_of(L, ws);
    if (!(supported && ldi(L.w, H_JOINT_COUNT) > 0 && art_build(L, A))) {
        art_indep_rest(L, A, P, 0);
        return;
    }
    /* b3_warm_start: this world's tree builds, so the articulated branch
     * runs whenever there are contacts */
    if (ldi(L.w, H_CONTACT_COUNT) > 0) art_warm_start(L, A);
    for (int s = 0; s < P.subs; s++) {
        art_integrate_vel(L, A, P.h);
        art_solve_contacts(L, A, P.inv_h, P.contact_speed, 1, kArtContactIters);
        art_solve_cuts(L, A, P.inv_h, 1, kArtCutIters);
        art_integrate_pos(L, A, P.h, P.inv_dt);
        art_solve_contacts(L, A, P.inv_h, P.contact_speed, 0, kArtContactIters);
        art_solve_cuts(L, A, P.inv_h, 0, kArtCutIters);
        wrow_restitution(L, P.rest_threshold);
    }
    finalize(L);
    vel_store(L);
}

}  // namespace b3d

#endif
