/*
 * b3d_lane.h - one world's step, written for one GPU lane.
 *
 * Device layout ("word-transposed tiles").  The engine keeps each batch as
 * tiles of kLanes = 64 worlds.  A world is viewed as the array of 32-bit
 * words of its B3World (include/b3_types.h, byte-identical to the
 * reference's src/puffysics/02_types.inl:306-332); word k of world w lives
 * at
 *     tile[w / 64][k][w % 64]
 * so a wave that handles one tile reads any field of all 64 worlds as one
 * contiguous 256-byte row.  Loops over bodies, shapes, contacts and joints
 * walk the same index in every lane, so almost every access is a coalesced
 * row; only lookups through a per-lane body index (contact.body_a ...)
 * scatter, and the hottest of those (velocities) are staged in LDS.
 *
 * Per-lane memory handed to the step:
 *   w    live world words    (HBM)    word k at w[k * 64]
 *   scr  per-step scratch    (HBM)    shape bounds and the old warm cache
 *   vel  body velocity rows  (LDS)    body b component c at vel[(b*7+c)*64],
 *                                     c = 0..5 lin/ang velocity, 6 = flags
 * Body velocities stay in `vel` for the whole step (b3d_vel_load /
 * b3d_vel_store move them), everything else is read and written in place.
 *
 * The arithmetic is the reference's default b3_step path, operation for
 * operation (src/puffysics/08_contacts.inl, 06_joints.inl, 07_packed.inl,
 * 09_step.inl); each function names the lines it follows.  Structure that
 * differs from the reference, with identical results:
 *   - contact creation, warm-start matching and contact preparation run in
 *     one pass over the shape pairs (preparation reads only body state that
 *     contact generation does not change);
 *   - the warm-start lookup walks the old contact list with a merge pointer
 *     when that list is strictly sorted by shape pair (the case for every
 *     list the step itself produces), else scans it like the reference;
 *   - the joint-connection test loops over the joints instead of building a
 *     bit matrix.
 */
#ifndef PUFFYSICS_AMD_B3D_LANE_H
#define PUFFYSICS_AMD_B3D_LANE_H

#include <stddef.h>

#include "b3_types.h"
#include "b3d_collide.h"

namespace b3d {

constexpr int kLanes = 64;
constexpr int kVelWords = 7;

/* ---- word offsets of the B3 structs ---- */
#define B3D_W(T, f) ((int)(offsetof(T, f) / 4))
constexpr int kBodyWords = (int)(sizeof(B3Body) / 4);
constexpr int kShapeWords = (int)(sizeof(B3Shape) / 4);
constexpr int kContactWords = (int)(sizeof(B3Contact) / 4);
constexpr int kPointWords = (int)(sizeof(B3Point) / 4);
constexpr int kJointWords = (int)(sizeof(B3Joint) / 4);
constexpr int kHeaderWords = (int)(sizeof(B3WorldHeader) / 4);

/* world header */
constexpr int H_GRAVITY = B3D_W(B3WorldHeader, gravity);
constexpr int H_CONTACT_HERTZ = B3D_W(B3WorldHeader, contact_hertz);
constexpr int H_CONTACT_DAMPING = B3D_W(B3WorldHeader, contact_damping);
constexpr int H_CONTACT_SPEED = B3D_W(B3WorldHeader, contact_speed);
constexpr int H_RESTITUTION_THRESHOLD = B3D_W(B3WorldHeader, restitution_threshold);
constexpr int H_MAX_LINEAR_SPEED = B3D_W(B3WorldHeader, max_linear_speed);
constexpr int H_BODY_COUNT = B3D_W(B3WorldHeader, body_count);
constexpr int H_SHAPE_COUNT = B3D_W(B3WorldHeader, shape_count);
constexpr int H_CONTACT_COUNT = B3D_W(B3WorldHeader, contact_count);
constexpr int H_JOINT_COUNT = B3D_W(B3WorldHeader, joint_count);
constexpr int H_CONTACT_OVERFLOW = B3D_W(B3WorldHeader, contact_overflow);
constexpr int H_CONTACTS_DROPPED = B3D_W(B3WorldHeader, contacts_dropped);

/* body */
constexpr int B_POSITION = B3D_W(B3Body, position);
constexpr int B_ROTATION = B3D_W(B3Body, rotation);
constexpr int B_CENTER = B3D_W(B3Body, center);
constexpr int B_LOCAL_CENTER = B3D_W(B3Body, local_center);
constexpr int B_LIN_VEL = B3D_W(B3Body, lin_vel);
constexpr int B_ANG_VEL = B3D_W(B3Body, ang_vel);
constexpr int B_FORCE = B3D_W(B3Body, force);
constexpr int B_TORQUE = B3D_W(B3Body, torque);
constexpr int B_DELTA_POS = B3D_W(B3Body, delta_pos);
constexpr int B_DELTA_ROT = B3D_W(B3Body, delta_rot);
constexpr int B_INV_MASS = B3D_W(B3Body, inv_mass);
constexpr int B_INV_INERTIA = B3D_W(B3Body, inv_inertia);
constexpr int B_INV_I_WORLD = B3D_W(B3Body, inv_i_world);
constexpr int B_LINEAR_DAMPING = B3D_W(B3Body, linear_damping);
constexpr int B_ANGULAR_DAMPING = B3D_W(B3Body, angular_damping);
constexpr int B_GRAVITY_SCALE = B3D_W(B3Body, gravity_scale);
constexpr int B_TYPE = B3D_W(B3Body, type);
constexpr int B_FLAGS = B3D_W(B3Body, flags);

/* shape */
constexpr int S_BODY = B3D_W(B3Shape, body);
constexpr int S_TYPE = B3D_W(B3Shape, type);
constexpr int S_LOCAL_POS = B3D_W(B3Shape, local_pos);
constexpr int S_LOCAL_ROT = B3D_W(B3Shape, local_rot);
constexpr int S_RADIUS = B3D_W(B3Shape, radius);
constexpr int S_HALF = B3D_W(B3Shape, half);
constexpr int S_FRICTION = B3D_W(B3Shape, friction);
constexpr int S_RESTITUTION = B3D_W(B3Shape, restitution);
constexpr int S_ROLLING = B3D_W(B3Shape, rolling);
constexpr int S_CATEGORY = B3D_W(B3Shape, category);
constexpr int S_MASK = B3D_W(B3Shape, mask);

/* contact and its points */
constexpr int C_SHAPE_A = B3D_W(B3Contact, shape_a);
constexpr int C_SHAPE_B = B3D_W(B3Contact, shape_b);
constexpr int C_BODY_A = B3D_W(B3Contact, body_a);
constexpr int C_BODY_B = B3D_W(B3Contact, body_b);
constexpr int C_POINT_COUNT = B3D_W(B3Contact, point_count);
constexpr int C_STATIC = B3D_W(B3Contact, static_contact);
constexpr int C_NORMAL = B3D_W(B3Contact, normal);
constexpr int C_TANGENT1 = B3D_W(B3Contact, tangent1);
constexpr int C_TANGENT2 = B3D_W(B3Contact, tangent2);
constexpr int C_POINTS = B3D_W(B3Contact, points);
constexpr int C_CENTER_A = B3D_W(B3Contact, center_a);
constexpr int C_CENTER_B = B3D_W(B3Contact, center_b);
constexpr int C_FRICTION = B3D_W(B3Contact, friction);
constexpr int C_RESTITUTION = B3D_W(B3Contact, restitution);
constexpr int C_ROLLING = B3D_W(B3Contact, rolling);
constexpr int C_TWIST_MASS = B3D_W(B3Contact, twist_mass);
constexpr int C_TWIST_IMPULSE = B3D_W(B3Contact, twist_impulse);
constexpr int C_FRICTION_IMPULSE = B3D_W(B3Contact, friction_impulse);
constexpr int C_ROLLING_IMPULSE = B3D_W(B3Contact, rolling_impulse);
constexpr int C_TANGENT_MASS = B3D_W(B3Contact, tangent_mass);
constexpr int C_ROLLING_MASS = B3D_W(B3Contact, rolling_mass);
constexpr int C_INV_MASS_A = B3D_W(B3Contact, inv_mass_a);
constexpr int C_INV_MASS_B = B3D_W(B3Contact, inv_mass_b);
constexpr int C_INV_I_A = B3D_W(B3Contact, inv_i_a);
constexpr int C_INV_I_B = B3D_W(B3Contact, inv_i_b);
constexpr int C_SOFTNESS = B3D_W(B3Contact, softness);
constexpr int P_R_A = B3D_W(B3Point, r_a);
constexpr int P_R_B = B3D_W(B3Point, r_b);
constexpr int P_BASE_SEP = B3D_W(B3Point, base_sep);
constexpr int P_REL_VEL = B3D_W(B3Point, rel_vel);
constexpr int P_NORMAL_IMPULSE = B3D_W(B3Point, normal_impulse);
constexpr int P_TOTAL_NORMAL = B3D_W(B3Point, total_normal);
constexpr int P_NORMAL_MASS = B3D_W(B3Point, normal_mass);
constexpr int P_LEVER = B3D_W(B3Point, lever);
constexpr int P_FEATURE = B3D_W(B3Point, feature);

/* joint */
constexpr int J_TYPE = B3D_W(B3Joint, type);
constexpr int J_BODY_A = B3D_W(B3Joint, body_a);
constexpr int J_BODY_B = B3D_W(B3Joint, body_b);
constexpr int J_COLLIDE_CONNECTED = B3D_W(B3Joint, collide_connected);
constexpr int J_FIXED_ROTATION = B3D_W(B3Joint, fixed_rotation);
constexpr int J_LOCAL_ANCHOR_A = B3D_W(B3Joint, local_anchor_a);
constexpr int J_LOCAL_ANCHOR_B = B3D_W(B3Joint, local_anchor_b);
constexpr int J_LOCAL_ROT_A = B3D_W(B3Joint, local_rot_a);
constexpr int J_LOCAL_ROT_B = B3D_W(B3Joint, local_rot_b);
constexpr int J_CONSTRAINT_HERTZ = B3D_W(B3Joint, constraint_hertz);
constexpr int J_CONSTRAINT_DAMPING = B3D_W(B3Joint, constraint_damping);
constexpr int J_SOFTNESS = B3D_W(B3Joint, softness);
constexpr int J_INV_MASS_A = B3D_W(B3Joint, inv_mass_a);
constexpr int J_INV_MASS_B = B3D_W(B3Joint, inv_mass_b);
constexpr int J_INV_I_A = B3D_W(B3Joint, inv_i_a);
constexpr int J_INV_I_B = B3D_W(B3Joint, inv_i_b);
constexpr int J_FRAME_P_A = B3D_W(B3Joint, frame_p_a);
constexpr int J_FRAME_P_B = B3D_W(B3Joint, frame_p_b);
constexpr int J_FRAME_Q_A = B3D_W(B3Joint, frame_q_a);
constexpr int J_FRAME_Q_B = B3D_W(B3Joint, frame_q_b);
constexpr int J_DELTA_CENTER = B3D_W(B3Joint, delta_center);
constexpr int J_LINEAR_IMPULSE = B3D_W(B3Joint, linear_impulse);
constexpr int J_ANGULAR_IMPULSE = B3D_W(B3Joint, angular_impulse);
constexpr int J_ANGULAR_MASS = B3D_W(B3Joint, angular_mass);
constexpr int J_LINEAR_HERTZ = B3D_W(B3Joint, linear_hertz);
constexpr int J_LINEAR_DAMPING = B3D_W(B3Joint, linear_damping);
constexpr int J_ANGULAR_HERTZ = B3D_W(B3Joint, angular_hertz);
constexpr int J_ANGULAR_DAMPING = B3D_W(B3Joint, angular_damping);
constexpr int J_LINEAR_SPRING = B3D_W(B3Joint, linear_spring);
constexpr int J_ANGULAR_SPRING = B3D_W(B3Joint, angular_spring);
constexpr int J_PERP_IMPULSE = B3D_W(B3Joint, perp_impulse);
constexpr int J_SPRING_IMPULSE = B3D_W(B3Joint, spring_impulse);
constexpr int J_MOTOR_IMPULSE = B3D_W(B3Joint, motor_impulse);
constexpr int J_LOWER_IMPULSE = B3D_W(B3Joint, lower_impulse);
constexpr int J_UPPER_IMPULSE = B3D_W(B3Joint, upper_impulse);
constexpr int J_HERTZ = B3D_W(B3Joint, hertz);
constexpr int J_DAMPING_RATIO = B3D_W(B3Joint, damping_ratio);
constexpr int J_MAX_MOTOR_TORQUE = B3D_W(B3Joint, max_motor_torque);
constexpr int J_MOTOR_SPEED = B3D_W(B3Joint, motor_speed);
constexpr int J_TARGET_ANGLE = B3D_W(B3Joint, target_angle);
constexpr int J_LOWER_ANGLE = B3D_W(B3Joint, lower_angle);
constexpr int J_UPPER_ANGLE = B3D_W(B3Joint, upper_angle);
constexpr int J_ENABLE_SPRING = B3D_W(B3Joint, enable_spring);
constexpr int J_ENABLE_MOTOR = B3D_W(B3Joint, enable_motor);
constexpr int J_ENABLE_LIMIT = B3D_W(B3Joint, enable_limit);
constexpr int J_ROTATION_AXIS = B3D_W(B3Joint, rotation_axis);
constexpr int J_PERP_X = B3D_W(B3Joint, perp_x);
constexpr int J_PERP_Y = B3D_W(B3Joint, perp_y);
constexpr int J_AXIAL_MASS = B3D_W(B3Joint, axial_mass);
constexpr int J_SPRING_SOFTNESS = B3D_W(B3Joint, spring_softness);

/* old warm-cache record in scratch (the reference's B3Warm, 02_types.inl:133-142) */
constexpr int O_SHAPE_A = 0, O_SHAPE_B = 1, O_POINT_COUNT = 2, O_FEATURE = 3, O_NORMAL_IMPULSE = 7,
              O_FRICTION_IMPULSE = 11, O_TWIST_IMPULSE = 13, O_ROLLING_IMPULSE = 14, kOldWords = 17;
constexpr int kAabbWords = 6;

constexpr int kStatic = 0, kKinematic = 1, kDynamic = 2;
constexpr uint32_t kFlagDynamic = 0x00001000u;
constexpr int kJointWeld = 0, kJointRevolute = 1;
constexpr int kJointIters = 2, kRelaxIters = 2;  /* B3_JOINT_ITERS, B3_RELAX_ITERS */
constexpr float kMaxRotation = 0.25f * 3.14159265359f;
constexpr float kMinFrictionW = 1.0e-10f;

/* Array geometry of one capacity set, in words. */
struct Geometry {
    int max_b, max_s, max_c, max_j;
    int bo, so, co, jo;   /* word offsets of bodies, shapes, contacts, joints */
    int world_words;      /* words per world (sizeof(B3World) / 4) */
    int scr_aabb, scr_old, scr_words;
};

/* Geometry of a capacity signature; false when it is invalid. */
B3D_FN bool geometry_of(unsigned long long sig, Geometry* g, size_t* world_bytes) {
    B3Layout L;
    if (!b3_layout_of(sig, &L)) return false;
    if ((L.bodies_off | L.shapes_off | L.contacts_off | L.joints_off | L.world_size) & 3u) return false;
    g->max_b = L.max_bodies;
    g->max_s = L.max_shapes;
    g->max_c = L.max_contacts;
    g->max_j = L.max_joints;
    g->bo = (int)(L.bodies_off / 4);
    g->so = (int)(L.shapes_off / 4);
    g->co = (int)(L.contacts_off / 4);
    g->jo = (int)(L.joints_off / 4);
    g->world_words = (int)(L.world_size / 4);
    g->scr_aabb = 0;
    g->scr_old = g->max_s * kAabbWords;
    g->scr_words = g->scr_old + g->max_c * kOldWords;
    *world_bytes = L.world_size;
    return true;
}

/* Per-lane view of one world. */
struct Lane {
    uint32_t* w;    /* live tile + lane */
    uint32_t* scr;  /* scratch tile + lane */
    float* vel;     /* velocity rows + lane */
    Geometry g;
};

/* Word ranges [lo[i], hi[i]) that a snapshot restore copies: header,
 * bodies and shapes; the snapshot's live contacts; every joint slot.  These
 * are all the words b3_step reads before writing (b3_batch_restore copies
 * the whole struct, b3_batch.cuh:53-60; the rest is dead contact storage). */
B3D_FN void restore_ranges(const Geometry& g, int snap_contacts, int lo[3], int hi[3]) {
    int cc = snap_contacts < 0 ? 0 : (snap_contacts > g.max_c ? g.max_c : snap_contacts);
    lo[0] = 0;
    hi[0] = g.co;
    lo[1] = g.co;
    hi[1] = g.co + cc * kContactWords;
    lo[2] = g.jo;
    hi[2] = g.jo + g.max_j * kJointWords;
}

/* ---- word access (stride kLanes) ---- */
B3D_FN float ldf(const uint32_t* p, int k) { return __builtin_bit_cast(float, p[k * kLanes]); }
B3D_FN int ldi(const uint32_t* p, int k) { return (int)p[k * kLanes]; }
B3D_FN uint32_t ldu(const uint32_t* p, int k) { return p[k * kLanes]; }
B3D_FN void stf(uint32_t* p, int k, float v) { p[k * kLanes] = __builtin_bit_cast(uint32_t, v); }
B3D_FN void sti(uint32_t* p, int k, int v) { p[k * kLanes] = (uint32_t)v; }
B3D_FN V3 ld3(const uint32_t* p, int k) { return v3(ldf(p, k), ldf(p, k + 1), ldf(p, k + 2)); }
B3D_FN void st3(uint32_t* p, int k, V3 v) { stf(p, k, v.x); stf(p, k + 1, v.y); stf(p, k + 2, v.z); }
B3D_FN Q ldq(const uint32_t* p, int k) { return q4(ldf(p, k), ldf(p, k + 1), ldf(p, k + 2), ldf(p, k + 3)); }
B3D_FN void stq(uint32_t* p, int k, Q q) { st3(p, k, q.v); stf(p, k + 3, q.s); }
B3D_FN M3 ldm3(const uint32_t* p, int k) { M3 m; m.cx = ld3(p, k); m.cy = ld3(p, k + 3); m.cz = ld3(p, k + 6); return m; }
B3D_FN void stm3(uint32_t* p, int k, M3 m) { st3(p, k, m.cx); st3(p, k + 3, m.cy); st3(p, k + 6, m.cz); }
B3D_FN Soft ldsoft(const uint32_t* p, int k) { Soft s; s.bias_rate = ldf(p, k); s.mass_scale = ldf(p, k + 1); s.impulse_scale = ldf(p, k + 2); return s; }
B3D_FN void stsoft(uint32_t* p, int k, Soft s) { stf(p, k, s.bias_rate); stf(p, k + 1, s.mass_scale); stf(p, k + 2, s.impulse_scale); }
B3D_FN uint64_t ldu64(const uint32_t* p, int k) { return (uint64_t)ldu(p, k) | ((uint64_t)ldu(p, k + 1) << 32); }

B3D_FN int bw(const Lane& L, int b, int f) { return L.g.bo + b * kBodyWords + f; }
B3D_FN int sw(const Lane& L, int s, int f) { return L.g.so + s * kShapeWords + f; }
B3D_FN int cw(const Lane& L, int c, int f) { return L.g.co + c * kContactWords + f; }
B3D_FN int pw(const Lane& L, int c, int p, int f) { return L.g.co + c * kContactWords + C_POINTS + p * kPointWords + f; }
B3D_FN int jw(const Lane& L, int j, int f) { return L.g.jo + j * kJointWords + f; }
B3D_FN int clampi(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }

/* ---- body velocity rows ---- */
B3D_FN V3 vlin(const Lane& L, int b) { const float* v = L.vel + b * kVelWords * kLanes; return v3(v[0], v[kLanes], v[2 * kLanes]); }
B3D_FN V3 vang(const Lane& L, int b) { const float* v = L.vel + (b * kVelWords + 3) * kLanes; return v3(v[0], v[kLanes], v[2 * kLanes]); }
B3D_FN void set_vlin(const Lane& L, int b, V3 x) { float* v = L.vel + b * kVelWords * kLanes; v[0] = x.x; v[kLanes] = x.y; v[2 * kLanes] = x.z; }
B3D_FN void set_vang(const Lane& L, int b, V3 x) { float* v = L.vel + (b * kVelWords + 3) * kLanes; v[0] = x.x; v[kLanes] = x.y; v[2 * kLanes] = x.z; }
B3D_FN int is_dyn_flag(const Lane& L, int b) {
    return (__builtin_bit_cast(uint32_t, L.vel[(b * kVelWords + 6) * kLanes]) & kFlagDynamic) != 0;
}

B3D_FN int body_count(const Lane& L) { return clampi(ldi(L.w, H_BODY_COUNT), 0, L.g.max_b); }

/* Stage velocities and flags of every body into the velocity rows. */
B3D_FN void vel_load(const Lane& L) {
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        float* v = L.vel + b * kVelWords * kLanes;
        for (int c = 0; c < 6; c++) v[c * kLanes] = ldf(L.w, bw(L, b, B_LIN_VEL + c));
        v[6 * kLanes] = ldf(L.w, bw(L, b, B_FLAGS));
    }
}
B3D_FN void vel_store(const Lane& L) {
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        const float* v = L.vel + b * kVelWords * kLanes;
        for (int c = 0; c < 6; c++) stf(L.w, bw(L, b, B_LIN_VEL + c), v[c * kLanes]);
    }
}

/* ---- shape pose and bounds (04_world.inl:293-336) ---- */
B3D_FN Posed pose_shape(const Lane& L, int s, V3 bpos, Q brot) {
    Posed P;
    P.type = ldi(L.w, sw(L, s, S_TYPE));
    P.p = xf(bpos, brot, ld3(L.w, sw(L, s, S_LOCAL_POS)));
    P.q = qmul(brot, ldq(L.w, sw(L, s, S_LOCAL_ROT)));
    P.radius = ldf(L.w, sw(L, s, S_RADIUS));
    P.half = ld3(L.w, sw(L, s, S_HALF));
    return P;
}
B3D_FN void shape_aabb(const Posed& P, V3* lo, V3* hi) {
    if (P.type == kSphere) {
        V3 e = v3(P.radius, P.radius, P.radius);
        *lo = sub(P.p, e);
        *hi = add(P.p, e);
        return;
    }
    if (P.type == kCapsule) {
        V3 y = rot(P.q, v3(0.0f, P.half.y, 0.0f));
        V3 c1 = sub(P.p, y);
        V3 c2 = add(P.p, y);
        V3 e = v3(P.radius, P.radius, P.radius);
        V3 l = v3(minf(c1.x, c2.x), minf(c1.y, c2.y), minf(c1.z, c2.z));
        V3 h = v3(maxf(c1.x, c2.x), maxf(c1.y, c2.y), maxf(c1.z, c2.z));
        *lo = sub(l, e);
        *hi = add(h, e);
        return;
    }
    V3 ax, ay, az;
    axes(P.q, &ax, &ay, &az);
    V3 e = v3(fabsf(ax.x) * P.half.x + fabsf(ay.x) * P.half.y + fabsf(az.x) * P.half.z,
        fabsf(ax.y) * P.half.x + fabsf(ay.y) * P.half.y + fabsf(az.y) * P.half.z,
        fabsf(ax.z) * P.half.x + fabsf(ay.z) * P.half.y + fabsf(az.z) * P.half.z);
    *lo = sub(P.p, e);
    *hi = add(P.p, e);
}

/* Is there a joint with collide_connected == 0 between bodies a and b? */
B3D_FN int joined(const Lane& L, int nj, int a, int b) {
    for (int i = 0; i < nj; i++) {
        if (ldi(L.w, jw(L, i, J_COLLIDE_CONNECTED))) continue;
        int ja = ldi(L.w, jw(L, i, J_BODY_A)), jb = ldi(L.w, jw(L, i, J_BODY_B));
        if ((ja == a && jb == b) || (ja == b && jb == a)) return 1;
    }
    return 0;
}

struct BodyLite { V3 center; int type; float inv_mass; M3 inv_i; };

B3D_FN BodyLite body_lite(const Lane& L, int b) {
    BodyLite r;
    r.center = ld3(L.w, bw(L, b, B_CENTER));
    r.type = ldi(L.w, bw(L, b, B_TYPE));
    r.inv_mass = ldf(L.w, bw(L, b, B_INV_MASS));
    r.inv_i = ldm3(L.w, bw(L, b, B_INV_I_WORLD));
    return r;
}

/* Copy one contact's warm-start data into the old-cache scratch
 * (08_contacts.inl:65-91). */
B3D_FN void save_old(const Lane& L, int k) {
    uint32_t* o = L.scr + (L.g.scr_old + k * kOldWords) * kLanes;
    int pc = clampi(ldi(L.w, cw(L, k, C_POINT_COUNT)), 0, kMaxManifold);
    sti(o, O_SHAPE_A, ldi(L.w, cw(L, k, C_SHAPE_A)));
    sti(o, O_SHAPE_B, ldi(L.w, cw(L, k, C_SHAPE_B)));
    sti(o, O_POINT_COUNT, pc);
    for (int p = 0; p < pc; p++) {
        sti(o, O_FEATURE + p, ldi(L.w, pw(L, k, p, P_FEATURE)));
        stf(o, O_NORMAL_IMPULSE + p, ldf(L.w, pw(L, k, p, P_NORMAL_IMPULSE)));
    }
    stf(o, O_FRICTION_IMPULSE, ldf(L.w, cw(L, k, C_FRICTION_IMPULSE)));
    stf(o, O_FRICTION_IMPULSE + 1, ldf(L.w, cw(L, k, C_FRICTION_IMPULSE + 1)));
    stf(o, O_TWIST_IMPULSE, ldf(L.w, cw(L, k, C_TWIST_IMPULSE)));
    st3(o, O_ROLLING_IMPULSE, ld3(L.w, cw(L, k, C_ROLLING_IMPULSE)));
}

/* A new contact assembled in registers before it is written out. */
struct NewContact {
    int count;
    V3 normal, t1, t2;
    V3 r_a[kMaxManifold], r_b[kMaxManifold];
    float base_sep[kMaxManifold];
    uint32_t feature[kMaxManifold];
    float ni[kMaxManifold];
    V2 fi;
    float twist;
    V3 roll;
};

/* Take the impulses of old record k for the points whose feature matches
 * (08_contacts.inl:154-170; the last matching old point wins). */
B3D_FN void warm_from_old(const Lane& L, int k, NewContact* nc) {
    const uint32_t* o = L.scr + (L.g.scr_old + k * kOldWords) * kLanes;
    int opc = ldi(o, O_POINT_COUNT);
    for (int p = 0; p < nc->count; p++)
        for (int q = 0; q < opc; q++)
            if (nc->feature[p] == ldu(o, O_FEATURE + q)) nc->ni[p] = ldf(o, O_NORMAL_IMPULSE + q);
    nc->fi.x = ldf(o, O_FRICTION_IMPULSE);
    nc->fi.y = ldf(o, O_FRICTION_IMPULSE + 1);
    nc->twist = ldf(o, O_TWIST_IMPULSE);
    nc->roll = ld3(o, O_ROLLING_IMPULSE);
}

B3D_FN int pair_less(int a0, int b0, int a1, int b1) { return a0 < a1 || (a0 == a1 && b0 < b1); }

/* Contact generation, warm start and contact preparation for one world:
 * b3_find_contacts (08_contacts.inl:64-173) with b3_contact_from_mani
 * (08:5-39) and b3_prepare_one_contact (08:234-291) applied to each new
 * contact as it is produced. */
B3D_FN void collide_and_prepare(const Lane& L, Soft cs, Soft ss) {
    const Geometry& g = L.g;
    int old_n = clampi(ldi(L.w, H_CONTACT_COUNT), 0, g.max_c);
    int sorted = 1;
    int pa_prev = 0, pb_prev = 0;
    for (int k = 0; k < old_n; k++) {
        save_old(L, k);
        int a = ldi(L.w, cw(L, k, C_SHAPE_A)), b = ldi(L.w, cw(L, k, C_SHAPE_B));
        if (k > 0 && !pair_less(pa_prev, pb_prev, a, b)) sorted = 0;
        pa_prev = a;
        pb_prev = b;
    }
    int ns = clampi(ldi(L.w, H_SHAPE_COUNT), 0, g.max_s);
    int nj = clampi(ldi(L.w, H_JOINT_COUNT), 0, g.max_j);
    V3 pad = v3(kSpeculative, kSpeculative, kSpeculative);
    for (int s = 0; s < ns; s++) {
        int b = ldi(L.w, sw(L, s, S_BODY));
        Posed P = pose_shape(L, s, ld3(L.w, bw(L, b, B_POSITION)), ldq(L.w, bw(L, b, B_ROTATION)));
        V3 lo, hi;
        shape_aabb(P, &lo, &hi);
        uint32_t* a = L.scr + (g.scr_aabb + s * kAabbWords) * kLanes;
        st3(a, 0, sub(lo, pad));
        st3(a, 3, add(hi, pad));
    }
    int cc = 0;
    int overflow = ldi(L.w, H_CONTACT_OVERFLOW);
    int dropped = ldi(L.w, H_CONTACTS_DROPPED);
    int optr = 0;
    const float inv_tau = 1.0f / kSpeculative;
    for (int i = 0; i < ns; i++) {
        const uint32_t* ai = L.scr + (g.scr_aabb + i * kAabbWords) * kLanes;
        V3 lo_i = ld3(ai, 0), hi_i = ld3(ai, 3);
        int body_i = ldi(L.w, sw(L, i, S_BODY));
        int type_bi = ldi(L.w, bw(L, body_i, B_TYPE));
        uint64_t cat_i = ldu64(L.w, sw(L, i, S_CATEGORY));
        uint64_t mask_i = ldu64(L.w, sw(L, i, S_MASK));
        for (int j = i + 1; j < ns; j++) {
            /* b3_broadphase_pair (08:45-62): bounds first, then the rest */
            const uint32_t* aj = L.scr + (g.scr_aabb + j * kAabbWords) * kLanes;
            V3 lo_j = ld3(aj, 0), hi_j = ld3(aj, 3);
            if (!(lo_i.x <= hi_j.x && hi_i.x >= lo_j.x && lo_i.y <= hi_j.y && hi_i.y >= lo_j.y
                    && lo_i.z <= hi_j.z && hi_i.z >= lo_j.z))
                continue;
            int body_j = ldi(L.w, sw(L, j, S_BODY));
            if (body_i == body_j) continue;
            int type_bj = ldi(L.w, bw(L, body_j, B_TYPE));
            if (type_bi == kStatic && type_bj == kStatic) continue;
            if ((cat_i & ldu64(L.w, sw(L, j, S_MASK))) == 0 || (ldu64(L.w, sw(L, j, S_CATEGORY)) & mask_i) == 0)
                continue;
            if (joined(L, nj, body_i, body_j)) continue;

            Posed A = pose_shape(L, i, ld3(L.w, bw(L, body_i, B_POSITION)), ldq(L.w, bw(L, body_i, B_ROTATION)));
            Posed B = pose_shape(L, j, ld3(L.w, bw(L, body_j, B_POSITION)), ldq(L.w, bw(L, body_j, B_ROTATION)));
            Mani m;
            collide_pair(&m, A, B);
            if (m.count == 0) continue;
            if (cc >= g.max_c) {
                overflow = 1;
                dropped++;
                continue;
            }
            /* b3_contact_from_mani (08:5-39) */
            NewContact nc;
            nc.count = m.count;
            nc.normal = m.normal;
            nc.t1 = perp(m.normal);
            nc.t2 = cross(nc.t1, m.normal);
            BodyLite ba = body_lite(L, body_i);
            BodyLite bb = body_lite(L, body_j);
            float fa = ldf(L.w, sw(L, i, S_FRICTION)), fb = ldf(L.w, sw(L, j, S_FRICTION));
            float ea = ldf(L.w, sw(L, i, S_RESTITUTION)), eb = ldf(L.w, sw(L, j, S_RESTITUTION));
            float rolling = maxf(ldf(L.w, sw(L, i, S_ROLLING)), ldf(L.w, sw(L, j, S_ROLLING)));
            float friction = sqrtf(fa * fb);
            float restitution = ea > eb ? ea : eb;
            int static_contact = ba.type != kDynamic || bb.type != kDynamic;
            for (int p = 0; p < m.count; p++) {
                nc.r_a[p] = sub(m.p_a[p], ba.center);
                nc.r_b[p] = sub(m.p_b[p], bb.center);
                nc.base_sep[p] = m.sep[p] - dot(sub(nc.r_b[p], nc.r_a[p]), m.normal);
                nc.feature[p] = m.feature[p];
                nc.ni[p] = 0.0f;
            }
            nc.fi = V2{0.0f, 0.0f};
            nc.twist = 0.0f;
            nc.roll = zero3();
            /* warm start from the previous step's cache */
            if (sorted) {
                while (optr < old_n) {
                    const uint32_t* o = L.scr + (g.scr_old + optr * kOldWords) * kLanes;
                    if (!pair_less(ldi(o, O_SHAPE_A), ldi(o, O_SHAPE_B), i, j)) break;
                    optr++;
                }
                if (optr < old_n) {
                    const uint32_t* o = L.scr + (g.scr_old + optr * kOldWords) * kLanes;
                    if (ldi(o, O_SHAPE_A) == i && ldi(o, O_SHAPE_B) == j) warm_from_old(L, optr, &nc);
                }
            } else {
                for (int k = 0; k < old_n; k++) {
                    const uint32_t* o = L.scr + (g.scr_old + k * kOldWords) * kLanes;
                    if (ldi(o, O_SHAPE_A) == i && ldi(o, O_SHAPE_B) == j) warm_from_old(L, k, &nc);
                }
            }

            /* b3_prepare_one_contact (08:234-291) */
            float ma = ba.type == kDynamic ? ba.inv_mass : 0.0f;
            float mb = bb.type == kDynamic ? bb.inv_mass : 0.0f;
            M3 ia = ba.type == kDynamic ? ba.inv_i : m3zero();
            M3 ib = bb.type == kDynamic ? bb.inv_i : m3zero();
            V3 n = nc.normal;
            V3 va = vlin(L, body_i), wa = vang(L, body_i);
            V3 vb = vlin(L, body_j), wb = vang(L, body_j);
            V3 center_a = zero3(), center_b = zero3();
            float wsum = 0.0f;
            float nmass[kMaxManifold], rel_vel[kMaxManifold];
            for (int p = 0; p < nc.count; p++) {
                V3 rn_a = cross(nc.r_a[p], n);
                V3 rn_b = cross(nc.r_b[p], n);
                float kn = ma + mb + dot(rn_a, mv(ia, rn_a)) + dot(rn_b, mv(ib, rn_b));
                nmass[p] = kn > 0.0f ? 1.0f / kn : 0.0f;
                V3 vra = add(va, cross(wa, nc.r_a[p]));
                V3 vrb = add(vb, cross(wb, nc.r_b[p]));
                rel_vel[p] = dot(n, sub(vrb, vra));
                float sep = nc.base_sep[p] + dot(sub(nc.r_b[p], nc.r_a[p]), n);
                float weight = clampf(2.0f - sep * inv_tau, kMinFrictionW, 1.0f);
                center_a = madd(center_a, weight, nc.r_a[p]);
                center_b = madd(center_b, weight, nc.r_b[p]);
                wsum += weight;
            }
            float invw = wsum > 0.0f ? 1.0f / wsum : 0.0f;
            center_a = scale(center_a, invw);
            center_b = scale(center_b, invw);
            V3 rt_a1 = cross(center_a, nc.t1);
            V3 rt_a2 = cross(center_a, nc.t2);
            V3 rt_b1 = cross(center_b, nc.t1);
            V3 rt_b2 = cross(center_b, nc.t2);
            M2 k2;
            k2.cx.x = ma + mb + dot(rt_a1, mv(ia, rt_a1)) + dot(rt_b1, mv(ib, rt_b1));
            k2.cy.y = ma + mb + dot(rt_a2, mv(ia, rt_a2)) + dot(rt_b2, mv(ib, rt_b2));
            k2.cx.y = dot(rt_a1, mv(ia, rt_a2)) + dot(rt_b1, mv(ib, rt_b2));
            k2.cy.x = k2.cx.y;
            M2 tmass = inv2(k2);
            M3 isum = madd3(ia, ib);
            float kt = dot(n, mv(isum, n));
            float twist_mass = kt > 0.0f ? 1.0f / kt : 0.0f;

            /* write the contact row */
            uint32_t* w = L.w;
            sti(w, cw(L, cc, C_SHAPE_A), i);
            sti(w, cw(L, cc, C_SHAPE_B), j);
            sti(w, cw(L, cc, C_BODY_A), body_i);
            sti(w, cw(L, cc, C_BODY_B), body_j);
            sti(w, cw(L, cc, C_POINT_COUNT), nc.count);
            sti(w, cw(L, cc, C_STATIC), static_contact);
            st3(w, cw(L, cc, C_NORMAL), nc.normal);
            st3(w, cw(L, cc, C_TANGENT1), nc.t1);
            st3(w, cw(L, cc, C_TANGENT2), nc.t2);
            for (int p = 0; p < nc.count; p++) {
                st3(w, pw(L, cc, p, P_R_A), nc.r_a[p]);
                st3(w, pw(L, cc, p, P_R_B), nc.r_b[p]);
                stf(w, pw(L, cc, p, P_BASE_SEP), nc.base_sep[p]);
                stf(w, pw(L, cc, p, P_REL_VEL), rel_vel[p]);
                stf(w, pw(L, cc, p, P_NORMAL_IMPULSE), nc.ni[p]);
                stf(w, pw(L, cc, p, P_TOTAL_NORMAL), 0.0f);
                stf(w, pw(L, cc, p, P_NORMAL_MASS), nmass[p]);
                stf(w, pw(L, cc, p, P_LEVER), len(sub(nc.r_a[p], center_a)));
                sti(w, pw(L, cc, p, P_FEATURE), (int)nc.feature[p]);
            }
            st3(w, cw(L, cc, C_CENTER_A), center_a);
            st3(w, cw(L, cc, C_CENTER_B), center_b);
            stf(w, cw(L, cc, C_FRICTION), friction);
            stf(w, cw(L, cc, C_RESTITUTION), restitution);
            stf(w, cw(L, cc, C_ROLLING), rolling);
            stf(w, cw(L, cc, C_TWIST_MASS), twist_mass);
            stf(w, cw(L, cc, C_TWIST_IMPULSE), nc.twist);
            stf(w, cw(L, cc, C_FRICTION_IMPULSE), nc.fi.x);
            stf(w, cw(L, cc, C_FRICTION_IMPULSE + 1), nc.fi.y);
            st3(w, cw(L, cc, C_ROLLING_IMPULSE), nc.roll);
            stf(w, cw(L, cc, C_TANGENT_MASS), tmass.cx.x);
            stf(w, cw(L, cc, C_TANGENT_MASS + 1), tmass.cx.y);
            stf(w, cw(L, cc, C_TANGENT_MASS + 2), tmass.cy.x);
            stf(w, cw(L, cc, C_TANGENT_MASS + 3), tmass.cy.y);
            stm3(w, cw(L, cc, C_ROLLING_MASS), inv3(isum));
            stf(w, cw(L, cc, C_INV_MASS_A), ma);
            stf(w, cw(L, cc, C_INV_MASS_B), mb);
            stm3(w, cw(L, cc, C_INV_I_A), ia);
            stm3(w, cw(L, cc, C_INV_I_B), ib);
            stsoft(w, cw(L, cc, C_SOFTNESS), static_contact ? ss : cs);
            cc++;
        }
    }
    sti(L.w, H_CONTACT_COUNT, cc);
    sti(L.w, H_CONTACT_OVERFLOW, overflow);
    sti(L.w, H_CONTACTS_DROPPED, dropped);
}

/* b3_prepare_joints (06_joints.inl:161-202). */
B3D_FN void prepare_joints(const Lane& L, float h) {
    int nj = clampi(ldi(L.w, H_JOINT_COUNT), 0, L.g.max_j);
    uint32_t* w = L.w;
    for (int i = 0; i < nj; i++) {
        int a = ldi(w, jw(L, i, J_BODY_A)), b = ldi(w, jw(L, i, J_BODY_B));
        int ta = ldi(w, bw(L, a, B_TYPE)), tb = ldi(w, bw(L, b, B_TYPE));
        float ma = ta == kDynamic ? ldf(w, bw(L, a, B_INV_MASS)) : 0.0f;
        float mb = tb == kDynamic ? ldf(w, bw(L, b, B_INV_MASS)) : 0.0f;
        M3 ia = ta == kDynamic ? ldm3(w, bw(L, a, B_INV_I_WORLD)) : m3zero();
        M3 ib = tb == kDynamic ? ldm3(w, bw(L, b, B_INV_I_WORLD)) : m3zero();
        stf(w, jw(L, i, J_INV_MASS_A), ma);
        stf(w, jw(L, i, J_INV_MASS_B), mb);
        stm3(w, jw(L, i, J_INV_I_A), ia);
        stm3(w, jw(L, i, J_INV_I_B), ib);
        M3 isum = madd3(ia, ib);
        sti(w, jw(L, i, J_FIXED_ROTATION), dot(isum.cx, cross(isum.cy, isum.cz)) < 1.0e-20f);
        Soft soft = make_soft(ldf(w, jw(L, i, J_CONSTRAINT_HERTZ)), ldf(w, jw(L, i, J_CONSTRAINT_DAMPING)), h);
        stsoft(w, jw(L, i, J_SOFTNESS), soft);
        Q rot_a = ldq(w, bw(L, a, B_ROTATION)), rot_b = ldq(w, bw(L, b, B_ROTATION));
        Q fqa = qmul(rot_a, ldq(w, jw(L, i, J_LOCAL_ROT_A)));
        Q fqb = qmul(rot_b, ldq(w, jw(L, i, J_LOCAL_ROT_B)));
        stq(w, jw(L, i, J_FRAME_Q_A), fqa);
        stq(w, jw(L, i, J_FRAME_Q_B), fqb);
        st3(w, jw(L, i, J_FRAME_P_A), rot(rot_a, sub(ld3(w, jw(L, i, J_LOCAL_ANCHOR_A)), ld3(w, bw(L, a, B_LOCAL_CENTER)))));
        st3(w, jw(L, i, J_FRAME_P_B), rot(rot_b, sub(ld3(w, jw(L, i, J_LOCAL_ANCHOR_B)), ld3(w, bw(L, b, B_LOCAL_CENTER)))));
        st3(w, jw(L, i, J_DELTA_CENTER), sub(ld3(w, bw(L, b, B_CENTER)), ld3(w, bw(L, a, B_CENTER))));
        if (ldi(w, jw(L, i, J_TYPE)) == kJointWeld) {
            stm3(w, jw(L, i, J_ANGULAR_MASS), inv3(isum));
            float lh = ldf(w, jw(L, i, J_LINEAR_HERTZ)), ah = ldf(w, jw(L, i, J_ANGULAR_HERTZ));
            stsoft(w, jw(L, i, J_LINEAR_SPRING), lh == 0.0f ? soft : make_soft(lh, ldf(w, jw(L, i, J_LINEAR_DAMPING)), h));
            stsoft(w, jw(L, i, J_ANGULAR_SPRING), ah == 0.0f ? soft : make_soft(ah, ldf(w, jw(L, i, J_ANGULAR_DAMPING)), h));
        } else {
            V3 axis = rot(fqa, v3(0.0f, 0.0f, 1.0f));
            float k = dot(axis, mv(isum, axis));
            stf(w, jw(L, i, J_AXIAL_MASS), k > 0.0f ? 1.0f / k : 0.0f);
            st3(w, jw(L, i, J_ROTATION_AXIS), axis);
            Q rel = qinv_mul(fqa, fqb);
            V3 px, py;
            hinge_perps(fqa, rel, &px, &py);
            st3(w, jw(L, i, J_PERP_X), px);
            st3(w, jw(L, i, J_PERP_Y), py);
            stsoft(w, jw(L, i, J_SPRING_SOFTNESS), make_soft(ldf(w, jw(L, i, J_HERTZ)), ldf(w, jw(L, i, J_DAMPING_RATIO)), h));
        }
    }
}

/* b3_apply_impulse (08:184-192) on staged velocities. */
B3D_FN void apply_impulse(const Lane& L, int b, float m, M3 i, V3 r, V3 p, float s) {
    if (!is_dyn_flag(L, b)) return;
    set_vlin(L, b, madd(vlin(L, b), s * m, p));
    set_vang(L, b, add(vang(L, b), mv(i, scale(cross(r, p), s))));
}

/* b3_warm_start over contacts (08:194-232, 293-313). */
B3D_FN void warm_start_contacts(const Lane& L) {
    int cc = ldi(L.w, H_CONTACT_COUNT);
    const uint32_t* w = L.w;
    for (int c = 0; c < cc; c++) {
        int a = ldi(w, cw(L, c, C_BODY_A)), b = ldi(w, cw(L, c, C_BODY_B));
        int pc = ldi(w, cw(L, c, C_POINT_COUNT));
        float ma = ldf(w, cw(L, c, C_INV_MASS_A)), mb = ldf(w, cw(L, c, C_INV_MASS_B));
        M3 ia = ldm3(w, cw(L, c, C_INV_I_A)), ib = ldm3(w, cw(L, c, C_INV_I_B));
        V3 n = ld3(w, cw(L, c, C_NORMAL));
        for (int p = 0; p < pc; p++) {
            V3 P = scale(n, ldf(w, pw(L, c, p, P_NORMAL_IMPULSE)));
            apply_impulse(L, a, ma, ia, ld3(w, pw(L, c, p, P_R_A)), P, -1.0f);
            apply_impulse(L, b, mb, ib, ld3(w, pw(L, c, p, P_R_B)), P, 1.0f);
        }
        V3 f = add(scale(ld3(w, cw(L, c, C_TANGENT1)), ldf(w, cw(L, c, C_FRICTION_IMPULSE))),
            scale(ld3(w, cw(L, c, C_TANGENT2)), ldf(w, cw(L, c, C_FRICTION_IMPULSE + 1))));
        apply_impulse(L, a, ma, ia, ld3(w, cw(L, c, C_CENTER_A)), f, -1.0f);
        apply_impulse(L, b, mb, ib, ld3(w, cw(L, c, C_CENTER_B)), f, 1.0f);
        V3 tr = add(scale(n, ldf(w, cw(L, c, C_TWIST_IMPULSE))), ld3(w, cw(L, c, C_ROLLING_IMPULSE)));
        if (is_dyn_flag(L, a)) set_vang(L, a, sub(vang(L, a), mv(ia, tr)));
        if (is_dyn_flag(L, b)) set_vang(L, b, add(vang(L, b), mv(ib, tr)));
    }
}

/* b3_warm_start_joints (06:204-239). */
B3D_FN void warm_start_joints(const Lane& L) {
    int nj = clampi(ldi(L.w, H_JOINT_COUNT), 0, L.g.max_j);
    const uint32_t* w = L.w;
    for (int i = 0; i < nj; i++) {
        int a = ldi(w, jw(L, i, J_BODY_A)), b = ldi(w, jw(L, i, J_BODY_B));
        V3 ra = rot(ldq(w, bw(L, a, B_DELTA_ROT)), ld3(w, jw(L, i, J_FRAME_P_A)));
        V3 rb = rot(ldq(w, bw(L, b, B_DELTA_ROT)), ld3(w, jw(L, i, J_FRAME_P_B)));
        V3 lin = ld3(w, jw(L, i, J_LINEAR_IMPULSE));
        V3 ang = ld3(w, jw(L, i, J_ANGULAR_IMPULSE));
        if (ldi(w, jw(L, i, J_TYPE)) == kJointRevolute) {
            float axial = ldf(w, jw(L, i, J_SPRING_IMPULSE)) + ldf(w, jw(L, i, J_MOTOR_IMPULSE))
                + ldf(w, jw(L, i, J_LOWER_IMPULSE)) - ldf(w, jw(L, i, J_UPPER_IMPULSE));
            ang = add(scale(ld3(w, jw(L, i, J_PERP_X)), ldf(w, jw(L, i, J_PERP_IMPULSE))),
                scale(ld3(w, jw(L, i, J_PERP_Y)), ldf(w, jw(L, i, J_PERP_IMPULSE + 1))));
            ang = madd(ang, axial, ld3(w, jw(L, i, J_ROTATION_AXIS)));
        }
        if (is_dyn_flag(L, a)) {
            set_vlin(L, a, msub(vlin(L, a), ldf(w, jw(L, i, J_INV_MASS_A)), lin));
            set_vang(L, a, sub(vang(L, a), mv(ldm3(w, jw(L, i, J_INV_I_A)), add(cross(ra, lin), ang))));
        }
        if (is_dyn_flag(L, b)) {
            set_vlin(L, b, madd(vlin(L, b), ldf(w, jw(L, i, J_INV_MASS_B)), lin));
            set_vang(L, b, add(vang(L, b), mv(ldm3(w, jw(L, i, J_INV_I_B)), add(cross(rb, lin), ang))));
        }
    }
}

/* Rolling resistance (07_packed.inl:24-45). */
B3D_FN void solve_rolling(V3 t1, V3 t2, float rolling, float total_n, M3 ia, M3 ib, V3* impulse, V3* wa, V3* wb) {
    if (rolling <= 0.0f) return;
    M3 isum = madd3(ia, ib);
    M2 k;
    k.cx.x = dot(t1, mv(isum, t1));
    k.cy.y = dot(t2, mv(isum, t2));
    k.cx.y = dot(t1, mv(isum, t2));
    k.cy.x = k.cx.y;
    V3 wr = sub(*wb, *wa);
    V2 rhs;
    rhs.x = dot(wr, t1);
    rhs.y = dot(wr, t2);
    V2 d = mv2(inv2(k), rhs);
    V3 next = sub(*impulse, add(scale(t1, d.x), scale(t2, d.y)));
    float limit = rolling * total_n;
    float l2 = len2(next);
    if (l2 > limit * limit && l2 > 0.0f) next = scale(next, rsqrt_scale(limit, l2));
    V3 delta = sub(next, *impulse);
    *impulse = next;
    *wa = sub(*wa, mv(ia, delta));
    *wb = add(*wb, mv(ib, delta));
}

/* One contact, b3_solve_one_contact (08:315-413): soft normal rows, then in
 * the relax pass twist friction, 2-D friction at the anchor and rolling. */
B3D_FN void solve_contact(const Lane& L, int c, float inv_h, float contact_speed, int use_bias) {
    uint32_t* w = L.w;
    int a = ldi(w, cw(L, c, C_BODY_A)), b = ldi(w, cw(L, c, C_BODY_B));
    int pc = ldi(w, cw(L, c, C_POINT_COUNT));
    V3 va = vlin(L, a), wa = vang(L, a), vb = vlin(L, b), wb = vang(L, b);
    Q dqa = ldq(w, bw(L, a, B_DELTA_ROT)), dqb = ldq(w, bw(L, b, B_DELTA_ROT));
    V3 dp = sub(ld3(w, bw(L, b, B_DELTA_POS)), ld3(w, bw(L, a, B_DELTA_POS)));
    V3 n = ld3(w, cw(L, c, C_NORMAL));
    float ma = ldf(w, cw(L, c, C_INV_MASS_A)), mb = ldf(w, cw(L, c, C_INV_MASS_B));
    M3 ia = ldm3(w, cw(L, c, C_INV_I_A)), ib = ldm3(w, cw(L, c, C_INV_I_B));
    Soft soft = ldsoft(w, cw(L, c, C_SOFTNESS));
    float total_n = 0.0f;
    float twist_lim = 0.0f;
    for (int p = 0; p < pc; p++) {
        V3 ra = ld3(w, pw(L, c, p, P_R_A)), rb = ld3(w, pw(L, c, p, P_R_B));
        V3 ds = add(dp, sub(rot(dqb, rb), rot(dqa, ra)));
        float sep = dot(ds, n) + ldf(w, pw(L, c, p, P_BASE_SEP));
        float vbias = 0.0f, mscale = 1.0f, iscale = 0.0f;
        if (sep > 0.0f) {
            vbias = sep * inv_h;
        } else if (use_bias) {
            vbias = maxf(soft.mass_scale * soft.bias_rate * sep, -contact_speed);
            mscale = soft.mass_scale;
            iscale = soft.impulse_scale;
        }
        V3 vra = add(va, cross(wa, ra));
        V3 vrb = add(vb, cross(wb, rb));
        float vn = dot(sub(vrb, vra), n);
        float old = ldf(w, pw(L, c, p, P_NORMAL_IMPULSE));
        float dimp = -ldf(w, pw(L, c, p, P_NORMAL_MASS)) * (mscale * vn + vbias) - iscale * old;
        float nimp = maxf(old + dimp, 0.0f);
        dimp = nimp - old;
        stf(w, pw(L, c, p, P_NORMAL_IMPULSE), nimp);
        stf(w, pw(L, c, p, P_TOTAL_NORMAL), ldf(w, pw(L, c, p, P_TOTAL_NORMAL)) + nimp);
        total_n += nimp;
        twist_lim += ldf(w, pw(L, c, p, P_LEVER)) * nimp;
        V3 P = scale(n, dimp);
        va = msub(va, ma, P);
        wa = sub(wa, mv(ia, cross(ra, P)));
        vb = madd(vb, mb, P);
        wb = add(wb, mv(ib, cross(rb, P)));
    }
    if (!use_bias) {
        float friction = ldf(w, cw(L, c, C_FRICTION));
        float twist_s = dot(n, sub(wb, wa));
        float max_t = friction * twist_lim;
        float dtw = -ldf(w, cw(L, c, C_TWIST_MASS)) * twist_s;
        float old_t = ldf(w, cw(L, c, C_TWIST_IMPULSE));
        float new_t = clampf(old_t + dtw, -max_t, max_t);
        stf(w, cw(L, c, C_TWIST_IMPULSE), new_t);
        dtw = new_t - old_t;
        wa = sub(wa, mv(ia, scale(n, dtw)));
        wb = add(wb, mv(ib, scale(n, dtw)));

        V3 t1 = ld3(w, cw(L, c, C_TANGENT1)), t2 = ld3(w, cw(L, c, C_TANGENT2));
        V3 ra = ld3(w, cw(L, c, C_CENTER_A)), rb = ld3(w, cw(L, c, C_CENTER_B));
        V3 vra = add(va, cross(wa, ra));
        V3 vrb = add(vb, cross(wb, rb));
        V3 vr = sub(vrb, vra);
        V2 vt;
        vt.x = dot(vr, t1);
        vt.y = dot(vr, t2);
        M2 tm;
        tm.cx.x = ldf(w, cw(L, c, C_TANGENT_MASS));
        tm.cx.y = ldf(w, cw(L, c, C_TANGENT_MASS + 1));
        tm.cy.x = ldf(w, cw(L, c, C_TANGENT_MASS + 2));
        tm.cy.y = ldf(w, cw(L, c, C_TANGENT_MASS + 3));
        V2 tmv = mv2(tm, vt);
        V2 fi_old;
        fi_old.x = ldf(w, cw(L, c, C_FRICTION_IMPULSE));
        fi_old.y = ldf(w, cw(L, c, C_FRICTION_IMPULSE + 1));
        V2 ni;
        ni.x = fi_old.x - tmv.x;
        ni.y = fi_old.y - tmv.y;
        float max_f = friction * total_n;
        float fl2 = ni.x * ni.x + ni.y * ni.y;
        if (fl2 > max_f * max_f && fl2 > 0.0f) {
            float sc = rsqrt_scale(max_f, fl2);
            ni.x *= sc;
            ni.y *= sc;
        }
        V2 df;
        df.x = ni.x - fi_old.x;
        df.y = ni.y - fi_old.y;
        stf(w, cw(L, c, C_FRICTION_IMPULSE), ni.x);
        stf(w, cw(L, c, C_FRICTION_IMPULSE + 1), ni.y);
        V3 P = add(scale(t1, df.x), scale(t2, df.y));
        va = msub(va, ma, P);
        wa = sub(wa, mv(ia, cross(ra, P)));
        vb = madd(vb, mb, P);
        wb = add(wb, mv(ib, cross(rb, P)));
        float rolling = ldf(w, cw(L, c, C_ROLLING));
        if (rolling > 0.0f) {
            V3 ri = ld3(w, cw(L, c, C_ROLLING_IMPULSE));
            solve_rolling(t1, t2, rolling, total_n, ia, ib, &ri, &wa, &wb);
            st3(w, cw(L, c, C_ROLLING_IMPULSE), ri);
        }
    }
    if (is_dyn_flag(L, a)) {
        set_vlin(L, a, va);
        set_vang(L, a, wa);
    }
    if (is_dyn_flag(L, b)) {
        set_vlin(L, b, vb);
        set_vang(L, b, wb);
    }
}

/* b3_apply_restitution (08:439-480). */
B3D_FN void apply_restitution(const Lane& L, float threshold) {
    uint32_t* w = L.w;
    int cc = ldi(w, H_CONTACT_COUNT);
    for (int c = 0; c < cc; c++) {
        float e = ldf(w, cw(L, c, C_RESTITUTION));
        if (e == 0.0f) continue;
        int a = ldi(w, cw(L, c, C_BODY_A)), b = ldi(w, cw(L, c, C_BODY_B));
        int pc = ldi(w, cw(L, c, C_POINT_COUNT));
        V3 va = vlin(L, a), wa = vang(L, a), vb = vlin(L, b), wb = vang(L, b);
        V3 n = ld3(w, cw(L, c, C_NORMAL));
        float ma = ldf(w, cw(L, c, C_INV_MASS_A)), mb = ldf(w, cw(L, c, C_INV_MASS_B));
        M3 ia = ldm3(w, cw(L, c, C_INV_I_A)), ib = ldm3(w, cw(L, c, C_INV_I_B));
        for (int p = 0; p < pc; p++) {
            float rv = ldf(w, pw(L, c, p, P_REL_VEL));
            if (rv > -threshold || ldf(w, pw(L, c, p, P_TOTAL_NORMAL)) == 0.0f) continue;
            V3 ra = ld3(w, pw(L, c, p, P_R_A)), rb = ld3(w, pw(L, c, p, P_R_B));
            V3 vra = add(va, cross(wa, ra));
            V3 vrb = add(vb, cross(wb, rb));
            float vn = dot(sub(vrb, vra), n);
            float old = ldf(w, pw(L, c, p, P_NORMAL_IMPULSE));
            float imp = -ldf(w, pw(L, c, p, P_NORMAL_MASS)) * (vn + e * rv);
            float nimp = maxf(old + imp, 0.0f);
            imp = nimp - old;
            stf(w, pw(L, c, p, P_NORMAL_IMPULSE), nimp);
            V3 P = scale(n, imp);
            va = msub(va, ma, P);
            wa = sub(wa, mv(ia, cross(ra, P)));
            vb = madd(vb, mb, P);
            wb = add(wb, mv(ib, cross(rb, P)));
        }
        if (is_dyn_flag(L, a)) {
            set_vlin(L, a, va);
            set_vang(L, a, wa);
        }
        if (is_dyn_flag(L, b)) {
            set_vlin(L, b, vb);
            set_vang(L, b, wb);
        }
    }
}

/* Point constraint rows shared by weld and revolute (06:241-282). */
B3D_FN M3 point_k(float ma, float mb, M3 ia, M3 ib, V3 ra, V3 rb) {
    float msum = ma + mb;
    M3 k;
    k.cx = v3(msum, 0.0f, 0.0f);
    k.cy = v3(0.0f, msum, 0.0f);
    k.cz = v3(0.0f, 0.0f, msum);
    k.cx = sub(k.cx, cross(ra, mv(ia, v3(0.0f, ra.z, -ra.y))));
    k.cy = sub(k.cy, cross(ra, mv(ia, v3(-ra.z, 0.0f, ra.x))));
    k.cz = sub(k.cz, cross(ra, mv(ia, v3(ra.y, -ra.x, 0.0f))));
    k.cx = sub(k.cx, cross(rb, mv(ib, v3(0.0f, rb.z, -rb.y))));
    k.cy = sub(k.cy, cross(rb, mv(ib, v3(-rb.z, 0.0f, rb.x))));
    k.cz = sub(k.cz, cross(rb, mv(ib, v3(rb.y, -rb.x, 0.0f))));
    return k;
}

struct JointBodies {
    int a, b;
    float ma, mb;
    M3 ia, ib;
    Q dqa, dqb;   /* delta rotations */
    V3 dpa, dpb;  /* delta positions */
};

B3D_FN void solve_point(const Lane& L, int j, const JointBodies& jb, V3* va, V3* wa, V3* vb, V3* wb,
        Soft soft, int use_bias) {
    uint32_t* w = L.w;
    V3 ra = rot(jb.dqa, ld3(w, jw(L, j, J_FRAME_P_A)));
    V3 rb = rot(jb.dqb, ld3(w, jw(L, j, J_FRAME_P_B)));
    V3 cdot = sub(add(*vb, cross(*wb, rb)), add(*va, cross(*wa, ra)));
    V3 bias = zero3();
    float mscale = 1.0f, iscale = 0.0f;
    if (use_bias) {
        V3 sep = add(add(sub(jb.dpb, jb.dpa), sub(rb, ra)), ld3(w, jw(L, j, J_DELTA_CENTER)));
        bias = scale(sep, soft.bias_rate);
        mscale = soft.mass_scale;
        iscale = soft.impulse_scale;
    }
    V3 bsol = solve3(point_k(jb.ma, jb.mb, jb.ia, jb.ib, ra, rb), add(cdot, bias));
    V3 lin_old = ld3(w, jw(L, j, J_LINEAR_IMPULSE));
    V3 impulse = msub(scale(bsol, -mscale), iscale, lin_old);
    st3(w, jw(L, j, J_LINEAR_IMPULSE), add(lin_old, impulse));
    *va = msub(*va, jb.ma, impulse);
    *wa = sub(*wa, mv(jb.ia, cross(ra, impulse)));
    *vb = madd(*vb, jb.mb, impulse);
    *wb = add(*wb, mv(jb.ib, cross(rb, impulse)));
}

/* b3_solve_weld (06:285-332). */
B3D_FN void solve_weld(const Lane& L, int j, const JointBodies& jb, int use_bias) {
    uint32_t* w = L.w;
    V3 va = vlin(L, jb.a), wa = vang(L, jb.a), vb = vlin(L, jb.b), wb = vang(L, jb.b);
    Q qa = qmul(jb.dqa, ldq(w, jw(L, j, J_FRAME_Q_A)));
    Q qb = qmul(jb.dqb, ldq(w, jw(L, j, J_FRAME_Q_B)));
    if (qdot(qa, qb) < 0.0f) qb = qneg(qb);
    Q rel = qinv_mul(qa, qb);
    float ang_hz = ldf(w, jw(L, j, J_ANGULAR_HERTZ));
    if (!ldi(w, jw(L, j, J_FIXED_ROTATION))) {
        V3 bias = zero3();
        float mscale = 1.0f, iscale = 0.0f;
        if (use_bias || ang_hz > 0.0f) {
            Q s = rel;
            if (rel.s < 0.0f) s = qneg(rel);
            Q diff = q4(-s.v.x, -s.v.y, -s.v.z, 1.0f - s.s);
            V3 cv = neg(rot(qa, scale(qmul(diff, qconj(s)).v, 2.0f)));
            Soft as = ldsoft(w, jw(L, j, J_ANGULAR_SPRING));
            bias = scale(cv, as.bias_rate);
            mscale = as.mass_scale;
            iscale = as.impulse_scale;
        }
        V3 cdot = sub(wb, wa);
        V3 ang_old = ld3(w, jw(L, j, J_ANGULAR_IMPULSE));
        V3 impulse = msub(scale(mv(ldm3(w, jw(L, j, J_ANGULAR_MASS)), add(cdot, bias)), -mscale), iscale, ang_old);
        st3(w, jw(L, j, J_ANGULAR_IMPULSE), add(ang_old, impulse));
        wa = sub(wa, mv(jb.ia, impulse));
        wb = add(wb, mv(jb.ib, impulse));
    }
    int lin_bias = use_bias || ldf(w, jw(L, j, J_LINEAR_HERTZ)) > 0.0f;
    solve_point(L, j, jb, &va, &wa, &vb, &wb, ldsoft(w, jw(L, j, J_LINEAR_SPRING)), lin_bias);
    if (is_dyn_flag(L, jb.a)) {
        set_vlin(L, jb.a, va);
        set_vang(L, jb.a, wa);
    }
    if (is_dyn_flag(L, jb.b)) {
        set_vlin(L, jb.b, vb);
        set_vang(L, jb.b, wb);
    }
}

/* One clamped one-sided limit row (06:419-433). */
B3D_FN float limit_impulse(float c, float cdot, float inv_h, int use_bias, Soft soft, float axial_mass, float old) {
    float bias = 0.0f, mscale = 1.0f, iscale = 0.0f;
    if (c > 0.0f) {
        bias = c * inv_h;
    } else if (use_bias) {
        bias = soft.bias_rate * c;
        mscale = soft.mass_scale;
        iscale = soft.impulse_scale;
    }
    float dimp = -mscale * axial_mass * (cdot + bias) - iscale * old;
    return maxf(old + dimp, 0.0f);
}

/* b3_solve_revolute (06:436-642): spring, motor, lower and upper limit,
 * two perpendicular angular rows, then the point rows. */
B3D_FN void solve_revolute(const Lane& L, int j, const JointBodies& jb, float h, float inv_h, int use_bias) {
    uint32_t* w = L.w;
    V3 va = vlin(L, jb.a), wa = vang(L, jb.a), vb = vlin(L, jb.b), wb = vang(L, jb.b);
    Q qa = qmul(jb.dqa, ldq(w, jw(L, j, J_FRAME_Q_A)));
    Q qb = qmul(jb.dqb, ldq(w, jw(L, j, J_FRAME_Q_B)));
    if (qdot(qa, qb) < 0.0f) qb = qneg(qb);
    Q rel = qinv_mul(qa, qb);
    V3 axis = ld3(w, jw(L, j, J_ROTATION_AXIS));
    int fixed = ldi(w, jw(L, j, J_FIXED_ROTATION));
    int en_spring = ldi(w, jw(L, j, J_ENABLE_SPRING));
    int en_motor = ldi(w, jw(L, j, J_ENABLE_MOTOR));
    int en_limit = ldi(w, jw(L, j, J_ENABLE_LIMIT));
    float axial_mass = ldf(w, jw(L, j, J_AXIAL_MASS));
    float max_torque = ldf(w, jw(L, j, J_MAX_MOTOR_TORQUE));
    V3 ia_ax = zero3(), ib_ax = zero3();
    float tw = 0.0f;
    if (!fixed) {
        ia_ax = mv(jb.ia, axis);
        ib_ax = mv(jb.ib, axis);
    }
    if ((en_spring || en_limit || en_motor) && !fixed) tw = twist(rel);
    if (en_spring && !fixed) {
        Soft ss = ldsoft(w, jw(L, j, J_SPRING_SOFTNESS));
        float c = tw - ldf(w, jw(L, j, J_TARGET_ANGLE));
        float bias = ss.bias_rate * c;
        float cdot = dot(sub(wb, wa), axis);
        float old = ldf(w, jw(L, j, J_SPRING_IMPULSE));
        float dimp = -ss.mass_scale * axial_mass * (cdot + bias) - ss.impulse_scale * old;
        float nimp = old + dimp;
        if (max_torque > 0.0f) {
            float maxp = max_torque * h;
            nimp = clampf(nimp, -maxp, maxp);
        }
        dimp = nimp - old;
        stf(w, jw(L, j, J_SPRING_IMPULSE), nimp);
        wa = msub(wa, dimp, ia_ax);
        wb = madd(wb, dimp, ib_ax);
    }
    if (en_motor && !fixed) {
        float speed = ldf(w, jw(L, j, J_MOTOR_SPEED));
        int blocked = 0;
        if (en_limit) {
            if (tw >= ldf(w, jw(L, j, J_UPPER_ANGLE)) - 0.01f && speed > 0.0f) blocked = 1;
            if (tw <= ldf(w, jw(L, j, J_LOWER_ANGLE)) + 0.01f && speed < 0.0f) blocked = 1;
        }
        if (blocked) {
            stf(w, jw(L, j, J_MOTOR_IMPULSE), 0.0f);
        } else {
            float old = ldf(w, jw(L, j, J_MOTOR_IMPULSE));
            float cdot = dot(sub(wb, wa), axis) - speed;
            float dimp = -axial_mass * cdot;
            float nimp = old + dimp;
            float maxp = max_torque * h;
            nimp = clampf(nimp, -maxp, maxp);
            dimp = nimp - old;
            stf(w, jw(L, j, J_MOTOR_IMPULSE), nimp);
            wa = msub(wa, dimp, ia_ax);
            wb = madd(wb, dimp, ib_ax);
        }
    }
    if (en_limit && !fixed) {
        Soft soft = ldsoft(w, jw(L, j, J_SOFTNESS));
        float old = ldf(w, jw(L, j, J_LOWER_IMPULSE));
        float lo = limit_impulse(tw - ldf(w, jw(L, j, J_LOWER_ANGLE)), dot(sub(wb, wa), axis), inv_h,
            use_bias, soft, axial_mass, old);
        stf(w, jw(L, j, J_LOWER_IMPULSE), lo);
        float dimp = lo - old;
        wa = msub(wa, dimp, ia_ax);
        wb = madd(wb, dimp, ib_ax);
        old = ldf(w, jw(L, j, J_UPPER_IMPULSE));
        float up = limit_impulse(ldf(w, jw(L, j, J_UPPER_ANGLE)) - tw, dot(sub(wa, wb), axis), inv_h,
            use_bias, soft, axial_mass, old);
        stf(w, jw(L, j, J_UPPER_IMPULSE), up);
        dimp = up - old;
        wa = madd(wa, dimp, ia_ax);
        wb = msub(wb, dimp, ib_ax);
    }
    if (!fixed) {
        V2 bias;
        bias.x = 0.0f;
        bias.y = 0.0f;
        float mscale = 1.0f, iscale = 0.0f;
        if (use_bias) {
            Soft soft = ldsoft(w, jw(L, j, J_SOFTNESS));
            bias.x = soft.bias_rate * rel.v.x;
            bias.y = soft.bias_rate * rel.v.y;
            mscale = soft.mass_scale;
            iscale = soft.impulse_scale;
        }
        V3 px, py;
        hinge_perps(qa, rel, &px, &py);
        st3(w, jw(L, j, J_PERP_X), px);
        st3(w, jw(L, j, J_PERP_Y), py);
        M3 isum = madd3(jb.ia, jb.ib);
        M2 kang;
        kang.cx.x = dot(px, mv(isum, px));
        kang.cy.y = dot(py, mv(isum, py));
        kang.cx.y = dot(px, mv(isum, py));
        kang.cy.x = kang.cx.y;
        V3 wrel = sub(wb, wa);
        V2 rhs;
        rhs.x = dot(wrel, px) + bias.x;
        rhs.y = dot(wrel, py) + bias.y;
        V2 sol = solve2(kang, rhs);
        V2 old;
        old.x = ldf(w, jw(L, j, J_PERP_IMPULSE));
        old.y = ldf(w, jw(L, j, J_PERP_IMPULSE + 1));
        V2 dimp;
        dimp.x = -mscale * sol.x - iscale * old.x;
        dimp.y = -mscale * sol.y - iscale * old.y;
        stf(w, jw(L, j, J_PERP_IMPULSE), old.x + dimp.x);
        stf(w, jw(L, j, J_PERP_IMPULSE + 1), old.y + dimp.y);
        V3 ang = add(scale(px, dimp.x), scale(py, dimp.y));
        wa = sub(wa, mv(jb.ia, ang));
        wb = add(wb, mv(jb.ib, ang));
    }
    solve_point(L, j, jb, &va, &wa, &vb, &wb, ldsoft(w, jw(L, j, J_SOFTNESS)), use_bias);
    if (is_dyn_flag(L, jb.a)) {
        set_vlin(L, jb.a, va);
        set_vang(L, jb.a, wa);
    }
    if (is_dyn_flag(L, jb.b)) {
        set_vlin(L, jb.b, vb);
        set_vang(L, jb.b, wb);
    }
}

/* b3_solve_joints_global (07_packed.inl:48-81): sweeps in joint order. */
B3D_FN void solve_joints(const Lane& L, float h, float inv_h, int use_bias) {
    uint32_t* w = L.w;
    int nj = clampi(ldi(w, H_JOINT_COUNT), 0, L.g.max_j);
    int iters = use_bias ? kJointIters : kRelaxIters;
    for (int it = 0; it < iters; it++) {
        for (int j = 0; j < nj; j++) {
            JointBodies jb;
            jb.a = ldi(w, jw(L, j, J_BODY_A));
            jb.b = ldi(w, jw(L, j, J_BODY_B));
            jb.ma = ldf(w, jw(L, j, J_INV_MASS_A));
            jb.mb = ldf(w, jw(L, j, J_INV_MASS_B));
            jb.ia = ldm3(w, jw(L, j, J_INV_I_A));
            jb.ib = ldm3(w, jw(L, j, J_INV_I_B));
            jb.dqa = ldq(w, bw(L, jb.a, B_DELTA_ROT));
            jb.dqb = ldq(w, bw(L, jb.b, B_DELTA_ROT));
            jb.dpa = ld3(w, bw(L, jb.a, B_DELTA_POS));
            jb.dpb = ld3(w, bw(L, jb.b, B_DELTA_POS));
            if (ldi(w, jw(L, j, J_TYPE)) == kJointWeld) solve_weld(L, j, jb, use_bias);
            else solve_revolute(L, j, jb, h, inv_h, use_bias);
        }
    }
}

/* Gravity, applied force and damping for dynamic bodies (09_step.inl:5-18, 41-53). */
B3D_FN void integrate_velocities(const Lane& L, float h) {
    uint32_t* w = L.w;
    V3 g = ld3(w, H_GRAVITY);
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        if (ldi(w, bw(L, b, B_TYPE)) != kDynamic) continue;
        float inv_mass = ldf(w, bw(L, b, B_INV_MASS));
        float ld = 1.0f / (1.0f + h * ldf(w, bw(L, b, B_LINEAR_DAMPING)));
        float ad = 1.0f / (1.0f + h * ldf(w, bw(L, b, B_ANGULAR_DAMPING)));
        float gs = inv_mass > 0.0f ? ldf(w, bw(L, b, B_GRAVITY_SCALE)) : 0.0f;
        V3 dv = add(scale(ld3(w, bw(L, b, B_FORCE)), h * inv_mass), scale(g, h * gs));
        set_vlin(L, b, madd(dv, ld, vlin(L, b)));
        V3 dw = scale(mv(ldm3(w, bw(L, b, B_INV_I_WORLD)), ld3(w, bw(L, b, B_TORQUE))), h);
        set_vang(L, b, madd(dw, ad, vang(L, b)));
    }
}

/* Axis locks, speed clamps and the substep pose update (09_step.inl:55-107). */
B3D_FN void integrate_positions(const Lane& L, float h, float inv_dt) {
    uint32_t* w = L.w;
    float max_lin = ldf(w, H_MAX_LINEAR_SPEED);
    float max_ang = kMaxRotation * inv_dt;
    float max_lin2 = max_lin * max_lin;
    float max_ang2 = max_ang * max_ang;
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        if (ldi(w, bw(L, b, B_TYPE)) == kStatic) continue;
        uint32_t flags = ldu(w, bw(L, b, B_FLAGS));
        V3 v = vlin(L, b), av = vang(L, b);
        if (flags & 0x01u) v.x = 0.0f;
        if (flags & 0x02u) v.y = 0.0f;
        if (flags & 0x04u) v.z = 0.0f;
        if (flags & 0x08u) av.x = 0.0f;
        if (flags & 0x10u) av.y = 0.0f;
        if (flags & 0x20u) av.z = 0.0f;
        float v2 = len2(v);
        if (v2 > max_lin2 && v2 > 0.0f) v = scale(v, rsqrt_scale(max_lin, v2));
        float w2 = len2(av);
        if (w2 > max_ang2 && w2 > 0.0f) av = scale(av, rsqrt_scale(max_ang, w2));
        set_vlin(L, b, v);
        set_vang(L, b, av);
        st3(w, bw(L, b, B_DELTA_POS), madd(ld3(w, bw(L, b, B_DELTA_POS)), h, v));
        stq(w, bw(L, b, B_DELTA_ROT), qintegrate(ldq(w, bw(L, b, B_DELTA_ROT)), scale(av, h)));
    }
}

/* Commit the accumulated deltas and clear forces (09_step.inl:109-130). */
B3D_FN void finalize(const Lane& L) {
    uint32_t* w = L.w;
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        int type = ldi(w, bw(L, b, B_TYPE));
        if (type == kStatic) continue;
        V3 center = add(ld3(w, bw(L, b, B_CENTER)), ld3(w, bw(L, b, B_DELTA_POS)));
        Q r = qnorm(qmul(ldq(w, bw(L, b, B_DELTA_ROT)), ldq(w, bw(L, b, B_ROTATION))));
        st3(w, bw(L, b, B_CENTER), center);
        stq(w, bw(L, b, B_ROTATION), r);
        st3(w, bw(L, b, B_POSITION), sub(center, rot(r, ld3(w, bw(L, b, B_LOCAL_CENTER)))));
        st3(w, bw(L, b, B_DELTA_POS), zero3());
        stq(w, bw(L, b, B_DELTA_ROT), qid());
        st3(w, bw(L, b, B_FORCE), zero3());
        st3(w, bw(L, b, B_TORQUE), zero3());
        if (type == kDynamic) stm3(w, bw(L, b, B_INV_I_WORLD), world_inv_i(r, ld3(w, bw(L, b, B_INV_INERTIA))));
    }
}

/* One world's b3_step (09_step.inl:148-264, default configuration).  The
 * caller has staged velocities with vel_load and stores them afterwards. */
B3D_FN void step_world(const Lane& L, float dt, int substeps) {
    if (!(dt > 0.0f)) return;
    int subs = substeps < 1 ? 1 : substeps;
    float h = dt / (float)subs;
    float inv_dt = 1.0f / dt;
    float inv_h = (float)subs * inv_dt;
    float hertz = minf(ldf(L.w, H_CONTACT_HERTZ), 0.25f * inv_h);
    float damping = ldf(L.w, H_CONTACT_DAMPING);
    Soft cs = make_soft(hertz, damping, h);
    Soft ss = make_soft(2.0f * hertz, 0.5f * damping, h);
    float contact_speed = ldf(L.w, H_CONTACT_SPEED);
    float rest_threshold = ldf(L.w, H_RESTITUTION_THRESHOLD);

    collide_and_prepare(L, cs, ss);
    prepare_joints(L, h);
    warm_start_contacts(L);
    warm_start_joints(L);
    int cc = ldi(L.w, H_CONTACT_COUNT);
    for (int s = 0; s < subs; s++) {
        integrate_velocities(L, h);
        for (int c = 0; c < cc; c++) solve_contact(L, c, inv_h, contact_speed, 1);
        solve_joints(L, h, inv_h, 1);
        integrate_positions(L, h, inv_dt);
        for (int c = 0; c < cc; c++) solve_contact(L, c, inv_h, contact_speed, 0);
        solve_joints(L, h, inv_h, 0);
        apply_restitution(L, rest_threshold);
    }
    finalize(L);
}

}  // namespace b3d

#endif
