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
 * Body velocities stay in `vel` for the whole step (body_prepass fills the
 * rows, vel_store writes them back), everything else is read and written
 * in place.
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

constexpr int kLanes = B3D_LANES;
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
              O_FRICTION_IMPULSE = 11, O_TWIST_IMPULSE = 13, O_ROLLING_IMPULSE = 14, O_KEY = 17, kOldWords = 18;

/* Per-step shape record in scratch: world pose, size and owning body, the
 * collision filter and the material, written once per step by the shape
 * pass so that the pair loop reads one record per shape and never follows
 * a body index.  The padded bounds go to LDS when they fit (or to the
 * scratch bounds area). */
constexpr int SS_P = 0, SS_RADIUS = 3, SS_Q = 4, SS_HALF = 8, SS_TYPE = 11, SS_CENTER = 12, SS_BODY = 15,
              SS_CATEGORY = 16, SS_MASK = 18, SS_BFLAGS = 20, SS_FRICTION = 21, SS_RESTITUTION = 22,
              SS_ROLLING = 23, kShapeRows = 6;
constexpr int kBodyStatic = 1, kBodyDynamic = 2;   /* SS_BFLAGS bits */
/* Loops over bodies, shapes and contacts run in chunks, every load of a
 * chunk issued before any of its results is used. */
constexpr int kChunk = 4;
constexpr int kShapeChunk = 4;
/* Per-step body records: the velocity increments of 09_step.inl:5-18 (all
 * their inputs are fixed for the step) and the damping factors (BS_*); the
 * delta pose, which the step keeps here and commits in finalize, and the
 * body kind (type and axis-lock flags) (BD_*). */
constexpr int BS_DV = 0, BS_LD = 3, BS_DW = 4, BS_AD = 7, kBodyRows = 2;
constexpr int BD_DP = 0, BD_KIND = 3, BD_DQ = 4, kDeltaRows = 2;
constexpr int kKindDynamic = 1 << 8, kKindStatic = 1 << 9;  /* BD_KIND bits; low byte = lock flags */
/* BD_KIND bits: the world's delta pose, force or torque words at the start
 * of the step are not already the bits finalize writes (zero, identity), so
 * finalize must write them (the writes are skipped when they would not
 * change a bit). */
constexpr int kKindClearDelta = 1 << 10, kKindClearForce = 1 << 11;
/* Per-contact scratch head, written by the pair loop for prepare_contacts:
 * bodies (a | b << 16), point count and facts about the pair
 * (pc | flags << 8). */
constexpr int CH_AB = 0, CH_INFO = 1, kContactScr = 2;
constexpr int CF_DYN_A = 1, CF_DYN_B = 2, CF_STATIC = 4, CF_RESTITUTION = 8, CF_ROLLING = 16;
/* Packed records only: the body is static and its delta pose is exactly zero
 * and the identity for the whole step (nothing moves a static body), so the
 * sweeps use those values instead of loading its delta record. */
constexpr int CF_FIXED_A = 32, CF_FIXED_B = 64;
/* Per-lane step flags (scratch word scr_flags, written by the pair loop):
 * some contact of the world has restitution. */
constexpr int kLaneRestitution = 1;

/* Packed contact records.  Past the per-lane words, a tile's scratch is
 * quad rows: 64 slots of 4 words (1 KB).  Contact c of a lane owns kCRows
 * rows in slot `rank`, the number of the tile's stepping lanes below it that
 * also have a contact c; the kPRows rows of its point p use the rank among
 * the lanes whose contact c has a point p.  Every loop over contacts visits
 * c in the same order in all lanes, so the lanes that touch a row in one
 * access touch one contiguous span of it, and a quad is one 16-byte access.
 * The record holds everything the solver sweeps, warm start and restitution
 * read (prepare_contacts writes it once per step), and the impulses they
 * update, which go back to the world's contact rows at the end of the step.
 * Word k of a record is component k % 4 of quad row k / 4. */
constexpr int kRowWords = kLanes * 4;
constexpr int R_AB = 0, R_INFO = 1, R_FRICTION = 2, R_TWIST_MASS = 3,   /* row 0: head */
              R_N = 4, R_ROLLING = 7,                                   /* row 1 */
              R_MA = 8, R_IA = 9,                                       /* rows 2-4: body a (10 words) */
              R_IB_ZYZ = 18, R_MB = 20, R_IB = 21,                      /* rows 4-6: body b (10 words) */
              R_T1 = 28, R_TM_XX = 31, R_CA = 32, R_TM_XY = 35, R_CB = 36, R_TM_YY = 39,
              R_FI = 40, R_TWIST = 42, R_RESTITUTION = 43,              /* row 10 */
              R_ROLL = 44,                                              /* row 11 */
              R_REL_VEL = 48,                                           /* row 12: restitution only */
              R_BASE_SEP = 52,                                          /* row 13: point base separations */
              R_NI = 56, R_TN = 57,                                     /* rows 14-15: point p at +2p */
              kCRows = 16;
/* Point records: anchors, normal mass and twist lever.  A contact's
 * per-point values that change during the step (the accumulated impulses)
 * sit in whole rows of the contact record, so that each update writes full
 * quads. */
constexpr int PR_RA = 0, PR_NMASS = 3, PR_RB = 4, PR_LEVER = 7, kPRows = 2;
/* Joint record in scratch: the joint-connection key, the head written by
 * prepare_joints (bodies a | b << 16 and JF_* flags), then everything that
 * depends only on the bodies' delta poses (recomputed after every position
 * update): twist angle, the hinge perpendicular rows and the relative
 * rotation's x, y, the point anchors and separation, the weld's angular
 * error; the inverse of the point rows' 3x3 mass matrix (JS_PKI) and the
 * perpendicular rows' 2x2 mass matrix with its reciprocal determinant
 * (JS_KXX, JS_KXY, JS_KYY, JS_KINV; NaN when singular).  Last, fixed for
 * the step: the hinge axis through each body's inverse inertia (JS_IAX,
 * JS_IBX). */
constexpr int JS_KEY = 0, JS_AB = 1, JS_INFO = 2, JS_TW = 3, JS_RELX = 4, JS_RELY = 5, JS_PX = 6, JS_PY = 9,
              JS_RA = 12, JS_RB = 15, JS_PSEP = 18, JS_CV = 21, JS_PKI = 24, JS_KXX = 33, JS_KXY = 34, JS_KYY = 35,
              JS_KINV = 36, JS_IAX = 37, JS_IBX = 40, kJointScr = 43;
constexpr int JF_WELD = 1, JF_FIXED = 2, JF_SPRING = 4, JF_MOTOR = 8, JF_LIMIT = 16, JF_DYN_A = 32, JF_DYN_B = 64;

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
    int scr_old, scr_sep, scr_joint, scr_bounds, scr_cand, scr_flags;
    int scr_words;        /* per-lane scratch words (a multiple of 4) */
    int q_ct, q_pt;       /* first quad row of the contact and point records */
    int q_body, q_delta, q_shape;  /* first quad row of the body, delta-pose and shape records */
    int tile_scr_words;   /* scratch words per tile: 64 lanes' words, then the quad rows */
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
    g->scr_old = 0;
    g->scr_sep = g->scr_old + g->max_c * kOldWords;
    g->scr_joint = g->scr_sep + g->max_c * kContactScr;
    g->scr_bounds = g->scr_joint + g->max_j * kJointScr;
    g->scr_cand = g->scr_bounds + g->max_s * 6;
    g->scr_flags = g->scr_cand + g->max_s * (g->max_s - 1);
    g->scr_words = (g->scr_flags + 1 + 3) & ~3;
    g->q_ct = 0;
    g->q_pt = g->q_ct + g->max_c * kCRows;
    g->q_body = g->q_pt + g->max_c * kMaxManifold * kPRows;
    g->q_delta = g->q_body + g->max_b * kBodyRows;
    g->q_shape = g->q_delta + g->max_b * kDeltaRows;
    int qrows = g->q_shape + g->max_s * kShapeRows;
    g->tile_scr_words = g->scr_words * kLanes + qrows * kRowWords;
    *world_bytes = L.world_size;
    return true;
}

/* Manifolds of a tile's candidate pairs, computed by the tile's waves
 * together (small batches, where one wave per tile leaves CUs idle): the
 * lane's candidate count at word 0 (p[0], a row of the tile's 64 lanes),
 * then, past that row, one record of kStageWords words per candidate and
 * lane, lane-major (candidate t of lane l at record t * kLanes + l): the
 * manifold's kManiWords words (count, normal, then per point p_a, p_b,
 * separation, feature), the pair's shape key and its old contact (or -1),
 * and padding to 16 bytes.  A lane's record is contiguous, so the contact
 * writes, which take each lane's manifolds in its own contact order, read
 * whole records; only candidates with a manifold have one written. */
constexpr int kManiWords = 4 + 8 * kMaxManifold;
constexpr int kStageWords = kManiWords + 4;
static_assert(kStageWords % 4 == 0, "stage records are whole quads");
struct PairStage {
    uint32_t* p;     /* lane base */
    float* clip;     /* this wave's clip rows (lane base; waves < cwaves) */
    int wave, waves;
    int cwaves;      /* waves 0 .. cwaves-1 have clip rows and share the
                        narrowphase; every wave shares the rest */
    int lds_bounds;  /* the workgroup's LDS also holds wave 0's shape bounds */
};

/* Per-lane view of one world. */
struct Lane {
    uint32_t* w;    /* live tile + lane */
    uint32_t* scr;  /* scratch tile + lane */
    uint32_t* sq;   /* the tile's scratch quad rows */
    float* vel;     /* velocity rows + lane; before the velocities are
                       staged the same rows hold the clip polygons */
    int lane;
    int sslot;          /* rank among the tile's stepping lanes: the slot of
                           the body, delta-pose and shape records */
    unsigned int opts;  /* kKeepSolverFields */
    PairStage st;       /* with `staged`: the tile's waves share the narrowphase
                           (held by value, so that no pointer to a local
                           escapes and its pointers keep their memory spaces) */
    bool staged;
    bool active;        /* the lane steps its world.  Only a shared tile
                           (staged) runs idle lanes: they go through
                           every workgroup barrier with their work skipped */
    float* jl;          /* LDS joint rows + lane (shared tiles with room for
                           them, joint_rows_fit), else null */
    float* ji;          /* LDS joint impulses + lane (the one-wave step, when
                           they fit past the velocity rows: ji_fit), else null */
    Geometry g;
    /* The world's header counts, read once per step (a read of the header
     * word sits on the critical path of every phase that loops over them):
     * with `counted`, nb and nj are the clamped body and joint counts; with
     * `contacts_counted`, nc is the raw contact-count word as contact
     * generation left it.  Without the flags the accessors read the world. */
    bool counted = false;
    bool contacts_counted = false;
    int nb = 0, nj = 0, nc = 0;
};

/* Option: also write the prepared solver fields of every new contact
 * (b3_prepare_one_contact's inverse masses and inertias, softness, normal
 * and tangent masses, relative velocities, twist levers and mass, friction
 * anchors and rolling mass) to the world's contact rows.  The step itself
 * reads them from the packed records, and every step recomputes them before
 * use, so without the option those fields of a downloaded contact are
 * stale; everything else is identical.  Same value as
 * B3_ENGINE_KEEP_SOLVER_FIELDS. */
constexpr unsigned int kKeepSolverFields = 1u;

/* The lane view of world `lane` of tile `tile`, with the per-step scratch
 * of scratch tile `scr_tile` (the same by default; a tile whose lanes are
 * stepped by several workgroups gives each its own). */
B3D_FN Lane lane_view(uint32_t* live, uint32_t* scratch, float* vel_rows, const Geometry& g, int tile, int lane,
        unsigned int opts = 0, int scr_tile = -1) {
    Lane L;
    L.opts = opts;
    L.st = PairStage{};
    L.staged = false;
    L.sslot = lane;
    if (scr_tile < 0) scr_tile = tile;
    L.w = live + (size_t)tile * g.world_words * kLanes + lane;
    L.scr = scratch ? scratch + (size_t)scr_tile * g.tile_scr_words + lane : nullptr;
    L.sq = scratch ? scratch + (size_t)scr_tile * g.tile_scr_words + (size_t)g.scr_words * kLanes : nullptr;
    L.jl = nullptr;
    L.ji = nullptr;
    L.vel = vel_rows ? vel_rows + lane : nullptr;
    L.lane = lane;
    L.active = true;
    L.g = g;
    return L;
}

/* Rank of this lane among the lanes executing this point together: the slot
 * of its packed record.  Lanes run one at a time in a host build, where the
 * lane index serves. */
B3D_FN int wave_slot(const Lane& L) {
#ifdef __HIP_DEVICE_COMPILE__
    (void)L;
    uint64_t m = __ballot(1);
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
#else
    return L.lane;
#endif
}

/* Rank of this lane among its wave's stepping lanes (L.active): the slot of
 * the lane's body, delta-pose and shape records.  A shared tile computes
 * it with its idle lanes executing too. */
B3D_FN int wave_rank(const Lane& L) {
#ifdef __HIP_DEVICE_COMPILE__
    uint64_t m = __ballot(L.active);
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
#else
    return L.lane;
#endif
}

/* `v` holds in some active lane of the wave (on the host: in this lane).
 * Call where all of the tile's stepping lanes run: code that computes
 * record slots (wave_slot) must run in every lane that owns the record, so
 * a lane may only leave such code out when its whole wave does. */
B3D_FN bool wave_any(const Lane& L, bool v) {
#ifdef __HIP_DEVICE_COMPILE__
    (void)L;
    return __ballot(v) != 0;
#else
    (void)L;
    return v;
#endif
}

/* Workgroup barrier.  A host build runs one lane at a time and only counts
 * the barriers a lane passes (host_barriers), so a host test can check
 * that stepping and idle lanes of a shared tile meet the same ones. */
#ifdef __HIP_DEVICE_COMPILE__
#define B3D_BARRIER() __syncthreads()
#else
inline int host_barriers = 0;
#define B3D_BARRIER() ((void)++host_barriers)
#endif

/* Shape bounds stay in the LDS rows during contact generation when the
 * rows of kClipWords + 6 max_s words fit in this many words per lane;
 * otherwise they go to scratch. */
constexpr int kMaxLdsRows = 160;
B3D_FN bool bounds_in_lds(const Geometry& g) { return kClipWords + 6 * g.max_s <= kMaxLdsRows; }
/* Words of LDS rows per lane that one step needs. */
B3D_FN int lds_rows(const Geometry& g) {
    int v = g.max_b * kVelWords;
    int f = bounds_in_lds(g) ? kClipWords + 6 * g.max_s : kClipWords;
    return v > f ? v : f;
}

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

/* ---- packed record access (word k at quad row k / 4, component k % 4) ---- */
B3D_FN float qf(const uint32_t* r, int k) { return __builtin_bit_cast(float, r[(k >> 2) * kRowWords + (k & 3)]); }
B3D_FN uint32_t qu(const uint32_t* r, int k) { return r[(k >> 2) * kRowWords + (k & 3)]; }
B3D_FN void qsf(uint32_t* r, int k, float v) { r[(k >> 2) * kRowWords + (k & 3)] = __builtin_bit_cast(uint32_t, v); }
B3D_FN void qsu(uint32_t* r, int k, uint32_t v) { r[(k >> 2) * kRowWords + (k & 3)] = v; }
B3D_FN V3 q3(const uint32_t* r, int k) { return v3(qf(r, k), qf(r, k + 1), qf(r, k + 2)); }
B3D_FN void qs3(uint32_t* r, int k, V3 v) { qsf(r, k, v.x); qsf(r, k + 1, v.y); qsf(r, k + 2, v.z); }
B3D_FN Q qq(const uint32_t* r, int k) { return q4(qf(r, k), qf(r, k + 1), qf(r, k + 2), qf(r, k + 3)); }
B3D_FN void qsq(uint32_t* r, int k, Q q) { qs3(r, k, q.v); qsf(r, k + 3, q.s); }
B3D_FN uint64_t qu64(const uint32_t* r, int k) { return (uint64_t)qu(r, k) | ((uint64_t)qu(r, k + 1) << 32); }
/* Loads of quad records that a sweep reads once, streaming (non-temporal)
 * when S: in a large batch their next use is a whole sweep later, past what
 * the L2 keeps, so they leave the L2 to the data reused within a sweep (in
 * a small batch the records stay in the caches, and ordinary loads keep
 * them there). */
template <bool S>
B3D_FN uint32_t qus(const uint32_t* r, int k) {
#ifdef __HIP_DEVICE_COMPILE__
    if constexpr (S) return __builtin_nontemporal_load(r + (k >> 2) * kRowWords + (k & 3));
#endif
    return qu(r, k);
}
template <bool S>
B3D_FN float qfs(const uint32_t* r, int k) { return __builtin_bit_cast(float, qus<S>(r, k)); }
template <bool S>
B3D_FN V3 q3s(const uint32_t* r, int k) { return v3(qfs<S>(r, k), qfs<S>(r, k + 1), qfs<S>(r, k + 2)); }

/* ---- packed word rows (word k of a record at quad row k / 4, word row
 * k % 4 of it; slot s at column s) ---- */
B3D_FN float rf(const uint32_t* r, int k) { return __builtin_bit_cast(float, r[(k >> 2) * kRowWords + (k & 3) * kLanes]); }
B3D_FN uint32_t ru(const uint32_t* r, int k) { return r[(k >> 2) * kRowWords + (k & 3) * kLanes]; }
B3D_FN void rsf(uint32_t* r, int k, float v) { r[(k >> 2) * kRowWords + (k & 3) * kLanes] = __builtin_bit_cast(uint32_t, v); }
B3D_FN void rsu(uint32_t* r, int k, uint32_t v) { r[(k >> 2) * kRowWords + (k & 3) * kLanes] = v; }
B3D_FN V3 r3(const uint32_t* r, int k) { return v3(rf(r, k), rf(r, k + 1), rf(r, k + 2)); }
B3D_FN void rs3(uint32_t* r, int k, V3 v) { rsf(r, k, v.x); rsf(r, k + 1, v.y); rsf(r, k + 2, v.z); }
B3D_FN Q rq4(const uint32_t* r, int k) { return q4(rf(r, k), rf(r, k + 1), rf(r, k + 2), rf(r, k + 3)); }
B3D_FN void rsq(uint32_t* r, int k, Q q) { rs3(r, k, q.v); rsf(r, k + 3, q.s); }
B3D_FN uint64_t ru64(const uint32_t* r, int k) { return (uint64_t)ru(r, k) | ((uint64_t)ru(r, k + 1) << 32); }


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

B3D_FN int body_count(const Lane& L) { return L.counted ? L.nb : clampi(ldi(L.w, H_BODY_COUNT), 0, L.g.max_b); }
B3D_FN int joint_count(const Lane& L) { return L.counted ? L.nj : clampi(ldi(L.w, H_JOINT_COUNT), 0, L.g.max_j); }
/* the contact-count word, unclamped */
B3D_FN int contact_count_word(const Lane& L) { return L.contacts_counted ? L.nc : ldi(L.w, H_CONTACT_COUNT); }
/* Reads the header counts into the lane (an idle lane of a shared tile,
 * which runs no phase that reads them, keeps zeros). */
B3D_FN void count_bodies_and_joints(Lane& L) {
    if (L.active) {
        L.nb = body_count(L);
        L.nj = joint_count(L);
    }
    L.counted = true;
}
B3D_FN void count_contacts(Lane& L) {
    if (L.active) L.nc = ldi(L.w, H_CONTACT_COUNT);
    L.contacts_counted = true;
}

/* The velocity rows back to the bodies (the rows are filled by
 * body_prepass); bodies first, first + stride, ... (a shared tile's waves
 * split them). */
B3D_FN void vel_store(const Lane& L, int first = 0, int stride = 1) {
    int nb = body_count(L);
    for (int b = first; b < nb; b += stride) {
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

B3D_FN uint32_t* shape_rec(const Lane& L, int s) {
    return L.sq + (size_t)(L.g.q_shape + s * kShapeRows) * kRowWords + L.sslot;
}
B3D_FN uint32_t* old_rec(const Lane& L, int k) { return L.scr + (L.g.scr_old + k * kOldWords) * kLanes; }
B3D_FN uint32_t* chead_rec(const Lane& L, int c) { return L.scr + (L.g.scr_sep + c * kContactScr) * kLanes; }
/* Packed record of contact c and of its point p (see kCRows). */
B3D_FN uint32_t* crec(const Lane& L, int c, int slot) {
    return L.sq + (size_t)(L.g.q_ct + c * kCRows) * kRowWords + slot * 4;
}
B3D_FN uint32_t* prec(const Lane& L, int c, int p, int slot) {
    return L.sq + (size_t)(L.g.q_pt + (c * kMaxManifold + p) * kPRows) * kRowWords + slot * 4;
}
/* A contact's head: bodies, point count and CF_* flags, with its record
 * slot and, from a packed record, friction and twist mass. */
struct CHead { int a, b, pc, flags, slot; float friction, twist_mass; };
B3D_FN CHead head_of(uint32_t ab, uint32_t info) {
    CHead h;
    h.a = (int)(ab & 0xffffu);
    h.b = (int)(ab >> 16);
    h.pc = (int)(info & 0xffu);
    h.flags = (int)(info >> 8);
    h.slot = 0;
    h.friction = 0.0f;
    h.twist_mass = 0.0f;
    return h;
}
/* The head the pair loop left for prepare_contacts. */
B3D_FN CHead chead_load(const Lane& L, int c) {
    const uint32_t* hd = chead_rec(L, c);
    return head_of(ldu(hd, CH_AB), ldu(hd, CH_INFO));
}
/* The head of a packed record; call where exactly the lanes with a contact
 * c run. */
B3D_FN CHead rhead_load(const Lane& L, int c) {
    int slot = wave_slot(L);
    const uint32_t* r = crec(L, c, slot);
    CHead h = head_of(qu(r, R_AB), qu(r, R_INFO));
    h.slot = slot;
    h.friction = qf(r, R_FRICTION);
    h.twist_mass = qf(r, R_TWIST_MASS);
    return h;
}
/* The head of contact c's packed record in a known slot. */
template <bool S = false>
B3D_FN CHead rhead_at(const Lane& L, int c, int slot) {
    const uint32_t* r = crec(L, c, slot);
    CHead h = head_of(qus<S>(r, R_AB), qus<S>(r, R_INFO));
    h.slot = slot;
    h.friction = qfs<S>(r, R_FRICTION);
    h.twist_mass = qfs<S>(r, R_TWIST_MASS);
    return h;
}
/* Inverse masses and world inertias of a record's bodies: exact zeros for a
 * body that is not dynamic (08:236-241), which are therefore not stored. */
B3D_FN void rec_masses(const uint32_t* r, int flags, float* ma, M3* ia, float* mb, M3* ib) {
    *ma = 0.0f;
    *mb = 0.0f;
    *ia = m3zero();
    *ib = m3zero();
    if (flags & CF_DYN_A) {
        *ma = qf(r, R_MA);
        ia->cx = q3(r, R_IA);
        ia->cy = q3(r, R_IA + 3);
        ia->cz = q3(r, R_IA + 6);
    }
    if (flags & CF_DYN_B) {
        *mb = qf(r, R_MB);
        ib->cx = q3(r, R_IB);
        ib->cy = q3(r, R_IB + 3);
        ib->cz = v3(qf(r, R_IB + 6), qf(r, R_IB_ZYZ), qf(r, R_IB_ZYZ + 1));
    }
}
B3D_FN void rec_store_masses(uint32_t* r, int flags, float ma, M3 ia, float mb, M3 ib) {
    if (flags & CF_DYN_A) {
        qsf(r, R_MA, ma);
        qs3(r, R_IA, ia.cx);
        qs3(r, R_IA + 3, ia.cy);
        qs3(r, R_IA + 6, ia.cz);
    }
    if (flags & CF_DYN_B) {
        qsf(r, R_MB, mb);
        qs3(r, R_IB, ib.cx);
        qs3(r, R_IB + 3, ib.cy);
        qsf(r, R_IB + 6, ib.cz.x);
        qsf(r, R_IB_ZYZ, ib.cz.y);
        qsf(r, R_IB_ZYZ + 1, ib.cz.z);
    }
}
B3D_FN uint32_t* joint_rec(const Lane& L, int j) { return L.scr + (L.g.scr_joint + j * kJointScr) * kLanes; }
/* Per-lane rows of LDS words (stride kLanes): a joint's LDS row (JL) or
 * impulse row (JI), word k at q[k * kLanes]. */
B3D_FN float jlf(const float* q, int k) { return q[k * kLanes]; }
B3D_FN V3 jl3(const float* q, int k) { return v3(q[k * kLanes], q[(k + 1) * kLanes], q[(k + 2) * kLanes]); }
B3D_FN M3 jlm3(const float* q, int k) { M3 m; m.cx = jl3(q, k); m.cy = jl3(q, k + 3); m.cz = jl3(q, k + 6); return m; }
B3D_FN Soft jlsoft(const float* q, int k) {
    Soft s;
    s.bias_rate = q[k * kLanes];
    s.mass_scale = q[(k + 1) * kLanes];
    s.impulse_scale = q[(k + 2) * kLanes];
    return s;
}
B3D_FN void jlsf(float* q, int k, float v) { q[k * kLanes] = v; }
B3D_FN void jls3(float* q, int k, V3 v) { jlsf(q, k, v.x); jlsf(q, k + 1, v.y); jlsf(q, k + 2, v.z); }
B3D_FN void jlsm3(float* q, int k, M3 m) { jls3(q, k, m.cx); jls3(q, k + 3, m.cy); jls3(q, k + 6, m.cz); }
B3D_FN void jlssoft(float* q, int k, Soft s) { jlsf(q, k, s.bias_rate); jlsf(q, k + 1, s.mass_scale); jlsf(q, k + 2, s.impulse_scale); }

/* Joint impulses in LDS (the one-wave step, JI): per joint kJIWords words
 * past the velocity rows, the accumulated impulses that the solves read and
 * write.  The joint warm start stages them from the joint's words, which
 * joint_impulse_writeback updates once at the end of the step; the solves'
 * other fields come from the world and the scratch record as without it.
 * A weld's angular impulse shares the revolute's perpendicular and spring
 * words. */
constexpr int JI_LIN = 0, JI_PERP = 3, JI_SPRING = 5, JI_MOTOR = 6, JI_LOWER = 7, JI_UPPER = 8, JI_ANG = 3,
              kJIWords = 9;
B3D_FN int ji_word(const Geometry& g) { return g.max_b * kVelWords; }
/* The impulses fit within the one-wave step's LDS rows (kMaxLdsRows words
 * per lane: four waves per CU). */
B3D_FN bool ji_fit(const Geometry& g) { return g.max_j > 0 && ji_word(g) + kJIWords * g.max_j <= kMaxLdsRows; }
B3D_FN int ji_lds_rows(const Geometry& g) {
    int r = ji_word(g) + kJIWords * g.max_j;
    return r > lds_rows(g) ? r : lds_rows(g);
}
B3D_FN float* ji_rec(const Lane& L, int j) { return L.ji + j * kJIWords * kLanes; }
/* The LDS word of a joint's impulse word. */
B3D_FN int ji_of(int world_word) {
    return world_word == J_LINEAR_IMPULSE ? JI_LIN
         : world_word == J_ANGULAR_IMPULSE ? JI_ANG
         : world_word == J_PERP_IMPULSE ? JI_PERP
         : world_word == J_PERP_IMPULSE + 1 ? JI_PERP + 1
         : world_word == J_SPRING_IMPULSE ? JI_SPRING
         : world_word == J_MOTOR_IMPULSE ? JI_MOTOR
         : world_word == J_LOWER_IMPULSE ? JI_LOWER : JI_UPPER;
}
/* An accumulated impulse of joint j as a solve reads it (JI: the LDS row). */
template <bool JI>
B3D_FN float jimp_ld(const Lane& L, int j, int world_word) {
    if constexpr (JI) return ji_rec(L, j)[ji_of(world_word) * kLanes];
    else return ldf(L.w, jw(L, j, world_word));
}
template <bool JI>
B3D_FN V3 jimp_ld3(const Lane& L, int j, int world_word) {
    if constexpr (JI) {
        const float* q = ji_rec(L, j) + ji_of(world_word) * kLanes;
        return v3(q[0], q[kLanes], q[2 * kLanes]);
    } else {
        return ld3(L.w, jw(L, j, world_word));
    }
}

B3D_FN uint32_t* body_rec(const Lane& L, int b) {
    return L.sq + (size_t)(L.g.q_body + b * kBodyRows) * kRowWords + L.sslot;
}
B3D_FN uint32_t* delta_rec(const Lane& L, int b) {
    return L.sq + (size_t)(L.g.q_delta + b * kDeltaRows) * kRowWords + L.sslot;
}
B3D_FN uint32_t pair_key(int a, int b) { return a < b ? ((uint32_t)a << 16) | (uint32_t)b : ((uint32_t)b << 16) | (uint32_t)a; }
/* Joint keys the pair loop keeps in registers (the rest it loads). */
constexpr int kJointKeyRegs = 8;

/* Shape pass: world pose, padded bounds and owning-body facts of every
 * shape (b3_shape_aabb plus the 0.02 pad, 08_contacts.inl:109-114).  The
 * bounds go to `bounds` (lane-strided lo.xyz, hi.xyz per shape), the rest to
 * the shape records.  Shapes are done in chunks, body poses requested for a
 * whole chunk at once. */
B3D_FN void shape_pass(const Lane& L, int ns, float* bounds, int first = 0, int stride = 1) {
    V3 pad = v3(kSpeculative, kSpeculative, kSpeculative);
    /* chunks of kShapeChunk shapes first, first + stride, ... (a shared
     * tile's waves split them); the next chunk's body indices are in
     * flight while a chunk is posed */
    const int step = stride * kShapeChunk;
    int bn[kShapeChunk];
#pragma unroll
    for (int k = 0; k < kShapeChunk; k++)
        if (first * kShapeChunk + k < ns) bn[k] = ldi(L.w, sw(L, first * kShapeChunk + k, S_BODY));
    for (int s0 = first * kShapeChunk; s0 < ns; s0 += step) {
        int b[kShapeChunk];
#pragma unroll
        for (int k = 0; k < kShapeChunk; k++) {
            b[k] = bn[k];
            if (s0 + step + k < ns) bn[k] = ldi(L.w, sw(L, s0 + step + k, S_BODY));
        }
        V3 bpos[kShapeChunk], center[kShapeChunk];
        Q brot[kShapeChunk];
        int btype[kShapeChunk];
        Posed P[kShapeChunk];
        uint32_t filt[kShapeChunk][4];
        float mat[kShapeChunk][3];
#pragma unroll
        for (int k = 0; k < kShapeChunk; k++) {
            int s = s0 + k;
            if (s >= ns) continue;
#pragma unroll
            for (int f = 0; f < 4; f++) filt[k][f] = ldu(L.w, sw(L, s, S_CATEGORY + f));
            mat[k][0] = ldf(L.w, sw(L, s, S_FRICTION));
            mat[k][1] = ldf(L.w, sw(L, s, S_RESTITUTION));
            mat[k][2] = ldf(L.w, sw(L, s, S_ROLLING));
            bpos[k] = ld3(L.w, bw(L, b[k], B_POSITION));
            brot[k] = ldq(L.w, bw(L, b[k], B_ROTATION));
            center[k] = ld3(L.w, bw(L, b[k], B_CENTER));
            btype[k] = ldi(L.w, bw(L, b[k], B_TYPE));
            P[k].type = ldi(L.w, sw(L, s, S_TYPE));
            P[k].p = ld3(L.w, sw(L, s, S_LOCAL_POS));
            P[k].q = ldq(L.w, sw(L, s, S_LOCAL_ROT));
            P[k].radius = ldf(L.w, sw(L, s, S_RADIUS));
            P[k].half = ld3(L.w, sw(L, s, S_HALF));
        }
#pragma unroll
        for (int k = 0; k < kShapeChunk; k++) {
            int s = s0 + k;
            if (s >= ns) continue;
            /* b3_shape_pos / b3_shape_rot (04_world.inl:293-299) */
            P[k].p = xf(bpos[k], brot[k], P[k].p);
            P[k].q = qmul(brot[k], P[k].q);
            V3 lo, hi;
            shape_aabb(P[k], &lo, &hi);
            uint32_t* r = shape_rec(L, s);
            rs3(r, SS_P, P[k].p);
            rsf(r, SS_RADIUS, P[k].radius);
            rsq(r, SS_Q, P[k].q);
            rs3(r, SS_HALF, P[k].half);
            rsu(r, SS_TYPE, (uint32_t)P[k].type);
            rs3(r, SS_CENTER, center[k]);
            rsu(r, SS_BODY, (uint32_t)b[k]);
#pragma unroll
            for (int f = 0; f < 4; f++) rsu(r, SS_CATEGORY + f, filt[k][f]);
            rsu(r, SS_BFLAGS, (uint32_t)((btype[k] == kStatic ? kBodyStatic : 0) | (btype[k] == kDynamic ? kBodyDynamic : 0)));
            rsf(r, SS_FRICTION, mat[k][0]);
            rsf(r, SS_RESTITUTION, mat[k][1]);
            rsf(r, SS_ROLLING, mat[k][2]);
            float* bd = bounds + s * 6 * kLanes;
            V3 l = sub(lo, pad), h = add(hi, pad);
            bd[0] = l.x;
            bd[kLanes] = l.y;
            bd[2 * kLanes] = l.z;
            bd[3 * kLanes] = h.x;
            bd[4 * kLanes] = h.y;
            bd[5 * kLanes] = h.z;
        }
    }
}

B3D_FN Posed posed_from(const uint32_t* r) {
    Posed P;
    P.p = r3(r, SS_P);
    P.q = rq4(r, SS_Q);
    P.radius = rf(r, SS_RADIUS);
    P.half = r3(r, SS_HALF);
    P.type = (int)ru(r, SS_TYPE);
    return P;
}

/* Shape pair (i, j) as one ordered 32-bit key (shape ids are below 2^16). */
B3D_FN uint32_t shape_key(int i, int j) { return ((uint32_t)i << 16) | (uint32_t)j; }

/* The contacts' warm-start data go to the old-cache scratch
 * (08_contacts.inl:65-91) in two parts, old_keys (which also tells whether
 * their shape pairs are strictly increasing, as every list the step itself
 * writes is) and old_warm_copy. */
/* With a shared narrowphase the workgroup's LDS also holds the old contacts'
 * keys, after wave 0's clip rows and shape bounds, for the candidate search
 * to merge against. */
B3D_FN bool lds_old_keys(const Lane& L) { return L.staged && L.st.lds_bounds; }
/* A shared tile's LDS, per lane: wave 0's rows (clip rows, then shape
 * bounds, later velocities) and the helpers' clip rows, then, past both
 * and past the shape bounds, the old contact keys, the bound-overlap masks
 * of the shape pairs and the candidates' hit bits, which the waves use
 * while colliding in their clip rows. */
/* The waves of a shared tile that collide: wave 0 in its own rows, waves
 * 1 .. kClipWaves-1 in clip rows of their own past them, and further waves
 * in wave 0's rows past its clip rows, as many as fit: those rows hold the
 * shape bounds until the candidates are listed (a barrier before the
 * narrowphase) and nothing else until the velocities are staged after
 * contact generation. */
constexpr int kClipWaves = 4;
B3D_FN int clip_waves(const Geometry& g, int waves) {
    int n = kClipWaves + (lds_rows(g) - kClipWords) / kClipWords;
    return n < waves ? n : waves;
}
/* First word (per lane) of colliding wave `wave`'s clip rows. */
B3D_FN int clip_row_word(const Geometry& g, int wave) {
    if (wave == 0) return 0;
    if (wave < kClipWaves) return lds_rows(g) + (wave - 1) * kClipWords;
    return (1 + wave - kClipWaves) * kClipWords;
}
B3D_FN int shared_keys_word(const Geometry& g) {
    int a = lds_rows(g) + (kClipWaves - 1) * kClipWords, b = kClipWords + 6 * g.max_s;
    return a > b ? a : b;
}
B3D_FN int shared_masks_word(const Geometry& g) { return shared_keys_word(g) + g.max_c; }
B3D_FN int shared_hits_word(const Geometry& g) { return shared_masks_word(g) + 2 * g.max_s; }
B3D_FN float* old_key_rows(const Lane& L) { return L.vel + shared_keys_word(L.g) * kLanes; }
B3D_FN uint32_t old_key(const Lane& L, int k) {
    if (lds_old_keys(L)) return __builtin_bit_cast(uint32_t, old_key_rows(L)[k * kLanes]);
    return ldu(old_rec(L, k), O_KEY);
}

/* The old contacts' shape pairs and keys (to the old-cache records and,
 * in a shared tile, to LDS); returns whether the pairs are strictly
 * increasing.  The heads of kKeyChunk contacts load together. */
constexpr int kKeyChunk = 8;
B3D_FN int old_keys(const Lane& L, int old_n) {
    int sorted = 1;
    uint32_t prev = 0;
    for (int k0 = 0; k0 < old_n; k0 += kKeyChunk) {
        int sa[kKeyChunk], sb[kKeyChunk];
#pragma unroll
        for (int q = 0; q < kKeyChunk; q++) {
            int k = k0 + q;
            if (k >= old_n) continue;
            sa[q] = ldi(L.w, cw(L, k, C_SHAPE_A));
            sb[q] = ldi(L.w, cw(L, k, C_SHAPE_B));
        }
#pragma unroll
        for (int q = 0; q < kKeyChunk; q++) {
            int k = k0 + q;
            if (k >= old_n) continue;
            uint32_t* o = old_rec(L, k);
            uint32_t key = shape_key(sa[q], sb[q]);
            if (k > 0 && !(prev < key && (uint32_t)sa[q] < 65536u && (uint32_t)sb[q] < 65536u)) sorted = 0;
            prev = key;
            sti(o, O_SHAPE_A, sa[q]);
            sti(o, O_SHAPE_B, sb[q]);
            sti(o, O_KEY, (int)key);
            if (lds_old_keys(L)) old_key_rows(L)[k * kLanes] = __builtin_bit_cast(float, key);
        }
    }
    return sorted;
}
/* The old contacts' warm-start data (point count, features, impulses) to
 * their old-cache records: chunks first, first + stride, ... (a shared
 * tile's waves split them). */
B3D_FN void old_warm_copy(const Lane& L, int old_n, int first = 0, int stride = 1) {
    for (int k0 = first * kChunk; k0 < old_n; k0 += stride * kChunk) {
        int pc[kChunk];
        uint32_t feat[kChunk][kMaxManifold];
        float ni[kChunk][kMaxManifold], fx[kChunk], fy[kChunk], tw[kChunk];
        V3 roll[kChunk];
#pragma unroll
        for (int q = 0; q < kChunk; q++) {
            int k = k0 + q;
            if (k >= old_n) continue;
            pc[q] = clampi(ldi(L.w, cw(L, k, C_POINT_COUNT)), 0, kMaxManifold);
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                feat[q][p] = ldu(L.w, pw(L, k, p, P_FEATURE));
                ni[q][p] = ldf(L.w, pw(L, k, p, P_NORMAL_IMPULSE));
            }
            fx[q] = ldf(L.w, cw(L, k, C_FRICTION_IMPULSE));
            fy[q] = ldf(L.w, cw(L, k, C_FRICTION_IMPULSE + 1));
            tw[q] = ldf(L.w, cw(L, k, C_TWIST_IMPULSE));
            roll[q] = ld3(L.w, cw(L, k, C_ROLLING_IMPULSE));
        }
#pragma unroll
        for (int q = 0; q < kChunk; q++) {
            int k = k0 + q;
            if (k >= old_n) continue;
            uint32_t* o = old_rec(L, k);
            sti(o, O_POINT_COUNT, pc[q]);
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= pc[q]) continue;
                sti(o, O_FEATURE + p, (int)feat[q][p]);
                stf(o, O_NORMAL_IMPULSE + p, ni[q][p]);
            }
            stf(o, O_FRICTION_IMPULSE, fx[q]);
            stf(o, O_FRICTION_IMPULSE + 1, fy[q]);
            stf(o, O_TWIST_IMPULSE, tw[q]);
            st3(o, O_ROLLING_IMPULSE, roll[q]);
        }
    }
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

/* A shape's padded bounds from its LDS rows (lower x y z, upper x y z), and
 * their overlap test: all six words load together and the comparisons
 * combine without branches (a chain of && would wait on each load in
 * turn). */
struct Box6 { float lx, ly, lz, hx, hy, hz; };
B3D_FN Box6 box_load(const float* b) {
    return Box6{b[0], b[kLanes], b[2 * kLanes], b[3 * kLanes], b[4 * kLanes], b[5 * kLanes]};
}
B3D_FN bool box_overlap(const Box6& a, const Box6& b) {
    return (a.lx <= b.hx) & (a.hx >= b.lx) & (a.ly <= b.hy) & (a.hy >= b.ly) & (a.lz <= b.hz) & (a.hz >= b.lz);
}

/* The pair loop's view of one shape (its per-step shape record). */
struct PairShape {
    Posed P;
    V3 center;
    int body, bflags;
    uint64_t cat, mask;
    float friction, restitution, rolling;
};
B3D_FN void pshape_load(const Lane& L, int s, PairShape* d) {
    const uint32_t* r = shape_rec(L, s);
    d->P = posed_from(r);
    d->center = r3(r, SS_CENTER);
    d->body = (int)ru(r, SS_BODY);
    d->bflags = (int)ru(r, SS_BFLAGS);
    d->cat = ru64(r, SS_CATEGORY);
    d->mask = ru64(r, SS_MASK);
    d->friction = rf(r, SS_FRICTION);
    d->restitution = rf(r, SS_RESTITUTION);
    d->rolling = rf(r, SS_ROLLING);
}

/* One old contact's warm-start data (the reference's B3Warm). */
struct OldWarm {
    uint32_t key;
    int pc;
    uint32_t feat[kMaxManifold];
    float ni[kMaxManifold];
    V2 fi;
    float twist;
    V3 roll;
};
B3D_FN void old_load(const Lane& L, int k, OldWarm* o) {
    const uint32_t* r = old_rec(L, k);
    o->key = ldu(r, O_KEY);
    o->pc = ldi(r, O_POINT_COUNT);
#pragma unroll
    for (int q = 0; q < kMaxManifold; q++) {
        o->feat[q] = ldu(r, O_FEATURE + q);
        o->ni[q] = ldf(r, O_NORMAL_IMPULSE + q);
    }
    o->fi.x = ldf(r, O_FRICTION_IMPULSE);
    o->fi.y = ldf(r, O_FRICTION_IMPULSE + 1);
    o->twist = ldf(r, O_TWIST_IMPULSE);
    o->roll = ld3(r, O_ROLLING_IMPULSE);
}
/* The impulses of an old contact for the points whose feature matches
 * (08_contacts.inl:154-170; the last matching old point wins). */
B3D_FN void warm_apply(const OldWarm& o, NewContact* nc) {
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++) {
        if (p >= nc->count) continue;
#pragma unroll
        for (int q = 0; q < kMaxManifold; q++)
            if (q < o.pc && nc->feature[p] == o.feat[q]) nc->ni[p] = o.ni[q];
    }
    nc->fi = o.fi;
    nc->twist = o.twist;
    nc->roll = o.roll;
}

/* The ordered pair loop of b3_find_contacts (08_contacts.inl:115-172):
 * broadphase filter (08:45-62), narrowphase, overflow accounting, warm
 * start and b3_contact_from_mani (08:5-39).  `bounds` holds the padded
 * shape bounds (LDS or scratch).
 *
 * First the bounds test of every pair i < j lists the overlapping pairs in
 * (i, j) order in scratch, each with the index of the old contact of the
 * same shape pair when the old list is strictly sorted (every list the step
 * writes is; the two sorted lists are merged).  Then the list is walked
 * with the next pair's shape records and old contact in flight while the
 * current pair is tested and collided. */
/* Lane `lane`'s record of candidate t, in 16-byte quads (aligned: the
 * stage's tiles are whole rows of 64 words, its records 40 words). */
struct alignas(16) Quad { uint32_t x, y, z, w; };
B3D_FN Quad* mani_rec(const PairStage& S, int lane, int t) {
    return reinterpret_cast<Quad*>(S.p - lane + kLanes + ((size_t)t * kLanes + lane) * kStageWords);
}
/* The record of a candidate with a manifold, as whole quads (the points past
 * its count hold whatever the collision left there and go unused). */
B3D_FN void mani_store(const PairStage& S, int lane, int t, const Mani& m, uint32_t key, int match) {
    uint32_t w[kStageWords];
    w[0] = (uint32_t)m.count;
    w[1] = __builtin_bit_cast(uint32_t, m.normal.x);
    w[2] = __builtin_bit_cast(uint32_t, m.normal.y);
    w[3] = __builtin_bit_cast(uint32_t, m.normal.z);
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++) {
        w[4 + 8 * p] = __builtin_bit_cast(uint32_t, m.p_a[p].x);
        w[5 + 8 * p] = __builtin_bit_cast(uint32_t, m.p_a[p].y);
        w[6 + 8 * p] = __builtin_bit_cast(uint32_t, m.p_a[p].z);
        w[7 + 8 * p] = __builtin_bit_cast(uint32_t, m.p_b[p].x);
        w[8 + 8 * p] = __builtin_bit_cast(uint32_t, m.p_b[p].y);
        w[9 + 8 * p] = __builtin_bit_cast(uint32_t, m.p_b[p].z);
        w[10 + 8 * p] = __builtin_bit_cast(uint32_t, m.sep[p]);
        w[11 + 8 * p] = m.feature[p];
    }
    w[kManiWords] = key;
    w[kManiWords + 1] = (uint32_t)match;
    w[kManiWords + 2] = 0u;
    w[kManiWords + 3] = 0u;
    Quad* r = mani_rec(S, lane, t);
#pragma unroll
    for (int q = 0; q < kStageWords / 4; q++) r[q] = Quad{w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]};
}
B3D_FN void mani_load(const PairStage& S, int lane, int t, Mani* m, uint32_t* key, int* match) {
    const Quad* r = mani_rec(S, lane, t);
    uint32_t w[kStageWords];
#pragma unroll
    for (int q = 0; q < kStageWords / 4; q++) {
        Quad v = r[q];
        w[4 * q] = v.x;
        w[4 * q + 1] = v.y;
        w[4 * q + 2] = v.z;
        w[4 * q + 3] = v.w;
    }
    m->count = (int)w[0];
    m->normal = v3(__builtin_bit_cast(float, w[1]), __builtin_bit_cast(float, w[2]), __builtin_bit_cast(float, w[3]));
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++) {
        m->p_a[p] = v3(__builtin_bit_cast(float, w[4 + 8 * p]), __builtin_bit_cast(float, w[5 + 8 * p]),
            __builtin_bit_cast(float, w[6 + 8 * p]));
        m->p_b[p] = v3(__builtin_bit_cast(float, w[7 + 8 * p]), __builtin_bit_cast(float, w[8 + 8 * p]),
            __builtin_bit_cast(float, w[9 + 8 * p]));
        m->sep[p] = __builtin_bit_cast(float, w[10 + 8 * p]);
        m->feature[p] = w[11 + 8 * p];
    }
    *key = w[kManiWords];
    *match = (int)w[kManiWords + 1];
}

/* Whether candidate pair (A, B) is filtered out before the narrowphase
 * (08:127-139): one body, both static, category / mask, or joined by a
 * joint that does not collide its bodies. */
B3D_FN bool pair_skipped(const Lane& L, const PairShape& A, const PairShape& B, const uint32_t* jkey, int nj) {
    uint32_t bkey = pair_key(A.body, B.body);
    int joined = 0;
#pragma unroll
    for (int k = 0; k < kJointKeyRegs; k++) joined |= jkey[k] == bkey;
    for (int k = kJointKeyRegs; k < nj; k++) joined |= ldu(joint_rec(L, k), JS_KEY) == bkey;
    return A.body == B.body || (A.bflags & B.bflags & kBodyStatic) || (A.cat & B.mask) == 0
        || (B.cat & A.mask) == 0 || joined;
}

/* Which candidates of a shared tile produced a manifold: one bit per
 * candidate, then a restitution flag and whether the old contacts were
 * sorted. */
B3D_FN int hit_words(const Geometry& g) { return (g.max_s * (g.max_s - 1) / 2 + 31) / 32; }
B3D_FN float* hit_rows(const Lane& L) { return L.vel + shared_hits_word(L.g) * kLanes; }
/* Words of a shared tile's LDS per lane. */
B3D_FN int shared_lds_words(const Geometry& g) { return shared_hits_word(g) + hit_words(g) + 2; }
B3D_FN void lds_or(float* p, uint32_t bits) {
#ifdef __HIP_DEVICE_COMPILE__
    atomicOr(reinterpret_cast<unsigned int*>(p), bits);
#else
    *p = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, *p) | bits);
#endif
}

/* Bound-overlap masks of a shared tile's shape pairs (bit j of row i:
 * shapes i < j overlap; at most 64 shapes), rows i = wave, wave + waves. */
B3D_FN uint64_t overlap_mask(const Lane& L, int i) {
    const float* r = L.vel + (shared_masks_word(L.g) + 2 * i) * kLanes;
    return (uint64_t)__builtin_bit_cast(uint32_t, r[0]) | ((uint64_t)__builtin_bit_cast(uint32_t, r[kLanes]) << 32);
}
B3D_FN void overlap_rows(const Lane& L, const float* bounds, int ns, const PairStage& S) {
    for (int i = S.wave; i < ns; i += S.waves) {
        Box6 bi = box_load(bounds + i * 6 * kLanes);
        uint64_t m = 0;
        /* four shapes' bounds in flight at a time */
        for (int j0 = i + 1; j0 < ns; j0 += 4) {
            Box6 bj[4];
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (j0 + k < ns) bj[k] = box_load(bounds + (j0 + k) * 6 * kLanes);
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (j0 + k < ns && box_overlap(bi, bj[k])) m |= 1ull << (j0 + k);
        }
        float* r = L.vel + (shared_masks_word(L.g) + 2 * i) * kLanes;
        r[0] = __builtin_bit_cast(float, (uint32_t)m);
        r[kLanes] = __builtin_bit_cast(float, (uint32_t)(m >> 32));
    }
}
/* Candidate t of the masks in (i, j) order; row and acc (candidates in
 * rows before it) carry the walk over increasing t. */
B3D_FN void mask_candidate(const Lane& L, int t, int* row, int* acc, int* i, int* j) {
    uint64_t m = overlap_mask(L, *row);
    int c = __builtin_popcountll(m);
    while (t >= *acc + c) {
        *acc += c;
        *row += 1;
        m = overlap_mask(L, *row);
        c = __builtin_popcountll(m);
    }
    for (int k = t - *acc; k > 0; k--) m &= m - 1;
    *i = *row;
    *j = __builtin_ctzll(m);
}
/* The old contact whose shape key equals key (the first at or past it in
 * the sorted keys: the merge of the sequential search), or -1. */
B3D_FN int old_match(const Lane& L, int old_n, uint32_t key) {
    int lo = 0, hi = old_n;
    while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (old_key(L, mid) < key) lo = mid + 1;
        else hi = mid;
    }
    return lo < old_n && old_key(L, lo) == key ? lo : -1;
}

/* Whether a shared tile's waves also split the candidate search through
 * the overlap masks; with few shapes wave 0 lists the candidates alone,
 * which costs less than the masks' extra barrier.  The shared launches are
 * specialised on it (template argument Masks of step_world, find_pairs and
 * pair_helper), as the masks' code costs the other variant registers. */
constexpr int kMaskMinShapes = 12;
B3D_FN bool shared_masks(const Geometry& g) { return g.max_s >= kMaskMinShapes && g.max_s <= 64; }
B3D_FN int mask_candidates(const Lane& L, int ns) {
    int n = 0;
    for (int i = 0; i < ns; i++) n += __builtin_popcountll(overlap_mask(L, i));
    return n;
}
/* Candidate t's shapes and old-contact match: from the masks (with a
 * search of the old keys), or from wave 0's list. */
B3D_FN void share_candidate(const Lane& L, bool masks, int t, int* row, int* acc, int* i, int* j, int* match,
        int old_n, int sorted) {
    const uint32_t* cand = L.scr + L.g.scr_cand * kLanes;
    if (masks) {
        mask_candidate(L, t, row, acc, i, j);
        *match = sorted ? old_match(L, old_n, shape_key(*i, *j)) : -1;
    } else {
        uint32_t key = ldu(cand, 2 * t);
        *match = ldi(cand, 2 * t + 1);
        *i = (int)(key >> 16);
        *j = (int)(key & 0xffffu);
    }
}

/* This wave's share of the tile's narrowphase: candidates t = wave, wave +
 * cwaves, ..., each collided (empty when filtered) into the stage; the next
 * share's shapes are in flight during a collision.  Waves past cwaves have
 * no clip rows and no share. */
B3D_FN void pair_share(const Lane& L, const PairStage& S, bool masks, int ncand, int nj, int old_n, int sorted) {
    if (S.wave >= S.cwaves) return;
    uint32_t jkey[kJointKeyRegs];
#pragma unroll
    for (int k = 0; k < kJointKeyRegs; k++) jkey[k] = k < nj ? ldu(joint_rec(L, k), JS_KEY) : 0xffffffffu;
    int row = 0, acc = 0, i = 0, j = 0, in = 0, jn = 0, match = -1, matchn = -1;
    PairShape A, B, An, Bn;
    int t = S.wave;
    if (t < ncand) {
        share_candidate(L, masks, t, &row, &acc, &i, &j, &match, old_n, sorted);
        pshape_load(L, i, &A);
        pshape_load(L, j, &B);
        An = A;
        Bn = B;
    }
    for (; t < ncand; t += S.cwaves) {
        int tn = t + S.cwaves;
        if (tn < ncand) {
            share_candidate(L, masks, tn, &row, &acc, &in, &jn, &matchn, old_n, sorted);
            pshape_load(L, in, &An);
            pshape_load(L, jn, &Bn);
        }
        Mani m;
        m.count = 0;
        if (!pair_skipped(L, A, B, jkey, nj)) collide_pair(&m, A.P, B.P, S.clip);
        if (m.count > 0) {
            mani_store(S, L.lane, t, m, shape_key(i, j), match);
            lds_or(hit_rows(L) + (t >> 5) * kLanes, 1u << (t & 31));
        }
        A = An;
        B = Bn;
        i = in;
        j = jn;
        match = matchn;
    }
}

/* Contact cc of the step from candidate pair (i, j)'s manifold m: its
 * anchors and base separations, the warm start from the matching old
 * contact, the world's contact row and the head for prepare_contacts
 * (08:140-170, b3_contact_from_mani 08:5-39).  Returns the CF_* flags. */
B3D_FN int write_new_contact(const Lane& L, int cc, int i, int j, const PairShape& A, const PairShape& B,
        const Mani& m, int sorted, int match, const OldWarm& orec, int old_n) {
    NewContact nc;
    nc.count = m.count;
    nc.normal = m.normal;
    nc.t1 = perp(m.normal);
    nc.t2 = cross(nc.t1, m.normal);
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++) {
        if (p >= m.count) continue;
        nc.r_a[p] = sub(m.p_a[p], A.center);
        nc.r_b[p] = sub(m.p_b[p], B.center);
        nc.base_sep[p] = m.sep[p] - dot(sub(nc.r_b[p], nc.r_a[p]), m.normal);
        nc.feature[p] = m.feature[p];
        nc.ni[p] = 0.0f;
    }
    nc.fi = V2{0.0f, 0.0f};
    nc.twist = 0.0f;
    nc.roll = zero3();
    /* warm start from the previous step's cache: every matching old
     * pair, the last one winning (08:154-170) */
    if (sorted) {
        if (match >= 0) warm_apply(orec, &nc);
    } else {
        for (int k = 0; k < old_n; k++) {
            const uint32_t* o = old_rec(L, k);
            if (ldi(o, O_SHAPE_A) == i && ldi(o, O_SHAPE_B) == j) {
                OldWarm ow;
                old_load(L, k, &ow);
                warm_apply(ow, &nc);
            }
        }
    }
    uint32_t* w = L.w;
    sti(w, cw(L, cc, C_SHAPE_A), i);
    sti(w, cw(L, cc, C_SHAPE_B), j);
    sti(w, cw(L, cc, C_BODY_A), A.body);
    sti(w, cw(L, cc, C_BODY_B), B.body);
    sti(w, cw(L, cc, C_POINT_COUNT), nc.count);
    sti(w, cw(L, cc, C_STATIC), !((A.bflags & B.bflags) & kBodyDynamic));
    st3(w, cw(L, cc, C_NORMAL), nc.normal);
    st3(w, cw(L, cc, C_TANGENT1), nc.t1);
    st3(w, cw(L, cc, C_TANGENT2), nc.t2);
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++) {
        if (p >= nc.count) continue;
        st3(w, pw(L, cc, p, P_R_A), nc.r_a[p]);
        st3(w, pw(L, cc, p, P_R_B), nc.r_b[p]);
        stf(w, pw(L, cc, p, P_BASE_SEP), nc.base_sep[p]);
        stf(w, pw(L, cc, p, P_NORMAL_IMPULSE), nc.ni[p]);
        sti(w, pw(L, cc, p, P_FEATURE), (int)nc.feature[p]);
    }
    float restitution = A.restitution > B.restitution ? A.restitution : B.restitution;
    float rolling = maxf(A.rolling, B.rolling);
    stf(w, cw(L, cc, C_FRICTION), sqrtf(A.friction * B.friction));
    stf(w, cw(L, cc, C_RESTITUTION), restitution);
    stf(w, cw(L, cc, C_ROLLING), rolling);
    int info = (A.bflags & kBodyDynamic ? CF_DYN_A : 0) | (B.bflags & kBodyDynamic ? CF_DYN_B : 0)
        | (!((A.bflags & B.bflags) & kBodyDynamic) ? CF_STATIC : 0) | (restitution != 0.0f ? CF_RESTITUTION : 0)
        | (!(rolling <= 0.0f) ? CF_ROLLING : 0);
    uint32_t* hd = chead_rec(L, cc);
    sti(hd, CH_AB, A.body | (B.body << 16));
    sti(hd, CH_INFO, nc.count | (info << 8));
    stf(w, cw(L, cc, C_TWIST_IMPULSE), nc.twist);
    stf(w, cw(L, cc, C_FRICTION_IMPULSE), nc.fi.x);
    stf(w, cw(L, cc, C_FRICTION_IMPULSE + 1), nc.fi.y);
    st3(w, cw(L, cc, C_ROLLING_IMPULSE), nc.roll);
    return info;
}

/* This wave's share of writing the new contacts: contacts k = wave, wave +
 * waves, ..., below the lane's count of candidates with a manifold and the
 * capacity.  Contact k is the candidate holding the lane's k-th manifold,
 * as the sequential append numbers them; those past the capacity are
 * dropped (the header is wave 0's).  All lanes write contact k at once, so
 * each field's store covers one row of the tile's lanes. */
B3D_FN void append_share(const Lane& L, const PairStage& S, int ncand, int old_n, int sorted) {
    const float* hit = hit_rows(L);
    int nwords = (ncand + 31) >> 5, total = 0;
    for (int k = 0; k < nwords; k++) total += __builtin_popcount(__builtin_bit_cast(uint32_t, hit[k * kLanes]));
    int cap = total < L.g.max_c ? total : L.g.max_c;
    int acc = 0, word = 0, rest = 0;
    for (int k = S.wave; k < cap; k += S.waves) {
        /* the word holding the k-th manifold (acc: manifolds in the words
         * before it), then the bit */
        uint32_t bits = __builtin_bit_cast(uint32_t, hit[word * kLanes]);
        while (acc + __builtin_popcount(bits) <= k) {
            acc += __builtin_popcount(bits);
            word++;
            bits = __builtin_bit_cast(uint32_t, hit[word * kLanes]);
        }
        for (int r = k - acc; r > 0; r--) bits &= bits - 1;
        int t = word * 32 + __builtin_ctz(bits);
        Mani m;
        uint32_t key;
        int match;
        mani_load(S, L.lane, t, &m, &key, &match);
        int i = (int)(key >> 16), j = (int)(key & 0xffffu);
        PairShape A, B;
        pshape_load(L, i, &A);
        pshape_load(L, j, &B);
        OldWarm orec;
        if (sorted && match >= 0) old_load(L, match, &orec);
        rest |= write_new_contact(L, k, i, j, A, B, m, sorted, match, orec, old_n) & CF_RESTITUTION;
    }
    if (rest) lds_or(const_cast<float*>(hit) + hit_words(L.g) * kLanes, 1u);
}

/* A helper wave of a staged tile: waits for wave 0's candidate lists, runs
 * its share of the narrowphase, and signals.  Runs in all lanes, like wave
 * 0; its stepping lanes rank as wave 0's, so its record slots are wave
 * 0's, and its idle lanes have no candidates. */
template <bool Masks>
B3D_FN void pair_helper(const Lane& L0, const PairStage& S) {
    Lane L = L0;
    L.sslot = wave_rank(L);
    int ns = L.active ? clampi(ldi(L.w, H_SHAPE_COUNT), 0, L.g.max_s) : 0;
    int nj = L.active ? clampi(ldi(L.w, H_JOINT_COUNT), 0, L.g.max_j) : 0;
    int old_n = L.active ? clampi(ldi(L.w, H_CONTACT_COUNT), 0, L.g.max_c) : 0;
    constexpr bool masks = Masks;
    if (masks && L.active) {
        /* this wave's share of the old contacts' warm data and of the
         * shape pass (find_contacts) */
        old_warm_copy(L, old_n, S.wave, S.waves);
        shape_pass(L, ns, L.vel + kClipWords * kLanes, S.wave, S.waves);
    }
    B3D_BARRIER();                 /* the shape bounds and old keys (or wave 0's candidates) */
    int ncand;
    if (masks) {
        overlap_rows(L, L.vel + kClipWords * kLanes, ns, S);
        B3D_BARRIER();             /* the overlap masks are complete */
        ncand = mask_candidates(L, ns);
    } else {
        ncand = L.active ? ldi(S.p, 0) : 0;
    }
    int sorted = L.active ? __builtin_bit_cast(int, hit_rows(L)[(hit_words(L.g) + 1) * kLanes]) : 0;
    pair_share(L, S, masks, ncand, nj, old_n, sorted);
    B3D_BARRIER();                 /* every manifold is staged */
    append_share(L, S, ncand, old_n, sorted);
    B3D_BARRIER();                 /* every new contact is written */
}

template <bool Masks>
B3D_FN void find_pairs(const Lane& L, const float* bounds, int ns, int nj, int old_n, int sorted) {
    const Geometry& g = L.g;
    uint32_t* cand = L.scr + g.scr_cand * kLanes;
    int ncand = 0;
    bool masks = Masks && L.staged;
    if (L.staged) {
        float* hit = hit_rows(L);
        for (int k = 0; k <= hit_words(g); k++) hit[k * kLanes] = 0.0f;
        hit[(hit_words(g) + 1) * kLanes] = __builtin_bit_cast(float, sorted);
    }
    if (masks) {
        /* the tile's waves test the bound pairs, then list the candidates
         * in the same order as below */
        B3D_BARRIER();
        overlap_rows(L, bounds, ns, L.st);
        B3D_BARRIER();
        ncand = mask_candidates(L, ns);
    } else {
        /* the old keys in chunks of four, the next chunk in flight */
        int op = 0, kbase = 0;
        uint32_t kc[4], kn[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            kc[q] = sorted && q < old_n ? old_key(L, q) : 0xffffffffu;
            kn[q] = sorted && 4 + q < old_n ? old_key(L, 4 + q) : 0xffffffffu;
        }
        uint32_t okey = kc[0];
        for (int i = 0; i < ns; i++) {
            Box6 bi = box_load(bounds + i * 6 * kLanes);
            for (int j0 = i + 1; j0 < ns; j0 += 4) {
                bool ov[4];
                Box6 bj[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (j0 + k < ns) bj[k] = box_load(bounds + (j0 + k) * 6 * kLanes);
#pragma unroll
                for (int k = 0; k < 4; k++) ov[k] = j0 + k < ns && box_overlap(bi, bj[k]);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if (!ov[k]) continue;
                    uint32_t key = shape_key(i, j0 + k);
                    int match = -1;
                    if (sorted) {
                        while (op < old_n && okey < key) {
                            op++;
                            if (op - kbase == 4) {
                                kbase += 4;
#pragma unroll
                                for (int q = 0; q < 4; q++) {
                                    kc[q] = kn[q];
                                    kn[q] = kbase + 4 + q < old_n ? old_key(L, kbase + 4 + q) : 0xffffffffu;
                                }
                            }
                            int d = op - kbase;
                            okey = d == 0 ? kc[0] : (d == 1 ? kc[1] : (d == 2 ? kc[2] : kc[3]));
                        }
                        if (op < old_n && okey == key) match = op;
                    }
                    sti(cand, 2 * ncand, (int)key);
                    sti(cand, 2 * ncand + 1, match);
                    ncand++;
                }
            }
        }
        if (L.staged) {
            sti(L.st.p, 0, ncand);
            B3D_BARRIER();
        }
    }
    if (L.staged) {
        /* the tile's waves split the narrowphase, then write the new
         * contacts at the places the candidate order gives them */
        const PairStage& S = L.st;
        const float* hit = hit_rows(L);
        pair_share(L, S, masks, ncand, nj, old_n, sorted);
        B3D_BARRIER();
        append_share(L, S, ncand, old_n, sorted);
        B3D_BARRIER();
        if (!L.active) return;
        int total = 0;
        for (int k = 0; k < hit_words(g); k++) total += __builtin_popcount(__builtin_bit_cast(uint32_t, hit[k * kLanes]));
        int cc = total < g.max_c ? total : g.max_c;
        int rest = __builtin_bit_cast(uint32_t, hit[hit_words(g) * kLanes]) != 0;
        sti(L.w, H_CONTACT_COUNT, cc);
        sti(L.w, H_CONTACT_OVERFLOW, ldi(L.w, H_CONTACT_OVERFLOW) | (total > g.max_c ? 1 : 0));
        sti(L.w, H_CONTACTS_DROPPED, ldi(L.w, H_CONTACTS_DROPPED) + (total - cc));
        sti(L.scr + L.g.scr_flags * kLanes, 0, rest ? kLaneRestitution : 0);
        return;
    }
    int cc = 0;
    int rest_any = 0;
    int overflow = ldi(L.w, H_CONTACT_OVERFLOW);
    int dropped = ldi(L.w, H_CONTACTS_DROPPED);
    /* the joint-connected body pairs, held in registers when there are few */
    uint32_t jkey[kJointKeyRegs];
#pragma unroll
    for (int k = 0; k < kJointKeyRegs; k++) jkey[k] = k < nj ? ldu(joint_rec(L, k), JS_KEY) : 0xffffffffu;
    PairShape A, B, An, Bn;
    OldWarm orec, orecn;
    uint32_t key = 0, key1 = 0;
    int match = -1, match1 = -1;
    if (ncand > 0) {
        key = ldu(cand, 0);
        match = ldi(cand, 1);
        pshape_load(L, (int)(key >> 16), &A);
        pshape_load(L, (int)(key & 0xffffu), &B);
        if (match >= 0) old_load(L, match, &orec);
    }
    if (ncand > 1) {
        key1 = ldu(cand, 2);
        match1 = ldi(cand, 3);
    }
    for (int t = 0; t < ncand; t++) {
        uint32_t key2 = 0;
        int match2 = -1;
        if (t + 2 < ncand) {
            key2 = ldu(cand, 2 * (t + 2));
            match2 = ldi(cand, 2 * (t + 2) + 1);
        }
        if (t + 1 < ncand) {
            if ((key1 >> 16) != (key >> 16)) pshape_load(L, (int)(key1 >> 16), &An);
            else An = A;
            pshape_load(L, (int)(key1 & 0xffffu), &Bn);
            if (match1 >= 0) old_load(L, match1, &orecn);
        }
        int i = (int)(key >> 16), j = (int)(key & 0xffffu);
        Mani m;
        m.count = 0;
        if (!pair_skipped(L, A, B, jkey, nj)) collide_pair(&m, A.P, B.P, L.vel);
        if (m.count > 0 && cc >= g.max_c) {
            overflow = 1;
            dropped++;
        } else if (m.count > 0) {
            rest_any |= write_new_contact(L, cc, i, j, A, B, m, sorted, match, orec, old_n) & CF_RESTITUTION;
            cc++;
        }
        A = An;
        B = Bn;
        orec = orecn;
        key = key1;
        key1 = key2;
        match = match1;
        match1 = match2;
    }
    sti(L.w, H_CONTACT_COUNT, cc);
    sti(L.w, H_CONTACT_OVERFLOW, overflow);
    sti(L.w, H_CONTACTS_DROPPED, dropped);
    sti(L.scr + L.g.scr_flags * kLanes, 0, rest_any ? kLaneRestitution : 0);
}

/* Contact generation and warm start: b3_find_contacts (08_contacts.inl:
 * 64-173).  The prepared fields are filled in by prepare_contacts. */
template <bool Masks = false>
B3D_FN void find_contacts(const Lane& L) {
    const Geometry& g = L.g;
    /* an idle lane of a shared tile has no old contacts, shapes or joints:
     * it only meets the other waves at find_pairs' barriers */
    int old_n = L.active ? clampi(ldi(L.w, H_CONTACT_COUNT), 0, g.max_c) : 0;
    /* with the overlap masks a shared tile's waves split the old contacts'
     * warm data and the shape pass before the first barrier (pair_helper);
     * wave 0 lists the keys */
    const bool split = Masks && L.staged;
    const int first = split ? L.st.wave : 0, stride = split ? L.st.waves : 1;
    int sorted = L.active ? old_keys(L, old_n) : 0;
    if (L.active) old_warm_copy(L, old_n, first, stride);
    int ns = L.active ? clampi(ldi(L.w, H_SHAPE_COUNT), 0, g.max_s) : 0;
    int nj = L.active ? clampi(ldi(L.w, H_JOINT_COUNT), 0, g.max_j) : 0;
    /* joint-connected body pairs (08:95-108) as sorted-pair keys */
    for (int j = 0; j < nj; j++) {
        uint32_t key = 0xffffffffu;
        if (!ldi(L.w, jw(L, j, J_COLLIDE_CONNECTED)))
            key = pair_key(ldi(L.w, jw(L, j, J_BODY_A)), ldi(L.w, jw(L, j, J_BODY_B)));
        sti(joint_rec(L, j), JS_KEY, (int)key);
    }
    if (bounds_in_lds(g) || (L.staged && L.st.lds_bounds)) {
        float* bounds = L.vel + kClipWords * kLanes;
        shape_pass(L, ns, bounds, first, stride);
        find_pairs<Masks>(L, bounds, ns, nj, old_n, sorted);
    } else {
        float* bounds = (float*)(L.scr + g.scr_bounds * kLanes);
        shape_pass(L, ns, bounds);
        find_pairs<Masks>(L, bounds, ns, nj, old_n, sorted);
    }
}

/* b3_apply_impulse (08:184-192) on staged velocities: impulse s * p at
 * lever r, dynamic bodies only. */
B3D_FN void apply_impulse(const Lane& L, int b, float m, M3 i, V3 r, V3 p, float s) {
    if (!is_dyn_flag(L, b)) return;
    set_vlin(L, b, madd(vlin(L, b), s * m, p));
    set_vang(L, b, add(vang(L, b), mv(i, scale(cross(r, p), s))));
}

/* b3_prepare_one_contact (08:234-291) for every new contact, two contacts
 * at a time: their heads, then their bodies and points, then the math.  The
 * prepared fields go to the world's contact rows and, with everything else
 * the solver reads, to the contact's packed record, whose point separations
 * start at the step's initial delta poses.
 *
 * The warm start of the contacts (08:194-232) applies their impulses in
 * contact order after all are prepared; preparation reads body velocities
 * only for the relative normal velocities, which only restitution and the
 * kept solver fields use.  A world with neither gets each contact's warm
 * start right after its preparation, with the same impulses in the same
 * order, and the function returns 1 (0: warm_start_contacts still to run). */
/* Contact levels for the shared sweeps (shared-narrowphase launches only).
 * A contact's solve reads and writes the velocities of its dynamic bodies
 * and nothing else a sweep changes, so two contacts with no dynamic body in
 * common give the same results in either order.  Level 1 + the highest
 * level among earlier contacts on the same dynamic bodies keeps every
 * body's sequence of updates in contact order; contacts of one level are
 * solved by the tile's waves together.
 * Per lane in the workgroup's LDS, past wave 0's rows: the lane's level
 * count, each body's last level, each contact's level (| its point count
 * << 16), and P: per level its contact count, then (prefix) its first
 * entry, then (after the fill) one past its last.  In the stage (free once
 * the manifolds are appended): the entries in level order, two words each
 * (contact, record slots: slot | point p's slot << 6 + 6p).
 * sched_build runs on wave 0 while the other waves prepare the contacts:
 * it needs only the contacts' heads, and it ranks the record slots itself. */
B3D_FN float* sched_rows(const Lane& L) { return L.vel + lds_rows(L.g) * kLanes; }
B3D_FN int sched_words(const Geometry& g) { return 2 + g.max_b + 2 * g.max_c; }
B3D_FN int sch_get(const Lane& L, int k) { return __builtin_bit_cast(int, sched_rows(L)[k * kLanes]); }
B3D_FN void sch_set(const Lane& L, int k, int v) { sched_rows(L)[k * kLanes] = __builtin_bit_cast(float, v); }
B3D_FN int sch_last(const Lane& L, int b) { return 1 + b; }
B3D_FN int sch_level(const Lane& L, int c) { return 1 + L.g.max_b + c; }
B3D_FN int sch_p(const Lane& L, int lev) { return 1 + L.g.max_b + L.g.max_c + lev; }
/* stage words of the schedule */
B3D_FN int stage_sched_words(const Geometry& g) { return 2 * g.max_c; }
B3D_FN uint32_t* sch_entry(const Lane& L, int i) { return L.st.p + (size_t)(1 + 2 * i) * kLanes; }

/* The largest level count among the tile's stepping lanes (every wave of
 * the tile gets the same value). */
B3D_FN int tile_levels(const Lane& L) {
    int v = sch_get(L, 0), m = 0;
    for (int bit = 15; bit >= 0; bit--) {
        int cand = m | (1 << bit);
        if (wave_any(L, v >= cand)) m = cand;
    }
    return m;
}

constexpr int kPrepChunk = 2;
B3D_FN int prepare_contacts(const Lane& L, Soft cs, Soft ss, int first = 0, int stride = 1) {
    uint32_t* w = L.w;
    int cc = contact_count_word(L);
    const float inv_tau = 1.0f / kSpeculative;
    const int keep = (L.opts & kKeepSolverFields) != 0;
    /* a shared tile prepares its contacts in parallel (chunks first,
     * first + stride, ... per wave) and warm-starts them afterwards, level
     * by level */
    const int fuse = !L.staged && !keep && !(ldi(L.scr + L.g.scr_flags * kLanes, 0) & kLaneRestitution);
    for (int c0 = first * kPrepChunk; c0 < cc; c0 += stride * kPrepChunk) {
        int a[kPrepChunk], b[kPrepChunk], pc[kPrepChunk], fl[kPrepChunk], slot[kPrepChunk];
        int pslot[kPrepChunk][kMaxManifold];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            slot[k] = wave_slot(L);
            CHead hd = chead_load(L, c);
            a[k] = hd.a;
            b[k] = hd.b;
            pc[k] = hd.pc;
            fl[k] = hd.flags;
        }
        int fixed[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int c = c0 + k;
            fixed[k] = 0;
            if (c >= cc) continue;
            /* a static body whose delta pose is untouched (no kKindClearDelta) */
            if (!(fl[k] & CF_DYN_A) && (ru(delta_rec(L, a[k]), BD_KIND) & (kKindStatic | kKindClearDelta)) == kKindStatic)
                fixed[k] |= CF_FIXED_A;
            if (!(fl[k] & CF_DYN_B) && (ru(delta_rec(L, b[k]), BD_KIND) & (kKindStatic | kKindClearDelta)) == kKindStatic)
                fixed[k] |= CF_FIXED_B;
        }
        float ima[kPrepChunk], imb[kPrepChunk];
        M3 iwa[kPrepChunk], iwb[kPrepChunk];
        V3 n[kPrepChunk], t1[kPrepChunk], ra[kPrepChunk][kMaxManifold], rb[kPrepChunk][kMaxManifold];
        float bs[kPrepChunk][kMaxManifold], ni[kPrepChunk][kMaxManifold];
        float fric[kPrepChunk], rest[kPrepChunk], roll_c[kPrepChunk], tw[kPrepChunk];
        V2 fi[kPrepChunk];
        V3 roll[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            fric[k] = ldf(w, cw(L, c, C_FRICTION));
            rest[k] = ldf(w, cw(L, c, C_RESTITUTION));
            roll_c[k] = ldf(w, cw(L, c, C_ROLLING));
            fi[k].x = ldf(w, cw(L, c, C_FRICTION_IMPULSE));
            fi[k].y = ldf(w, cw(L, c, C_FRICTION_IMPULSE + 1));
            tw[k] = ldf(w, cw(L, c, C_TWIST_IMPULSE));
            roll[k] = ld3(w, cw(L, c, C_ROLLING_IMPULSE));
            ima[k] = 0.0f;
            imb[k] = 0.0f;
            iwa[k] = m3zero();
            iwb[k] = m3zero();
            if (fl[k] & CF_DYN_A) {
                ima[k] = ldf(w, bw(L, a[k], B_INV_MASS));
                iwa[k] = ldm3(w, bw(L, a[k], B_INV_I_WORLD));
            }
            if (fl[k] & CF_DYN_B) {
                imb[k] = ldf(w, bw(L, b[k], B_INV_MASS));
                iwb[k] = ldm3(w, bw(L, b[k], B_INV_I_WORLD));
            }
            n[k] = ld3(w, cw(L, c, C_NORMAL));
            t1[k] = ld3(w, cw(L, c, C_TANGENT1));
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= pc[k]) continue;
                pslot[k][p] = wave_slot(L);
                ra[k][p] = ld3(w, pw(L, c, p, P_R_A));
                rb[k][p] = ld3(w, pw(L, c, p, P_R_B));
                bs[k][p] = ldf(w, pw(L, c, p, P_BASE_SEP));
                ni[k][p] = ldf(w, pw(L, c, p, P_NORMAL_IMPULSE));
            }
        }
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            uint32_t* r = crec(L, c, slot[k]);
            /* zero unless the body is dynamic (08:236-241) */
            float ma = ima[k], mb = imb[k];
            M3 ia = iwa[k], ib = iwb[k];
            const int need_rv = keep || (fl[k] & CF_RESTITUTION);
            V3 va = zero3(), wa = zero3(), vb = zero3(), wb = zero3();
            if (need_rv) {
                va = vlin(L, a[k]);
                wa = vang(L, a[k]);
                vb = vlin(L, b[k]);
                wb = vang(L, b[k]);
            }
            /* tangent2 = tangent1 x normal as written by b3_contact_from_mani */
            V3 t2 = cross(t1[k], n[k]);
            V3 center_a = zero3(), center_b = zero3();
            float wsum = 0.0f;
            float rel_vel[kMaxManifold], nmass[kMaxManifold], bsp[kMaxManifold],
                nip[kMaxManifold];
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                rel_vel[p] = 0.0f;
                nmass[p] = 0.0f;
                bsp[p] = 0.0f;
                nip[p] = 0.0f;
                if (p >= pc[k]) continue;
                V3 rap = ra[k][p], rbp = rb[k][p];
                V3 rn_a = cross(rap, n[k]);
                V3 rn_b = cross(rbp, n[k]);
                float kn = ma + mb + dot(rn_a, mv(ia, rn_a)) + dot(rn_b, mv(ib, rn_b));
                nmass[p] = kn > 0.0f ? 1.0f / kn : 0.0f;
                if (need_rv) {
                    V3 vra = add(va, cross(wa, rap));
                    V3 vrb = add(vb, cross(wb, rbp));
                    rel_vel[p] = dot(n[k], sub(vrb, vra));
                }
                float sep = bs[k][p] + dot(sub(rbp, rap), n[k]);
                float weight = clampf(2.0f - sep * inv_tau, kMinFrictionW, 1.0f);
                center_a = madd(center_a, weight, rap);
                center_b = madd(center_b, weight, rbp);
                wsum += weight;
                bsp[p] = bs[k][p];
                nip[p] = ni[k][p];
            }
            float invw = wsum > 0.0f ? 1.0f / wsum : 0.0f;
            center_a = scale(center_a, invw);
            center_b = scale(center_b, invw);
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= pc[k]) continue;
                float lever = len(sub(ra[k][p], center_a));
                uint32_t* pr = prec(L, c, p, pslot[k][p]);
                qs3(pr, PR_RA, ra[k][p]);
                qsf(pr, PR_NMASS, nmass[p]);
                qs3(pr, PR_RB, rb[k][p]);
                qsf(pr, PR_LEVER, lever);
                if (L.opts & kKeepSolverFields) {
                    stf(w, pw(L, c, p, P_NORMAL_MASS), nmass[p]);
                    stf(w, pw(L, c, p, P_REL_VEL), rel_vel[p]);
                    stf(w, pw(L, c, p, P_LEVER), lever);
                }
            }
            V3 rt_a1 = cross(center_a, t1[k]);
            V3 rt_a2 = cross(center_a, t2);
            V3 rt_b1 = cross(center_b, t1[k]);
            V3 rt_b2 = cross(center_b, t2);
            M2 k2;
            k2.cx.x = ma + mb + dot(rt_a1, mv(ia, rt_a1)) + dot(rt_b1, mv(ib, rt_b1));
            k2.cy.y = ma + mb + dot(rt_a2, mv(ia, rt_a2)) + dot(rt_b2, mv(ib, rt_b2));
            k2.cx.y = dot(rt_a1, mv(ia, rt_a2)) + dot(rt_b1, mv(ib, rt_b2));
            k2.cy.x = k2.cx.y;
            M2 tmass = inv2(k2);
            M3 isum = madd3(ia, ib);
            float kt = dot(n[k], mv(isum, n[k]));
            float twist_mass = kt > 0.0f ? 1.0f / kt : 0.0f;
            if (L.opts & kKeepSolverFields) {
                st3(w, cw(L, c, C_CENTER_A), center_a);
                st3(w, cw(L, c, C_CENTER_B), center_b);
                stf(w, cw(L, c, C_TWIST_MASS), twist_mass);
                stf(w, cw(L, c, C_TANGENT_MASS), tmass.cx.x);
                stf(w, cw(L, c, C_TANGENT_MASS + 1), tmass.cx.y);
                stf(w, cw(L, c, C_TANGENT_MASS + 2), tmass.cy.x);
                stf(w, cw(L, c, C_TANGENT_MASS + 3), tmass.cy.y);
                stm3(w, cw(L, c, C_ROLLING_MASS), inv3(isum));
                stf(w, cw(L, c, C_INV_MASS_A), ma);
                stf(w, cw(L, c, C_INV_MASS_B), mb);
                stm3(w, cw(L, c, C_INV_I_A), ia);
                stm3(w, cw(L, c, C_INV_I_B), ib);
                stsoft(w, cw(L, c, C_SOFTNESS), (fl[k] & CF_STATIC) ? ss : cs);
            }
            /* the packed record */
            qsu(r, R_AB, (uint32_t)(a[k] | (b[k] << 16)));
            qsu(r, R_INFO, (uint32_t)(pc[k] | ((fl[k] | fixed[k]) << 8)));
            qsf(r, R_FRICTION, fric[k]);
            qsf(r, R_TWIST_MASS, twist_mass);
            qs3(r, R_N, n[k]);
            qsf(r, R_ROLLING, roll_c[k]);
            rec_store_masses(r, fl[k], ma, ia, mb, ib);
            qs3(r, R_T1, t1[k]);
            qsf(r, R_TM_XX, tmass.cx.x);
            qs3(r, R_CA, center_a);
            qsf(r, R_TM_XY, tmass.cx.y);
            qs3(r, R_CB, center_b);
            qsf(r, R_TM_YY, tmass.cy.y);
            qsf(r, R_FI, fi[k].x);
            qsf(r, R_FI + 1, fi[k].y);
            qsf(r, R_TWIST, tw[k]);
            qsf(r, R_RESTITUTION, rest[k]);
            qs3(r, R_ROLL, roll[k]);
            if (fl[k] & CF_RESTITUTION) {
#pragma unroll
                for (int p = 0; p < kMaxManifold; p++) qsf(r, R_REL_VEL + p, rel_vel[p]);
            }
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                qsf(r, R_BASE_SEP + p, bsp[p]);
            }
#pragma unroll
            for (int p = 0; p < 2; p++) {
                qsf(r, R_NI + 2 * p, nip[p]);
                qsf(r, R_TN + 2 * p, 0.0f);
            }
            if (pc[k] > 2) {
#pragma unroll
                for (int p = 2; p < kMaxManifold; p++) {
                    qsf(r, R_NI + 2 * p, nip[p]);
                    qsf(r, R_TN + 2 * p, 0.0f);
                }
            }
            if (fuse) {
                /* warm_start_contacts' impulses for this contact */
#pragma unroll
                for (int p = 0; p < kMaxManifold; p++) {
                    if (p >= pc[k]) continue;
                    V3 P = scale(n[k], nip[p]);
                    apply_impulse(L, a[k], ma, ia, ra[k][p], P, -1.0f);
                    apply_impulse(L, b[k], mb, ib, rb[k][p], P, 1.0f);
                }
                V3 f = add(scale(t1[k], fi[k].x), scale(t2, fi[k].y));
                apply_impulse(L, a[k], ma, ia, center_a, f, -1.0f);
                apply_impulse(L, b[k], mb, ib, center_b, f, 1.0f);
                V3 tr = add(scale(n[k], tw[k]), roll[k]);
                if (is_dyn_flag(L, a[k])) set_vang(L, a[k], sub(vang(L, a[k]), mv(ia, tr)));
                if (is_dyn_flag(L, b[k])) set_vang(L, b[k], add(vang(L, b[k]), mv(ib, tr)));
            }
        }
    }
    return fuse;
}

/* A shared tile's contact levels (wave 0, after the parallel preparation):
 * each contact's level from its dynamic bodies' last levels, in contact
 * order, then a counting sort of the contacts by level into the entries. */
constexpr int kSchedChunk = 8;
B3D_FN void sched_build(const Lane& L) {
    int cc = clampi(contact_count_word(L), 0, L.g.max_c);
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) sch_set(L, sch_last(L, b), 0);
    for (int lev = 0; lev <= cc; lev++) sch_set(L, sch_p(L, lev), 0);
    int nlev = 0;
    /* the heads, then the slots, are loaded kSchedChunk contacts at a time
     * ahead of the LDS and stage writes, which the compiler would not move
     * loads across */
    for (int c0 = 0; c0 < cc; c0 += kSchedChunk) {
        CHead hds[kSchedChunk];
#pragma unroll
        for (int k = 0; k < kSchedChunk; k++)
            if (c0 + k < cc) hds[k] = chead_load(L, c0 + k);
#pragma unroll
        for (int k = 0; k < kSchedChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            const CHead& hd = hds[k];
            int la = (hd.flags & CF_DYN_A) ? sch_get(L, sch_last(L, hd.a)) : 0;
            int lb = (hd.flags & CF_DYN_B) ? sch_get(L, sch_last(L, hd.b)) : 0;
            int lev = (la > lb ? la : lb) + 1;
            if (hd.flags & CF_DYN_A) sch_set(L, sch_last(L, hd.a), lev);
            if (hd.flags & CF_DYN_B) sch_set(L, sch_last(L, hd.b), lev);
            sch_set(L, sch_level(L, c), lev | (hd.pc << 16));
            sch_set(L, sch_p(L, lev), sch_get(L, sch_p(L, lev)) + 1);
            if (lev > nlev) nlev = lev;
        }
    }
    sch_set(L, 0, nlev);
    int run = 0;
    for (int lev = 1; lev <= nlev; lev++) {
        int n = sch_get(L, sch_p(L, lev));
        sch_set(L, sch_p(L, lev), run);
        run += n;
    }
    /* each entry with the contact's record slots, ranked as
     * prepare_contacts ranks them: among the lanes with contact c, and
     * among those with its point p */
    for (int c = 0; c < cc; c++) {
        int lw = sch_get(L, sch_level(L, c));
        int lev = lw & 0xffff, pc = lw >> 16;
        int packed = wave_slot(L);
#pragma unroll
        for (int p = 0; p < kMaxManifold; p++) {
            if (p >= pc) continue;
            packed |= wave_slot(L) << (6 + 6 * p);
        }
        int at = sch_get(L, sch_p(L, lev));
        sch_set(L, sch_p(L, lev), at + 1);
        uint32_t* e = sch_entry(L, at);
        sti(e, 0, c);
        sti(e, 1, packed);
    }
}

/* b3_prepare_joints (06_joints.inl:161-202), plus the hinge axis through
 * each inverse inertia, which is fixed for the step. */
B3D_FN void prepare_joints(const Lane& L, float h, int first = 0, int stride = 1) {
    int nj = joint_count(L);
    uint32_t* w = L.w;
    /* chunks of kPrepChunk joints first, first + stride, ... (a shared
     * tile's waves split them) */
    for (int j0 = first * kPrepChunk; j0 < nj; j0 += stride * kPrepChunk) {
        /* the joints' own fields, then (through their body indices) the bodies' */
        int a[kPrepChunk], b[kPrepChunk], jtype[kPrepChunk], en[kPrepChunk];
        float chz[kPrepChunk], cdr[kPrepChunk], lh[kPrepChunk], ld[kPrepChunk], ah[kPrepChunk], ad[kPrepChunk];
        float hz[kPrepChunk], dr[kPrepChunk];
        Q lra[kPrepChunk], lrb[kPrepChunk];
        V3 laa[kPrepChunk], lab[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int i = j0 + k;
            if (i >= nj) continue;
            a[k] = ldi(w, jw(L, i, J_BODY_A));
            b[k] = ldi(w, jw(L, i, J_BODY_B));
            jtype[k] = ldi(w, jw(L, i, J_TYPE));
            en[k] = (ldi(w, jw(L, i, J_ENABLE_SPRING)) ? JF_SPRING : 0) | (ldi(w, jw(L, i, J_ENABLE_MOTOR)) ? JF_MOTOR : 0)
                | (ldi(w, jw(L, i, J_ENABLE_LIMIT)) ? JF_LIMIT : 0);
            chz[k] = ldf(w, jw(L, i, J_CONSTRAINT_HERTZ));
            cdr[k] = ldf(w, jw(L, i, J_CONSTRAINT_DAMPING));
            lra[k] = ldq(w, jw(L, i, J_LOCAL_ROT_A));
            lrb[k] = ldq(w, jw(L, i, J_LOCAL_ROT_B));
            laa[k] = ld3(w, jw(L, i, J_LOCAL_ANCHOR_A));
            lab[k] = ld3(w, jw(L, i, J_LOCAL_ANCHOR_B));
            lh[k] = ldf(w, jw(L, i, J_LINEAR_HERTZ));
            ld[k] = ldf(w, jw(L, i, J_LINEAR_DAMPING));
            ah[k] = ldf(w, jw(L, i, J_ANGULAR_HERTZ));
            ad[k] = ldf(w, jw(L, i, J_ANGULAR_DAMPING));
            hz[k] = ldf(w, jw(L, i, J_HERTZ));
            dr[k] = ldf(w, jw(L, i, J_DAMPING_RATIO));
        }
        int ta[kPrepChunk], tb[kPrepChunk];
        float ima[kPrepChunk], imb[kPrepChunk];
        M3 iwa[kPrepChunk], iwb[kPrepChunk];
        Q rot_a[kPrepChunk], rot_b[kPrepChunk];
        V3 lca[kPrepChunk], lcb[kPrepChunk], cen_a[kPrepChunk], cen_b[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int i = j0 + k;
            if (i >= nj) continue;
            ta[k] = ldi(w, bw(L, a[k], B_TYPE));
            tb[k] = ldi(w, bw(L, b[k], B_TYPE));
            ima[k] = ldf(w, bw(L, a[k], B_INV_MASS));
            imb[k] = ldf(w, bw(L, b[k], B_INV_MASS));
            iwa[k] = ldm3(w, bw(L, a[k], B_INV_I_WORLD));
            iwb[k] = ldm3(w, bw(L, b[k], B_INV_I_WORLD));
            rot_a[k] = ldq(w, bw(L, a[k], B_ROTATION));
            rot_b[k] = ldq(w, bw(L, b[k], B_ROTATION));
            lca[k] = ld3(w, bw(L, a[k], B_LOCAL_CENTER));
            lcb[k] = ld3(w, bw(L, b[k], B_LOCAL_CENTER));
            cen_a[k] = ld3(w, bw(L, a[k], B_CENTER));
            cen_b[k] = ld3(w, bw(L, b[k], B_CENTER));
        }
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int i = j0 + k;
            if (i >= nj) continue;
            /* zero unless the body is dynamic */
            float ma = ta[k] == kDynamic ? ima[k] : 0.0f;
            float mb = tb[k] == kDynamic ? imb[k] : 0.0f;
            M3 ia = ta[k] == kDynamic ? iwa[k] : m3zero();
            M3 ib = tb[k] == kDynamic ? iwb[k] : m3zero();
            stf(w, jw(L, i, J_INV_MASS_A), ma);
            stf(w, jw(L, i, J_INV_MASS_B), mb);
            stm3(w, jw(L, i, J_INV_I_A), ia);
            stm3(w, jw(L, i, J_INV_I_B), ib);
            M3 isum = madd3(ia, ib);
            int fixed = dot(isum.cx, cross(isum.cy, isum.cz)) < 1.0e-20f;
            sti(w, jw(L, i, J_FIXED_ROTATION), fixed);
            int info = (jtype[k] == kJointWeld ? JF_WELD : 0) | (fixed ? JF_FIXED : 0) | en[k]
                | (ta[k] == kDynamic ? JF_DYN_A : 0) | (tb[k] == kDynamic ? JF_DYN_B : 0);
            sti(joint_rec(L, i), JS_AB, a[k] | (b[k] << 16));
            sti(joint_rec(L, i), JS_INFO, info);
            Soft soft = make_soft(chz[k], cdr[k], h);
            stsoft(w, jw(L, i, J_SOFTNESS), soft);
            Q fqa = qmul(rot_a[k], lra[k]);
            Q fqb = qmul(rot_b[k], lrb[k]);
            stq(w, jw(L, i, J_FRAME_Q_A), fqa);
            stq(w, jw(L, i, J_FRAME_Q_B), fqb);
            st3(w, jw(L, i, J_FRAME_P_A), rot(rot_a[k], sub(laa[k], lca[k])));
            st3(w, jw(L, i, J_FRAME_P_B), rot(rot_b[k], sub(lab[k], lcb[k])));
            st3(w, jw(L, i, J_DELTA_CENTER), sub(cen_b[k], cen_a[k]));
            if (jtype[k] == kJointWeld) {
                stm3(w, jw(L, i, J_ANGULAR_MASS), inv3(isum));
                stsoft(w, jw(L, i, J_LINEAR_SPRING), lh[k] == 0.0f ? soft : make_soft(lh[k], ld[k], h));
                stsoft(w, jw(L, i, J_ANGULAR_SPRING), ah[k] == 0.0f ? soft : make_soft(ah[k], ad[k], h));
            } else {
                V3 axis = rot(fqa, v3(0.0f, 0.0f, 1.0f));
                float kk = dot(axis, mv(isum, axis));
                stf(w, jw(L, i, J_AXIAL_MASS), kk > 0.0f ? 1.0f / kk : 0.0f);
                st3(w, jw(L, i, J_ROTATION_AXIS), axis);
                /* the spring, motor and limit rows' angular impulse directions
                 * (06:470-560 multiply by the inverse inertias every solve) */
                st3(joint_rec(L, i), JS_IAX, mv(ia, axis));
                st3(joint_rec(L, i), JS_IBX, mv(ib, axis));
                Q rel = qinv_mul(fqa, fqb);
                V3 px, py;
                hinge_perps(fqa, rel, &px, &py);
                st3(w, jw(L, i, J_PERP_X), px);
                st3(w, jw(L, i, J_PERP_Y), py);
                stsoft(w, jw(L, i, J_SPRING_SOFTNESS), make_soft(hz[k], dr[k], h));
            }
        }
    }
}

/* b3_warm_start over contacts (08:194-232, 293-313), two contacts at a
 * time: heads, then records, then the impulses in contact order.  Lanes
 * whose warm start ran inside prepare_contacts (`done`) only take part in
 * the record slots' ranks. */
B3D_FN void warm_start_contacts(const Lane& L, int done) {
    int cc = contact_count_word(L);
    for (int c0 = 0; c0 < cc; c0 += kPrepChunk) {
        CHead hd[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            hd[k] = rhead_load(L, c);
        }
        float ma[kPrepChunk], mb[kPrepChunk], ni[kPrepChunk][kMaxManifold], tw[kPrepChunk];
        M3 ia[kPrepChunk], ib[kPrepChunk];
        V3 n[kPrepChunk], ra[kPrepChunk][kMaxManifold], rb[kPrepChunk][kMaxManifold], t1[kPrepChunk];
        V3 ca[kPrepChunk], cb[kPrepChunk], roll[kPrepChunk];
        V2 fi[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            /* every lane with the point takes part in its slot's rank */
            int ps[kMaxManifold];
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++)
                if (p < hd[k].pc) ps[p] = wave_slot(L);
            if (done) continue;
            const uint32_t* r = crec(L, c, hd[k].slot);
            rec_masses(r, hd[k].flags, &ma[k], &ia[k], &mb[k], &ib[k]);
            n[k] = q3(r, R_N);
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= hd[k].pc) continue;
                const uint32_t* pr = prec(L, c, p, ps[p]);
                ni[k][p] = qf(r, R_NI + 2 * p);
                ra[k][p] = q3(pr, PR_RA);
                rb[k][p] = q3(pr, PR_RB);
            }
            t1[k] = q3(r, R_T1);
            fi[k].x = qf(r, R_FI);
            fi[k].y = qf(r, R_FI + 1);
            ca[k] = q3(r, R_CA);
            cb[k] = q3(r, R_CB);
            tw[k] = qf(r, R_TWIST);
            roll[k] = q3(r, R_ROLL);
        }
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int c = c0 + k;
            if (c >= cc || done) continue;
            int a = hd[k].a, b = hd[k].b;
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= hd[k].pc) continue;
                V3 P = scale(n[k], ni[k][p]);
                apply_impulse(L, a, ma[k], ia[k], ra[k][p], P, -1.0f);
                apply_impulse(L, b, mb[k], ib[k], rb[k][p], P, 1.0f);
            }
            V3 t2 = cross(t1[k], n[k]);
            V3 f = add(scale(t1[k], fi[k].x), scale(t2, fi[k].y));
            apply_impulse(L, a, ma[k], ia[k], ca[k], f, -1.0f);
            apply_impulse(L, b, mb[k], ib[k], cb[k], f, 1.0f);
            V3 tr = add(scale(n[k], tw[k]), roll[k]);
            if (is_dyn_flag(L, a)) set_vang(L, a, sub(vang(L, a), mv(ia[k], tr)));
            if (is_dyn_flag(L, b)) set_vang(L, b, add(vang(L, b), mv(ib[k], tr)));
        }
    }
}

/* b3_warm_start_joints (06:204-239).  JI: also stages each joint's
 * accumulated impulses into its LDS impulse row, for the solves. */
template <bool JI = false>
B3D_FN void warm_start_joints(const Lane& L) {
    int nj = joint_count(L);
    const uint32_t* w = L.w;
    for (int i = 0; i < nj; i++) {
        int a = ldi(w, jw(L, i, J_BODY_A)), b = ldi(w, jw(L, i, J_BODY_B));
        V3 ra = rot(rq4(delta_rec(L, a), BD_DQ), ld3(w, jw(L, i, J_FRAME_P_A)));
        V3 rb = rot(rq4(delta_rec(L, b), BD_DQ), ld3(w, jw(L, i, J_FRAME_P_B)));
        V3 lin = ld3(w, jw(L, i, J_LINEAR_IMPULSE));
        V3 ang = ld3(w, jw(L, i, J_ANGULAR_IMPULSE));
        if constexpr (JI) {
            jls3(ji_rec(L, i), JI_LIN, lin);
            jls3(ji_rec(L, i), JI_ANG, ang);       /* a weld's; a hinge's words follow */
        }
        if (ldi(w, jw(L, i, J_TYPE)) == kJointRevolute) {
            float spring = ldf(w, jw(L, i, J_SPRING_IMPULSE)), motor = ldf(w, jw(L, i, J_MOTOR_IMPULSE));
            float lower = ldf(w, jw(L, i, J_LOWER_IMPULSE)), upper = ldf(w, jw(L, i, J_UPPER_IMPULSE));
            float px = ldf(w, jw(L, i, J_PERP_IMPULSE)), py = ldf(w, jw(L, i, J_PERP_IMPULSE + 1));
            if constexpr (JI) {
                float* q = ji_rec(L, i);
                jlsf(q, JI_PERP, px);
                jlsf(q, JI_PERP + 1, py);
                jlsf(q, JI_SPRING, spring);
                jlsf(q, JI_MOTOR, motor);
                jlsf(q, JI_LOWER, lower);
                jlsf(q, JI_UPPER, upper);
            }
            float axial = spring + motor + lower - upper;
            ang = add(scale(ld3(w, jw(L, i, J_PERP_X)), px), scale(ld3(w, jw(L, i, J_PERP_Y)), py));
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

/* Point constraint mass (06:241-255). */
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

/* Everything the contact and joint rows need from the bodies' delta poses
 * (delta_pos, delta_rot), which change only in integrate_positions.  The
 * reference recomputes these in every row solve (08_contacts.inl:331-333,
 * 06_joints.inl:257-282, 285-332, 436-642); computing them once per delta
 * state gives the same bits. */
B3D_FN void joint_geometry(const Lane& L, int first = 0, int stride = 1);

/* Geometry of the joints at new delta poses.  The contacts' separations
 * are computed by each solve from the bodies' delta poses. */
B3D_FN void delta_geometry(const Lane& L) { joint_geometry(L); }

/* The joint rows' delta-pose geometry, joints first, first + stride, ...
 * (a shared tile's waves split them). */
B3D_FN void joint_geometry(const Lane& L, int first, int stride) {
    uint32_t* w = L.w;
    int nj = joint_count(L);
    for (int j0 = first; j0 < nj; j0 += kPrepChunk * stride) {
        int a[kPrepChunk], b[kPrepChunk], info[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int j = j0 + k * stride;
            if (j >= nj) continue;
            uint32_t ab = ldu(joint_rec(L, j), JS_AB);
            a[k] = (int)(ab & 0xffffu);
            b[k] = (int)(ab >> 16);
            info[k] = ldi(joint_rec(L, j), JS_INFO);
        }
        Q dqa[kPrepChunk], dqb[kPrepChunk], fqa[kPrepChunk], fqb[kPrepChunk];
        V3 dpa[kPrepChunk], dpb[kPrepChunk], fpa[kPrepChunk], fpb[kPrepChunk], dcen[kPrepChunk];
        float ma[kPrepChunk], mb[kPrepChunk];
        M3 ia[kPrepChunk], ib[kPrepChunk];
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int j = j0 + k * stride;
            if (j >= nj) continue;
            const uint32_t* da = delta_rec(L, a[k]);
            const uint32_t* db = delta_rec(L, b[k]);
            dqa[k] = rq4(da, BD_DQ);
            dqb[k] = rq4(db, BD_DQ);
            dpa[k] = r3(da, BD_DP);
            dpb[k] = r3(db, BD_DP);
            fqa[k] = ldq(w, jw(L, j, J_FRAME_Q_A));
            fqb[k] = ldq(w, jw(L, j, J_FRAME_Q_B));
            fpa[k] = ld3(w, jw(L, j, J_FRAME_P_A));
            fpb[k] = ld3(w, jw(L, j, J_FRAME_P_B));
            dcen[k] = ld3(w, jw(L, j, J_DELTA_CENTER));
            /* the masses as jrow_load gives them to the solves */
            ma[k] = 0.0f;
            mb[k] = 0.0f;
            ia[k] = m3zero();
            ib[k] = m3zero();
            if (info[k] & JF_DYN_A) {
                ma[k] = ldf(w, jw(L, j, J_INV_MASS_A));
                ia[k] = ldm3(w, jw(L, j, J_INV_I_A));
            }
            if (info[k] & JF_DYN_B) {
                mb[k] = ldf(w, jw(L, j, J_INV_MASS_B));
                ib[k] = ldm3(w, jw(L, j, J_INV_I_B));
            }
        }
#pragma unroll
        for (int k = 0; k < kPrepChunk; k++) {
            int j = j0 + k * stride;
            if (j >= nj) continue;
            uint32_t* r = joint_rec(L, j);
            Q qa = qmul(dqa[k], fqa[k]);
            Q qb = qmul(dqb[k], fqb[k]);
            if (qdot(qa, qb) < 0.0f) qb = qneg(qb);
            Q rel = qinv_mul(qa, qb);
            V3 ra = rot(dqa[k], fpa[k]);
            V3 rb = rot(dqb[k], fpb[k]);
            st3(r, JS_RA, ra);
            st3(r, JS_RB, rb);
            st3(r, JS_PSEP, add(add(sub(dpb[k], dpa[k]), sub(rb, ra)), dcen[k]));
            /* the point rows' matrix as b3_solve3 inverts it in every solve
             * (06:241-255, 03_math.inl:343-345) */
            stm3(r, JS_PKI, inv3(point_k(ma[k], mb[k], ia[k], ib[k], ra, rb)));
            int fixed = info[k] & JF_FIXED;
            if (info[k] & JF_WELD) {
                if (fixed) continue;
                Q sq = rel;
                if (rel.s < 0.0f) sq = qneg(rel);
                Q diff = q4(-sq.v.x, -sq.v.y, -sq.v.z, 1.0f - sq.s);
                st3(r, JS_CV, neg(rot(qa, scale(qmul(diff, qconj(sq)).v, 2.0f))));
                continue;
            }
            int need_twist = (info[k] & (JF_SPRING | JF_MOTOR | JF_LIMIT)) && !fixed;
            stf(r, JS_TW, need_twist ? twist(rel) : 0.0f);
            stf(r, JS_RELX, rel.v.x);
            stf(r, JS_RELY, rel.v.y);
            if (!fixed) {
                V3 px, py;
                hinge_perps(qa, rel, &px, &py);
                st3(r, JS_PX, px);
                st3(r, JS_PY, py);
                /* the perpendicular rows' 2x2 matrix and b3_solve2's
                 * reciprocal determinant (06:600-626, 03_math.inl:347-359) */
                M3 isum = madd3(ia[k], ib[k]);
                float kxx = dot(px, mv(isum, px));
                float kyy = dot(py, mv(isum, py));
                float kxy = dot(px, mv(isum, py));
                float det = kxx * kyy - kxy * kxy;
                stf(r, JS_KXX, kxx);
                stf(r, JS_KXY, kxy);
                stf(r, JS_KYY, kyy);
                stf(r, JS_KINV, det <= 1.0e-12f ? __builtin_nanf("") : 1.0f / det);
                /* the solve's latest hinge rows are part of the joint state */
                st3(w, jw(L, j, J_PERP_X), px);
                st3(w, jw(L, j, J_PERP_Y), py);
            }
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

/* The contact row as one solve needs it, loaded ahead of use. */
struct CPoint { V3 ra, rb; float nmass, ni, tn, lever, base_sep; };
struct CRow {
    int a, b, pc, flags, slot;
    V3 n;
    V3 dpa, dpb;  /* the bodies' delta poses */
    Q dqa, dqb;
    float ma, mb;
    M3 ia, ib;
    Soft soft;
    CPoint pt[kMaxManifold];
    float friction, twist_mass, twist_imp, rolling;
    V2 fi;
    V3 t1, t2, ca, cb;
    M2 tm;
};

/* Masses of a row, loaded when its solve starts; the softness is the
 * world's static or dynamic contact softness. */
template <bool S>
B3D_FN void crow_masses(const Lane& L, int c, CRow* r, Soft cs, Soft ss) {
    const uint32_t* rc = crec(L, c, r->slot);
    r->ma = 0.0f;
    r->mb = 0.0f;
    r->ia = m3zero();
    r->ib = m3zero();
    if (r->flags & CF_DYN_A) {
        r->ma = qfs<S>(rc, R_MA);
        r->ia.cx = q3s<S>(rc, R_IA);
        r->ia.cy = q3s<S>(rc, R_IA + 3);
        r->ia.cz = q3s<S>(rc, R_IA + 6);
    }
    if (r->flags & CF_DYN_B) {
        r->mb = qfs<S>(rc, R_MB);
        r->ib.cx = q3s<S>(rc, R_IB);
        r->ib.cy = q3s<S>(rc, R_IB + 3);
        r->ib.cz = v3(qfs<S>(rc, R_IB + 6), qfs<S>(rc, R_IB_ZYZ), qfs<S>(rc, R_IB_ZYZ + 1));
    }
    /* field by field: a select between the two structs would be one between
     * their addresses, which stops the compiler from splitting a row kept
     * for the step (kept_row) into scalars */
    bool st = (r->flags & CF_STATIC) != 0;
    r->soft.bias_rate = st ? ss.bias_rate : cs.bias_rate;
    r->soft.mass_scale = st ? ss.mass_scale : cs.mass_scale;
    r->soft.impulse_scale = st ? ss.impulse_scale : cs.impulse_scale;
}

/* The delta poses of a row's bodies (a static body's are exactly zero and
 * the identity for the whole step). */
B3D_FN void crow_deltas(const Lane& L, CRow* r) {
    if (r->flags & CF_FIXED_A) {
        r->dpa = zero3();
        r->dqa = qid();
    } else {
        const uint32_t* da = delta_rec(L, r->a);
        r->dpa = r3(da, BD_DP);
        r->dqa = rq4(da, BD_DQ);
    }
    if (r->flags & CF_FIXED_B) {
        r->dpb = zero3();
        r->dqb = qid();
    } else {
        const uint32_t* db = delta_rec(L, r->b);
        r->dpb = r3(db, BD_DP);
        r->dqb = rq4(db, BD_DQ);
    }
}

/* Normal, points and friction data of a row: loaded one contact ahead.
 * Call where exactly the lanes with a contact c run. */
template <bool S>
B3D_FN void crow_load(const Lane& L, int c, CHead h, int relax, CRow* r, const int* ps = nullptr) {
    const uint32_t* rc = crec(L, c, h.slot);
    r->a = h.a;
    r->b = h.b;
    r->pc = h.pc;
    r->flags = h.flags;
    r->slot = h.slot;
    r->friction = h.friction;
    r->twist_mass = h.twist_mass;
    r->n = q3s<S>(rc, R_N);
    r->rolling = qfs<S>(rc, R_ROLLING);
    crow_deltas(L, r);
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++) {
        CPoint& q = r->pt[p];
        q.ni = 0.0f;
        q.tn = 0.0f;
        if (p >= h.pc) continue;
        const uint32_t* pr = prec(L, c, p, ps ? ps[p] : wave_slot(L));
        q.ra = q3s<S>(pr, PR_RA);
        q.nmass = qfs<S>(pr, PR_NMASS);
        q.rb = q3s<S>(pr, PR_RB);
        q.lever = relax ? qfs<S>(pr, PR_LEVER) : 0.0f;
        q.base_sep = qfs<S>(rc, R_BASE_SEP + p);
        q.ni = qfs<S>(rc, R_NI + 2 * p);
        q.tn = qfs<S>(rc, R_TN + 2 * p);
    }
    if (relax) {
        r->fi.x = qfs<S>(rc, R_FI);
        r->fi.y = qfs<S>(rc, R_FI + 1);
        r->twist_imp = qfs<S>(rc, R_TWIST);
        r->t1 = q3s<S>(rc, R_T1);
        /* tangent2 = tangent1 x normal as written by b3_contact_from_mani */
        r->t2 = cross(r->t1, r->n);
        r->ca = q3s<S>(rc, R_CA);
        r->cb = q3s<S>(rc, R_CB);
        /* the inverse of a symmetric 2x2 is stored symmetric bit for bit */
        r->tm.cx.x = qfs<S>(rc, R_TM_XX);
        r->tm.cx.y = qfs<S>(rc, R_TM_XY);
        r->tm.cy.x = r->tm.cx.y;
        r->tm.cy.y = qfs<S>(rc, R_TM_YY);
    }
}

/* One contact, b3_solve_one_contact (08:315-413): soft normal rows, then in
 * the relax pass twist friction, 2-D friction at the anchor and rolling. */
B3D_FN void crow_solve(const Lane& L, int c, CRow& r, float inv_h, float contact_speed, int use_bias) {
    uint32_t* rc = crec(L, c, r.slot);
    V3 va = vlin(L, r.a), wa = vang(L, r.a), vb = vlin(L, r.b), wb = vang(L, r.b);
    V3 n = r.n;
    float total_n = 0.0f;
    float twist_lim = 0.0f;
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++) {
        if (p >= r.pc) continue;
        CPoint& q = r.pt[p];
        /* the point's separation at the current delta poses (08:331-333) */
        V3 ds = add(sub(r.dpb, r.dpa), sub(rot(r.dqb, q.rb), rot(r.dqa, q.ra)));
        float sep = dot(ds, n) + q.base_sep;
        float vbias = 0.0f, mscale = 1.0f, iscale = 0.0f;
        if (sep > 0.0f) {
            vbias = sep * inv_h;
        } else if (use_bias) {
            vbias = maxf(r.soft.mass_scale * r.soft.bias_rate * sep, -contact_speed);
            mscale = r.soft.mass_scale;
            iscale = r.soft.impulse_scale;
        }
        V3 vra = add(va, cross(wa, q.ra));
        V3 vrb = add(vb, cross(wb, q.rb));
        float vn = dot(sub(vrb, vra), n);
        float dimp = -q.nmass * (mscale * vn + vbias) - iscale * q.ni;
        float nimp = maxf(q.ni + dimp, 0.0f);
        dimp = nimp - q.ni;
        q.ni = nimp;
        q.tn = q.tn + nimp;
        total_n += nimp;
        twist_lim += q.lever * nimp;
        V3 P = scale(n, dimp);
        va = msub(va, r.ma, P);
        wa = sub(wa, mv(r.ia, cross(q.ra, P)));
        vb = madd(vb, r.mb, P);
        wb = add(wb, mv(r.ib, cross(q.rb, P)));
    }
    /* the accumulated impulses go back as whole quads */
#pragma unroll
    for (int p = 0; p < 2; p++) {
        qsf(rc, R_NI + 2 * p, r.pt[p].ni);
        qsf(rc, R_TN + 2 * p, r.pt[p].tn);
    }
    if (r.pc > 2) {
#pragma unroll
        for (int p = 2; p < kMaxManifold; p++) {
            qsf(rc, R_NI + 2 * p, r.pt[p].ni);
            qsf(rc, R_TN + 2 * p, r.pt[p].tn);
        }
    }
    if (!use_bias) {
        float twist_s = dot(n, sub(wb, wa));
        float max_t = r.friction * twist_lim;
        float dtw = -r.twist_mass * twist_s;
        float new_t = clampf(r.twist_imp + dtw, -max_t, max_t);
        qsf(rc, R_TWIST, new_t);
        dtw = new_t - r.twist_imp;
        r.twist_imp = new_t;           /* the row stays current (a row kept for the step) */
        wa = sub(wa, mv(r.ia, scale(n, dtw)));
        wb = add(wb, mv(r.ib, scale(n, dtw)));

        V3 vra = add(va, cross(wa, r.ca));
        V3 vrb = add(vb, cross(wb, r.cb));
        V3 vr = sub(vrb, vra);
        V2 vt;
        vt.x = dot(vr, r.t1);
        vt.y = dot(vr, r.t2);
        V2 tmv = mv2(r.tm, vt);
        V2 ni;
        ni.x = r.fi.x - tmv.x;
        ni.y = r.fi.y - tmv.y;
        float max_f = r.friction * total_n;
        float fl2 = ni.x * ni.x + ni.y * ni.y;
        if (fl2 > max_f * max_f && fl2 > 0.0f) {
            float sc = rsqrt_scale(max_f, fl2);
            ni.x *= sc;
            ni.y *= sc;
        }
        V2 df;
        df.x = ni.x - r.fi.x;
        df.y = ni.y - r.fi.y;
        qsf(rc, R_FI, ni.x);
        qsf(rc, R_FI + 1, ni.y);
        r.fi = ni;
        V3 P = add(scale(r.t1, df.x), scale(r.t2, df.y));
        va = msub(va, r.ma, P);
        wa = sub(wa, mv(r.ia, cross(r.ca, P)));
        vb = madd(vb, r.mb, P);
        wb = add(wb, mv(r.ib, cross(r.cb, P)));
        if (r.flags & CF_ROLLING) {
            V3 ri = q3(rc, R_ROLL);
            solve_rolling(r.t1, r.t2, r.rolling, total_n, r.ia, r.ib, &ri, &wa, &wb);
            qs3(rc, R_ROLL, ri);
        }
    }
    if (is_dyn_flag(L, r.a)) {
        set_vlin(L, r.a, va);
        set_vang(L, r.a, wa);
    }
    if (is_dyn_flag(L, r.b)) {
        set_vlin(L, r.b, vb);
        set_vang(L, r.b, wb);
    }
}

/* b3_solve_contacts (08:415-437): one Gauss-Seidel sweep in contact order.
 * Rows c+1 and c+2 (masses included) are in flight while row c is solved,
 * and the head of row c+3 while row c+2 loads.  The one-wave step runs
 * large batches, so the rows are streamed (qus).  With `row0` and `have0`,
 * contact 0's row is the one the step keeps (kept_row), its impulses
 * current; `deltas`: its bodies' delta poses have moved since it was last
 * used (a position update), so they are loaded again.  (A null row0 is a
 * compile-time constant at every call: the kept row is never selected
 * through a pointer, which would stop the compiler from splitting it.) */
B3D_FN void solve_contacts(const Lane& L, float inv_h, float contact_speed, int use_bias, Soft cs, Soft ss,
        CRow* row0 = nullptr, int have0 = 0, bool deltas = false) {
    int cc = contact_count_word(L);
    if (cc <= 0) return;
    int relax = !use_bias;
    int c0 = 0;
    if (row0 && have0) {
        if (deltas) crow_deltas(L, row0);
        crow_solve(L, 0, *row0, inv_h, contact_speed, use_bias);
        c0 = 1;
        if (cc == 1) return;
    }
    CHead h = rhead_load(L, c0);
    CRow cur, nxt, nx2;
    crow_load<true>(L, c0, h, relax, &cur);
    crow_masses<true>(L, c0, &cur, cs, ss);
    if (cc > c0 + 1) {
        h = rhead_load(L, c0 + 1);
        crow_load<true>(L, c0 + 1, h, relax, &nxt);
        crow_masses<true>(L, c0 + 1, &nxt, cs, ss);
    }
    CHead h2 = h;
    if (cc > c0 + 2) h2 = rhead_load(L, c0 + 2);
    for (int c = c0; c < cc; c++) {
        CHead h3 = h2;
        if (c + 3 < cc) h3 = rhead_load(L, c + 3);
        if (c + 2 < cc) {
            crow_load<true>(L, c + 2, h2, relax, &nx2);
            crow_masses<true>(L, c + 2, &nx2, cs, ss);
        }
        crow_solve(L, c, cur, inv_h, contact_speed, use_bias);
        cur = nxt;
        nxt = nx2;
        h2 = h3;
    }
}

/* Contact 0's row, loaded once for the whole step (every field, masses
 * included); 0 when the lane has no contact.  A step whose worlds have at
 * most two shapes (one candidate pair, so at most one contact) keeps it for
 * the step, in registers or, where the kernel's registers are full, in the
 * lane's private memory: each sweep then waits on no head load, and loads
 * its bodies' delta poses only after a position update. */
B3D_FN int kept_row(const Lane& L, Soft cs, Soft ss, CRow* row) {
    if (contact_count_word(L) <= 0) return 0;
    CHead h = rhead_load(L, 0);
    crow_load<true>(L, 0, h, 1, row);
    crow_masses<true>(L, 0, row, cs, ss);
    return 1;
}
/* The kept row's normal impulses after restitution, which writes them. */
B3D_FN void kept_row_impulses(const Lane& L, CRow* row) {
    const uint32_t* rc = crec(L, 0, row->slot);
#pragma unroll
    for (int p = 0; p < kMaxManifold; p++)
        if (p < row->pc) row->pt[p].ni = qf(rc, R_NI + 2 * p);
}

/* One sweep of a shared-narrowphase tile: level by level, each of the
 * tile's waves solving every waves-th contact of the level (in contact
 * order), a workgroup barrier after each level and one before the first,
 * which also publishes wave 0's velocity updates since the last sweep.
 * Every wave runs 1 + nlev barriers (nlev from tile_levels). */
B3D_FN void solve_contacts_leveled(const Lane& L, float inv_h, float contact_speed, int use_bias, Soft cs, Soft ss,
        int nlev) {
    const PairStage& S = L.st;
    int relax = !use_bias;
    int mine = sch_get(L, 0);
    B3D_BARRIER();
    int first = 0;
    for (int lev = 1; lev <= nlev; lev++) {
        if (lev <= mine) {
            int end = sch_get(L, sch_p(L, lev));
            /* the entry of the next contact is in flight during a solve */
            int cn = 0, en = 0;
            if (first + S.wave < end) {
                const uint32_t* ep = sch_entry(L, first + S.wave);
                cn = ldi(ep, 0);
                en = ldi(ep, 1);
            }
            for (int i = first + S.wave; i < end; i += S.waves) {
                int c = cn, e = en;
                if (i + S.waves < end) {
                    const uint32_t* ep = sch_entry(L, i + S.waves);
                    cn = ldi(ep, 0);
                    en = ldi(ep, 1);
                }
                int ps[kMaxManifold];
#pragma unroll
                for (int p = 0; p < kMaxManifold; p++) ps[p] = (e >> (6 + 6 * p)) & 63;
                CHead h = rhead_at(L, c, e & 63);
                CRow r;
                crow_load<false>(L, c, h, relax, &r, ps);
                crow_masses<false>(L, c, &r, cs, ss);
                crow_solve(L, c, r, inv_h, contact_speed, use_bias);
            }
            first = end;
        }
        B3D_BARRIER();
    }
}

/* A wave's walk over its entries of a levelled contact pass: entries
 * first + wave, first + wave + waves, ... of each level [first, end) in
 * turn, among the lane's own `mine` levels.  The current entry comes with
 * its head, and the next entry is in flight: the entries (in the stage) and
 * the heads do not change during a pass, so they are loaded an item ahead,
 * across the level barriers. */
struct CWalk {
    int i, lev, c, e;      /* the current entry (i < 0: none left): its index,
                              level, contact and record slots */
    CHead h;
    int i1, lev1, c1, e1;  /* the next entry */
};
/* The wave's next entry after entry i of level *lev, or -1. */
B3D_FN int clevel_next(const Lane& L, int i, int* lev, int mine) {
    const PairStage& S = L.st;
    int end = sch_get(L, sch_p(L, *lev));
    if (i + S.waves < end) return i + S.waves;
    for (int l = *lev + 1; l <= mine; l++) {
        int start = end;
        end = sch_get(L, sch_p(L, l));
        if (start + S.wave < end) {
            *lev = l;
            return start + S.wave;
        }
    }
    return -1;
}
B3D_FN void centry_load(const Lane& L, int i, int* c, int* e) {
    *c = 0;
    *e = 0;
    if (i < 0) return;
    const uint32_t* ep = sch_entry(L, i);
    *c = ldi(ep, 0);
    *e = ldi(ep, 1);
}
/* The walk at entry i of level lev (contact c, slots e): its head, and the
 * next entry. */
B3D_FN CWalk cwalk_at(const Lane& L, int i, int lev, int c, int e, int mine) {
    CWalk w;
    w.i = i;
    w.lev = lev;
    w.c = c;
    w.e = e;
    w.h = head_of(0u, 0u);
    if (i >= 0) w.h = rhead_at(L, c, e & 63);
    w.lev1 = lev;
    w.i1 = i >= 0 ? clevel_next(L, i, &w.lev1, mine) : -1;
    centry_load(L, w.i1, &w.c1, &w.e1);
    return w;
}
B3D_FN CWalk cwalk_start(const Lane& L, int mine) {
    const PairStage& S = L.st;
    int lev = 1, i = -1, c, e;
    if (mine >= 1) i = S.wave < sch_get(L, sch_p(L, 1)) ? S.wave : clevel_next(L, S.wave - S.waves, &lev, mine);
    centry_load(L, i, &c, &e);
    return cwalk_at(L, i, lev, c, e, mine);
}

/* b3_warm_start (08:194-232) for a shared tile: each contact's impulses
 * as warm_start_contacts applies them, level by level like the sweeps
 * (1 + nlev barriers).  An item's row loads with the next item's head and
 * the entry after it (the walk), before its impulses are applied. */
B3D_FN void warm_contacts_leveled(const Lane& L, int nlev) {
    int mine = sch_get(L, 0);
    CWalk w = cwalk_start(L, mine);
    B3D_BARRIER();
    for (int l = 1; l <= nlev; l++) {
        while (w.i >= 0 && w.lev == l) {
            int c = w.c, e = w.e;
            CHead h = w.h;
            const uint32_t* r = crec(L, c, h.slot);
            float ma, mb;
            M3 ia, ib;
            rec_masses(r, h.flags, &ma, &ia, &mb, &ib);
            V3 n = q3(r, R_N);
            V3 ra[kMaxManifold], rb[kMaxManifold];
            float ni[kMaxManifold];
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= h.pc) continue;
                const uint32_t* pr = prec(L, c, p, (e >> (6 + 6 * p)) & 63);
                ra[p] = q3(pr, PR_RA);
                rb[p] = q3(pr, PR_RB);
                ni[p] = qf(r, R_NI + 2 * p);
            }
            V3 t1 = q3(r, R_T1);
            V2 fi;
            fi.x = qf(r, R_FI);
            fi.y = qf(r, R_FI + 1);
            V3 ca = q3(r, R_CA), cb = q3(r, R_CB);
            float twist = qf(r, R_TWIST);
            V3 roll = q3(r, R_ROLL);
            CWalk nx = cwalk_at(L, w.i1, w.lev1, w.c1, w.e1, mine);
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= h.pc) continue;
                V3 P = scale(n, ni[p]);
                apply_impulse(L, h.a, ma, ia, ra[p], P, -1.0f);
                apply_impulse(L, h.b, mb, ib, rb[p], P, 1.0f);
            }
            V3 t2 = cross(t1, n);
            V3 f = add(scale(t1, fi.x), scale(t2, fi.y));
            apply_impulse(L, h.a, ma, ia, ca, f, -1.0f);
            apply_impulse(L, h.b, mb, ib, cb, f, 1.0f);
            V3 tr = add(scale(n, twist), roll);
            if (is_dyn_flag(L, h.a)) set_vang(L, h.a, sub(vang(L, h.a), mv(ia, tr)));
            if (is_dyn_flag(L, h.b)) set_vang(L, h.b, add(vang(L, h.b), mv(ib, tr)));
            w = nx;
        }
        B3D_BARRIER();
    }
}

/* b3_apply_restitution (08:439-480). */
B3D_FN void apply_restitution(const Lane& L, float threshold) {
    int cc = contact_count_word(L);
    for (int c = 0; c < cc; c++) {
        CHead hd = rhead_load(L, c);
        int ps[kMaxManifold];
#pragma unroll
        for (int p = 0; p < kMaxManifold; p++)
            if (p < hd.pc) ps[p] = wave_slot(L);
        if (!(hd.flags & CF_RESTITUTION)) continue;
        uint32_t* rw = crec(L, c, hd.slot);
        const uint32_t* r = crec(L, c, hd.slot);
        float e = qf(r, R_RESTITUTION);
        int a = hd.a, b = hd.b;
        V3 va = vlin(L, a), wa = vang(L, a), vb = vlin(L, b), wb = vang(L, b);
        V3 n = q3(r, R_N);
        float ma, mb;
        M3 ia, ib;
        rec_masses(r, hd.flags, &ma, &ia, &mb, &ib);
#pragma unroll
        for (int p = 0; p < kMaxManifold; p++) {
            if (p >= hd.pc) continue;
            const uint32_t* pr = prec(L, c, p, ps[p]);
            float rv = qf(r, R_REL_VEL + p);
            if (rv > -threshold || qf(r, R_TN + 2 * p) == 0.0f) continue;
            V3 ra = q3(pr, PR_RA), rb = q3(pr, PR_RB);
            V3 vra = add(va, cross(wa, ra));
            V3 vrb = add(vb, cross(wb, rb));
            float vn = dot(sub(vrb, vra), n);
            float old = qf(r, R_NI + 2 * p);
            float imp = -qf(pr, PR_NMASS) * (vn + e * rv);
            float nimp = maxf(old + imp, 0.0f);
            imp = nimp - old;
            qsf(rw, R_NI + 2 * p, nimp);
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

/* The impulses the sweeps and restitution accumulated, back into the
 * world's contact rows (the warm-start cache of the next step). */
B3D_FN void contact_writeback(const Lane& L, int first = 0, int stride = 1) {
    uint32_t* w = L.w;
    int cc = contact_count_word(L);
    for (int c0 = first * kChunk; c0 < cc; c0 += stride * kChunk) {
        CHead hd[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            hd[k] = rhead_load(L, c);
        }
        float ni[kChunk][kMaxManifold], tn[kChunk][kMaxManifold], tw[kChunk];
        V2 fi[kChunk];
        V3 roll[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
            const uint32_t* r = crec(L, c, hd[k].slot);
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= hd[k].pc) continue;
                ni[k][p] = qf(r, R_NI + 2 * p);
                tn[k][p] = qf(r, R_TN + 2 * p);
            }
            fi[k].x = qf(r, R_FI);
            fi[k].y = qf(r, R_FI + 1);
            tw[k] = qf(r, R_TWIST);
            if (hd[k].flags & CF_ROLLING) roll[k] = q3(r, R_ROLL);
        }
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int c = c0 + k;
            if (c >= cc) continue;
#pragma unroll
            for (int p = 0; p < kMaxManifold; p++) {
                if (p >= hd[k].pc) continue;
                stf(w, pw(L, c, p, P_NORMAL_IMPULSE), ni[k][p]);
                stf(w, pw(L, c, p, P_TOTAL_NORMAL), tn[k][p]);
            }
            stf(w, cw(L, c, C_FRICTION_IMPULSE), fi[k].x);
            stf(w, cw(L, c, C_FRICTION_IMPULSE + 1), fi[k].y);
            stf(w, cw(L, c, C_TWIST_IMPULSE), tw[k]);
            if (hd[k].flags & CF_ROLLING) st3(w, cw(L, c, C_ROLLING_IMPULSE), roll[k]);
        }
    }
}

/* A joint row as one solve needs it: the prepared constants, the delta
 * state geometry and the accumulated impulses. */
struct JHead { int a, b, info; };
struct JRow {
    int a, b, info;
    float ma, mb;
    M3 ia, ib;
    Soft soft;
    V3 ra, rb, psep, lin_imp;
    M3 pki;                 /* inverse of the point rows' mass matrix */
    /* revolute */
    V3 axis, px, py;
    V3 ia_ax, ib_ax;        /* inverse inertias times the axis */
    float kxx, kxy, kyy, kinv;   /* perpendicular rows' matrix, 1 / det or NaN */
    float axial_mass, max_torque, speed, target, lower, upper;
    Soft spring_soft;
    float tw, relx, rely;
    float spring_imp, motor_imp, lower_imp, upper_imp;
    V2 perp_imp;
    /* weld */
    float ang_hz, lin_hz;
    Soft ang_spring, lin_spring;
    V3 cv, ang_imp;
    M3 ang_mass;
};

B3D_FN JHead jhead_load(const Lane& L, int j) {
    const uint32_t* r = joint_rec(L, j);
    uint32_t ab = ldu(r, JS_AB);
    JHead h;
    h.a = (int)(ab & 0xffffu);
    h.b = (int)(ab >> 16);
    h.info = ldi(r, JS_INFO);
    return h;
}

/* Everything one solve of joint j reads.  Fields of disabled rows and the
 * masses of bodies that are not dynamic (exact zeros in the row) are not
 * loaded.  JI: the accumulated impulses from the LDS impulse row. */
template <bool JI = false>
B3D_FN void jrow_load(const Lane& L, int j, JHead h, JRow* r) {
    const uint32_t* w = L.w;
    const uint32_t* g = joint_rec(L, j);
    int f = h.info;
    r->a = h.a;
    r->b = h.b;
    r->info = f;
    r->ma = 0.0f;
    r->mb = 0.0f;
    r->ia = m3zero();
    r->ib = m3zero();
    if (f & JF_DYN_A) {
        r->ma = ldf(w, jw(L, j, J_INV_MASS_A));
        r->ia = ldm3(w, jw(L, j, J_INV_I_A));
    }
    if (f & JF_DYN_B) {
        r->mb = ldf(w, jw(L, j, J_INV_MASS_B));
        r->ib = ldm3(w, jw(L, j, J_INV_I_B));
    }
    r->soft = ldsoft(w, jw(L, j, J_SOFTNESS));
    r->ra = ld3(g, JS_RA);
    r->rb = ld3(g, JS_RB);
    r->psep = ld3(g, JS_PSEP);
    r->lin_imp = jimp_ld3<JI>(L, j, J_LINEAR_IMPULSE);
    r->pki = ldm3(g, JS_PKI);
    int fixed = f & JF_FIXED;
    if (f & JF_WELD) {
        r->lin_hz = ldf(w, jw(L, j, J_LINEAR_HERTZ));
        r->lin_spring = ldsoft(w, jw(L, j, J_LINEAR_SPRING));
        if (!fixed) {
            r->ang_hz = ldf(w, jw(L, j, J_ANGULAR_HERTZ));
            r->ang_spring = ldsoft(w, jw(L, j, J_ANGULAR_SPRING));
            r->cv = ld3(g, JS_CV);
            r->ang_imp = jimp_ld3<JI>(L, j, J_ANGULAR_IMPULSE);
            r->ang_mass = ldm3(w, jw(L, j, J_ANGULAR_MASS));
        }
        return;
    }
    if (fixed) return;
    r->px = ld3(g, JS_PX);
    r->py = ld3(g, JS_PY);
    r->kxx = ldf(g, JS_KXX);
    r->kxy = ldf(g, JS_KXY);
    r->kyy = ldf(g, JS_KYY);
    r->kinv = ldf(g, JS_KINV);
    r->relx = ldf(g, JS_RELX);
    r->rely = ldf(g, JS_RELY);
    r->perp_imp.x = jimp_ld<JI>(L, j, J_PERP_IMPULSE);
    r->perp_imp.y = jimp_ld<JI>(L, j, J_PERP_IMPULSE + 1);
    if (f & (JF_SPRING | JF_MOTOR | JF_LIMIT)) {
        r->tw = ldf(g, JS_TW);
        r->axial_mass = ldf(w, jw(L, j, J_AXIAL_MASS));
        r->axis = ld3(w, jw(L, j, J_ROTATION_AXIS));
        r->ia_ax = ld3(g, JS_IAX);
        r->ib_ax = ld3(g, JS_IBX);
    }
    if (f & (JF_SPRING | JF_MOTOR)) r->max_torque = ldf(w, jw(L, j, J_MAX_MOTOR_TORQUE));
    if (f & JF_SPRING) {
        r->target = ldf(w, jw(L, j, J_TARGET_ANGLE));
        r->spring_soft = ldsoft(w, jw(L, j, J_SPRING_SOFTNESS));
        r->spring_imp = jimp_ld<JI>(L, j, J_SPRING_IMPULSE);
    }
    if (f & JF_MOTOR) {
        r->speed = ldf(w, jw(L, j, J_MOTOR_SPEED));
        r->motor_imp = jimp_ld<JI>(L, j, J_MOTOR_IMPULSE);
    }
    if (f & (JF_MOTOR | JF_LIMIT)) {
        r->lower = ldf(w, jw(L, j, J_LOWER_ANGLE));
        r->upper = ldf(w, jw(L, j, J_UPPER_ANGLE));
    }
    if (f & JF_LIMIT) {
        r->lower_imp = jimp_ld<JI>(L, j, J_LOWER_IMPULSE);
        r->upper_imp = jimp_ld<JI>(L, j, J_UPPER_IMPULSE);
    }
}

/* Joint rows in LDS (shared tiles, when they fit beside the velocity and
 * level rows): per joint, the head, the fields jrow_load reads from the
 * joint's words and the step's constants of the scratch record (fixed for
 * the step, staged once by stage_joint_rows), and the accumulated impulses,
 * which the solves update there and joint_writeback returns to the world
 * at the end of the step.  The delta-state geometry stays in the scratch
 * record (joint_geometry writes it), loaded one solve ahead.  A weld's
 * fields share the hinge fields' words. */
constexpr int JL_AB = 0, JL_INFO = 1, JL_MA = 2, JL_IA = 3, JL_MB = 12, JL_IB = 13, JL_SOFT = 22, JL_LIN_IMP = 25,
              JL_AXIAL = 28, JL_AXIS = 29, JL_IAX = 32, JL_IBX = 35, JL_MAXT = 38, JL_TARGET = 39, JL_SSOFT = 40,
              JL_SPEED = 43, JL_LOWER = 44, JL_UPPER = 45, JL_PERP_IMP = 46, JL_SPRING_IMP = 48, JL_MOTOR_IMP = 49,
              JL_LOWER_IMP = 50, JL_UPPER_IMP = 51,
              JL_LIN_HZ = 28, JL_LIN_SPRING = 29, JL_ANG_HZ = 32, JL_ANG_SPRING = 33, JL_ANG_MASS = 36,
              JL_ANG_IMP = 45, kJLWords = 52;
/* LDS words per lane that a shared tile may use (160 KB over 64 lanes). */
constexpr int kSharedLdsWordsMax = 640;
B3D_FN int joint_lds_word(const Geometry& g) { return lds_rows(g) + sched_words(g); }
/* Past the rows, the joint levels (joint_sched_build): the lane's level
 * count, per level one past its last entry, the entries (joint numbers) in
 * level order, and each body's last level. */
static_assert(kJointIters == kRelaxIters, "one joint schedule serves both passes");
B3D_FN int jsched_words(const Geometry& g) { return 1 + 2 * kJointIters * g.max_j + g.max_b; }
B3D_FN int joint_lds_words(const Geometry& g) { return g.max_j * kJLWords + jsched_words(g); }
B3D_FN bool joint_rows_fit(const Geometry& g) {
    return g.max_j > 0 && joint_lds_word(g) + joint_lds_words(g) <= kSharedLdsWordsMax;
}
B3D_FN float* jl_rec(const Lane& L, int j) { return L.jl + j * kJLWords * kLanes; }
/* An accumulated impulse of joint j: to the LDS row (JL), the LDS impulse
 * row (JI) or the joint's words. */
template <bool JL, bool JI = false>
B3D_FN void jimp_store(const Lane& L, int j, int world_word, int lds_word, float v) {
    if constexpr (JL) jlsf(jl_rec(L, j), lds_word, v);
    else if constexpr (JI) jlsf(ji_rec(L, j), ji_of(world_word), v);
    else stf(L.w, jw(L, j, world_word), v);
}
template <bool JL, bool JI = false>
B3D_FN void jimp_store3(const Lane& L, int j, int world_word, int lds_word, V3 v) {
    if constexpr (JL) jls3(jl_rec(L, j), lds_word, v);
    else if constexpr (JI) jls3(ji_rec(L, j), ji_of(world_word), v);
    else st3(L.w, jw(L, j, world_word), v);
}
/* The LDS impulses back to the joints' words: those the solves update (a
 * disabled row's impulse keeps the world's own value). */
B3D_FN void joint_impulse_writeback(const Lane& L) {
    int nj = joint_count(L);
    uint32_t* w = L.w;
    for (int j = 0; j < nj; j++) {
        const float* q = ji_rec(L, j);
        int info = ldi(joint_rec(L, j), JS_INFO);
        st3(w, jw(L, j, J_LINEAR_IMPULSE), jl3(q, JI_LIN));
        if (info & JF_FIXED) continue;
        if (info & JF_WELD) {
            st3(w, jw(L, j, J_ANGULAR_IMPULSE), jl3(q, JI_ANG));
            continue;
        }
        stf(w, jw(L, j, J_PERP_IMPULSE), jlf(q, JI_PERP));
        stf(w, jw(L, j, J_PERP_IMPULSE + 1), jlf(q, JI_PERP + 1));
        if (info & JF_SPRING) stf(w, jw(L, j, J_SPRING_IMPULSE), jlf(q, JI_SPRING));
        if (info & JF_MOTOR) stf(w, jw(L, j, J_MOTOR_IMPULSE), jlf(q, JI_MOTOR));
        if (info & JF_LIMIT) {
            stf(w, jw(L, j, J_LOWER_IMPULSE), jlf(q, JI_LOWER));
            stf(w, jw(L, j, J_UPPER_IMPULSE), jlf(q, JI_UPPER));
        }
    }
}

/* The step's joint rows to LDS (wave 0, after prepare_joints): each row as
 * jrow_load reads it, less the delta-state geometry. */
B3D_FN void jl_stage_row(const Lane& L, int j, const JRow& r) {
    float* q = jl_rec(L, j);
    jlsf(q, JL_AB, __builtin_bit_cast(float, (uint32_t)(r.a | (r.b << 16))));
    jlsf(q, JL_INFO, __builtin_bit_cast(float, r.info));
    jlsf(q, JL_MA, r.ma);
    jlsm3(q, JL_IA, r.ia);
    jlsf(q, JL_MB, r.mb);
    jlsm3(q, JL_IB, r.ib);
    jlssoft(q, JL_SOFT, r.soft);
    jls3(q, JL_LIN_IMP, r.lin_imp);
    if (r.info & JF_WELD) {
        jlsf(q, JL_LIN_HZ, r.lin_hz);
        jlssoft(q, JL_LIN_SPRING, r.lin_spring);
        jlsf(q, JL_ANG_HZ, r.ang_hz);
        jlssoft(q, JL_ANG_SPRING, r.ang_spring);
        jlsm3(q, JL_ANG_MASS, r.ang_mass);
        jls3(q, JL_ANG_IMP, r.ang_imp);
    } else {
        jlsf(q, JL_AXIAL, r.axial_mass);
        jls3(q, JL_AXIS, r.axis);
        jls3(q, JL_IAX, r.ia_ax);
        jls3(q, JL_IBX, r.ib_ax);
        jlsf(q, JL_MAXT, r.max_torque);
        jlsf(q, JL_TARGET, r.target);
        jlssoft(q, JL_SSOFT, r.spring_soft);
        jlsf(q, JL_SPEED, r.speed);
        jlsf(q, JL_LOWER, r.lower);
        jlsf(q, JL_UPPER, r.upper);
        jlsf(q, JL_PERP_IMP, r.perp_imp.x);
        jlsf(q, JL_PERP_IMP + 1, r.perp_imp.y);
        jlsf(q, JL_SPRING_IMP, r.spring_imp);
        jlsf(q, JL_MOTOR_IMP, r.motor_imp);
        jlsf(q, JL_LOWER_IMP, r.lower_imp);
        jlsf(q, JL_UPPER_IMP, r.upper_imp);
    }
}
/* Two joints at a time: both rows' loads in flight before either is staged;
 * pairs first, first + stride, ... (a shared tile's waves split them). */
B3D_FN void stage_joint_rows(const Lane& L, int first = 0, int stride = 1) {
    int nj = joint_count(L);
    for (int j0 = 2 * first; j0 < nj; j0 += 2 * stride) {
        JHead hd[2];
#pragma unroll
        for (int k = 0; k < 2; k++)
            if (j0 + k < nj) hd[k] = jhead_load(L, j0 + k);
        JRow r[2] = {};
#pragma unroll
        for (int k = 0; k < 2; k++)
            if (j0 + k < nj) jrow_load(L, j0 + k, hd[k], &r[k]);
#pragma unroll
        for (int k = 0; k < 2; k++)
            if (j0 + k < nj) jl_stage_row(L, j0 + k, r[k]);
    }
}

/* The LDS rows' impulses back to the joints' words (the words the solves
 * update; a disabled row's impulse is the world's own value, unchanged). */
B3D_FN void joint_writeback(const Lane& L, int first = 0, int stride = 1) {
    int nj = joint_count(L);
    uint32_t* w = L.w;
    for (int j = first; j < nj; j += stride) {
        const float* q = jl_rec(L, j);
        int info = __builtin_bit_cast(int, jlf(q, JL_INFO));
        st3(w, jw(L, j, J_LINEAR_IMPULSE), jl3(q, JL_LIN_IMP));
        if (info & JF_FIXED) continue;
        if (info & JF_WELD) {
            st3(w, jw(L, j, J_ANGULAR_IMPULSE), jl3(q, JL_ANG_IMP));
            continue;
        }
        stf(w, jw(L, j, J_PERP_IMPULSE), jlf(q, JL_PERP_IMP));
        stf(w, jw(L, j, J_PERP_IMPULSE + 1), jlf(q, JL_PERP_IMP + 1));
        if (info & JF_SPRING) stf(w, jw(L, j, J_SPRING_IMPULSE), jlf(q, JL_SPRING_IMP));
        if (info & JF_MOTOR) stf(w, jw(L, j, J_MOTOR_IMPULSE), jlf(q, JL_MOTOR_IMP));
        if (info & JF_LIMIT) {
            stf(w, jw(L, j, J_LOWER_IMPULSE), jlf(q, JL_LOWER_IMP));
            stf(w, jw(L, j, J_UPPER_IMPULSE), jlf(q, JL_UPPER_IMP));
        }
    }
}

/* Joint levels of a shared tile with LDS joint rows: a pass's solves
 * (joint t % nj for t < kJointIters * nj) each read and write the
 * velocities of their dynamic bodies and their own row, so level 1 + the
 * highest level among earlier solves on the same dynamic bodies keeps each
 * body's and each row's sequence of updates in pass order, and the solves
 * of one level are split among the tile's waves.  Both passes of a substep
 * share the schedule, built once per step by wave 0 from the joints' heads
 * (after prepare_joints). */
B3D_FN float* jsched(const Lane& L) { return L.jl + L.g.max_j * kJLWords * kLanes; }
B3D_FN int jsch_get(const Lane& L, int k) { return __builtin_bit_cast(int, jsched(L)[k * kLanes]); }
B3D_FN void jsch_set(const Lane& L, int k, int v) { jsched(L)[k * kLanes] = __builtin_bit_cast(float, v); }
B3D_FN int jsch_p(const Lane& L, int lev) { return lev; }                     /* lev >= 1 */
B3D_FN int jsch_entry(const Lane& L, int i) { return 1 + kJointIters * L.g.max_j + i; }
B3D_FN int jsch_last(const Lane& L, int b) { return 1 + 2 * kJointIters * L.g.max_j + b; }
/* Level of each solve of the pass, in pass order: count (place = 0) or,
 * from the level starts in P, place the entries. */
B3D_FN int joint_levels_scan(const Lane& L, int nj, int nb, int place) {
    int total = kJointIters * nj;
    for (int b = 0; b < nb; b++) jsch_set(L, jsch_last(L, b), 0);
    int nlev = 0;
    int j = 0;
    /* the first kJointKeyRegs joints' heads in registers, loaded together
     * ahead of the LDS writes (which the compiler would not move loads
     * across) */
    uint32_t abr[kJointKeyRegs];
#pragma unroll
    for (int k = 0; k < kJointKeyRegs; k++) abr[k] = k < nj ? ldu(joint_rec(L, k), JS_AB) : 0u;
    for (int t = 0; t < total; t++) {
        uint32_t ab = abr[0];
        if (j < kJointKeyRegs) {
#pragma unroll
            for (int k = 1; k < kJointKeyRegs; k++)
                if (j == k) ab = abr[k];
        } else {
            ab = ldu(joint_rec(L, j), JS_AB);
        }
        int a = (int)(ab & 0xffffu), b = (int)(ab >> 16);
        bool da = is_dyn_flag(L, a), db = is_dyn_flag(L, b);
        int la = da ? jsch_get(L, jsch_last(L, a)) : 0;
        int lb = db ? jsch_get(L, jsch_last(L, b)) : 0;
        int lev = (la > lb ? la : lb) + 1;
        if (da) jsch_set(L, jsch_last(L, a), lev);
        if (db) jsch_set(L, jsch_last(L, b), lev);
        int at = jsch_get(L, jsch_p(L, lev));
        jsch_set(L, jsch_p(L, lev), at + 1);
        if (place) jsch_set(L, jsch_entry(L, at), j);
        if (lev > nlev) nlev = lev;
        j = j + 1 == nj ? 0 : j + 1;
    }
    return nlev;
}
B3D_FN void joint_sched_build(const Lane& L) {
    int nj = joint_count(L);
    int nb = body_count(L);
    int total = kJointIters * nj;
    for (int lev = 1; lev <= total; lev++) jsch_set(L, jsch_p(L, lev), 0);
    int nlev = joint_levels_scan(L, nj, nb, 0);
    jsch_set(L, 0, nlev);
    int run = 0;
    for (int lev = 1; lev <= nlev; lev++) {
        int n = jsch_get(L, jsch_p(L, lev));
        jsch_set(L, jsch_p(L, lev), run);
        run += n;
    }
    joint_levels_scan(L, nj, nb, 1);
}
/* The tile's largest joint level count (every wave gets the same value). */
B3D_FN int tile_joint_levels(const Lane& L) {
    int v = jsch_get(L, 0), m = 0;
    for (int bit = 7; bit >= 0; bit--) {
        int cand = m | (1 << bit);
        if (wave_any(L, v >= cand)) m = cand;
    }
    return m;
}
/* The wave's next entry after entry i of level *lev (i + waves while in
 * that level, else its first entry of the next level that has one), or -1. */
B3D_FN int jlevel_next(const Lane& L, int i, int* lev, int mine) {
    const PairStage& S = L.st;
    int end = jsch_get(L, jsch_p(L, *lev));
    if (i + S.waves < end) return i + S.waves;
    for (int l = *lev + 1; l <= mine; l++) {
        int start = end;
        end = jsch_get(L, jsch_p(L, l));
        if (start + S.wave < end) {
            *lev = l;
            return start + S.wave;
        }
    }
    return -1;
}

/* A row's delta-state geometry from the scratch record (every field, in
 * one batch of loads), and the rest of the row from its LDS row. */
struct JGeo { V3 ra, rb, psep, px, py, cv; M3 pki; float kxx, kxy, kyy, kinv, relx, rely, tw; };
B3D_FN JGeo jgeo_load(const Lane& L, int j) {
    const uint32_t* g = joint_rec(L, j);
    JGeo o;
    o.tw = ldf(g, JS_TW);
    o.relx = ldf(g, JS_RELX);
    o.rely = ldf(g, JS_RELY);
    o.px = ld3(g, JS_PX);
    o.py = ld3(g, JS_PY);
    o.ra = ld3(g, JS_RA);
    o.rb = ld3(g, JS_RB);
    o.psep = ld3(g, JS_PSEP);
    o.cv = ld3(g, JS_CV);
    o.pki = ldm3(g, JS_PKI);
    o.kxx = ldf(g, JS_KXX);
    o.kxy = ldf(g, JS_KXY);
    o.kyy = ldf(g, JS_KYY);
    o.kinv = ldf(g, JS_KINV);
    return o;
}
B3D_FN void jrow_lds(const Lane& L, int j, const JGeo& g, JRow* r) {
    const float* q = jl_rec(L, j);
    uint32_t ab = __builtin_bit_cast(uint32_t, jlf(q, JL_AB));
    r->a = (int)(ab & 0xffffu);
    r->b = (int)(ab >> 16);
    r->info = __builtin_bit_cast(int, jlf(q, JL_INFO));
    r->ma = jlf(q, JL_MA);
    r->ia = jlm3(q, JL_IA);
    r->mb = jlf(q, JL_MB);
    r->ib = jlm3(q, JL_IB);
    r->soft = jlsoft(q, JL_SOFT);
    r->lin_imp = jl3(q, JL_LIN_IMP);
    r->ra = g.ra;
    r->rb = g.rb;
    r->psep = g.psep;
    r->pki = g.pki;
    if (r->info & JF_WELD) {
        r->lin_hz = jlf(q, JL_LIN_HZ);
        r->lin_spring = jlsoft(q, JL_LIN_SPRING);
        r->ang_hz = jlf(q, JL_ANG_HZ);
        r->ang_spring = jlsoft(q, JL_ANG_SPRING);
        r->ang_mass = jlm3(q, JL_ANG_MASS);
        r->ang_imp = jl3(q, JL_ANG_IMP);
        r->cv = g.cv;
        return;
    }
    r->axial_mass = jlf(q, JL_AXIAL);
    r->axis = jl3(q, JL_AXIS);
    r->ia_ax = jl3(q, JL_IAX);
    r->ib_ax = jl3(q, JL_IBX);
    r->max_torque = jlf(q, JL_MAXT);
    r->target = jlf(q, JL_TARGET);
    r->spring_soft = jlsoft(q, JL_SSOFT);
    r->speed = jlf(q, JL_SPEED);
    r->lower = jlf(q, JL_LOWER);
    r->upper = jlf(q, JL_UPPER);
    r->perp_imp.x = jlf(q, JL_PERP_IMP);
    r->perp_imp.y = jlf(q, JL_PERP_IMP + 1);
    r->spring_imp = jlf(q, JL_SPRING_IMP);
    r->motor_imp = jlf(q, JL_MOTOR_IMP);
    r->lower_imp = jlf(q, JL_LOWER_IMP);
    r->upper_imp = jlf(q, JL_UPPER_IMP);
    r->px = g.px;
    r->py = g.py;
    r->kxx = g.kxx;
    r->kxy = g.kxy;
    r->kyy = g.kyy;
    r->kinv = g.kinv;
    r->relx = g.relx;
    r->rely = g.rely;
    r->tw = g.tw;
}

/* Point rows shared by weld and revolute (06:257-282), with the anchors,
 * separation and inverted mass of the current delta state. */
template <bool JL, bool JI = false>
B3D_FN void solve_point(const Lane& L, int j, const JRow& r, V3* va, V3* wa, V3* vb, V3* wb, Soft soft,
        int use_bias) {
    V3 cdot = sub(add(*vb, cross(*wb, r.rb)), add(*va, cross(*wa, r.ra)));
    V3 bias = zero3();
    float mscale = 1.0f, iscale = 0.0f;
    if (use_bias) {
        bias = scale(r.psep, soft.bias_rate);
        mscale = soft.mass_scale;
        iscale = soft.impulse_scale;
    }
    /* b3_solve3 of the point mass (06:241-255, 03_math.inl:343-345), its
     * inverse taken once per delta state (joint_geometry) */
    V3 bsol = mv(r.pki, add(cdot, bias));
    V3 impulse = msub(scale(bsol, -mscale), iscale, r.lin_imp);
    jimp_store3<JL, JI>(L, j, J_LINEAR_IMPULSE, JL_LIN_IMP, add(r.lin_imp, impulse));
    *va = msub(*va, r.ma, impulse);
    *wa = sub(*wa, mv(r.ia, cross(r.ra, impulse)));
    *vb = madd(*vb, r.mb, impulse);
    *wb = add(*wb, mv(r.ib, cross(r.rb, impulse)));
}

/* b3_solve_weld (06:285-332). */
template <bool JL, bool JI = false>
B3D_FN void solve_weld(const Lane& L, int j, const JRow& r, int use_bias) {
    V3 va = vlin(L, r.a), wa = vang(L, r.a), vb = vlin(L, r.b), wb = vang(L, r.b);
    if (!(r.info & JF_FIXED)) {
        V3 bias = zero3();
        float mscale = 1.0f, iscale = 0.0f;
        if (use_bias || r.ang_hz > 0.0f) {
            bias = scale(r.cv, r.ang_spring.bias_rate);
            mscale = r.ang_spring.mass_scale;
            iscale = r.ang_spring.impulse_scale;
        }
        V3 cdot = sub(wb, wa);
        V3 impulse = msub(scale(mv(r.ang_mass, add(cdot, bias)), -mscale), iscale, r.ang_imp);
        jimp_store3<JL, JI>(L, j, J_ANGULAR_IMPULSE, JL_ANG_IMP, add(r.ang_imp, impulse));
        wa = sub(wa, mv(r.ia, impulse));
        wb = add(wb, mv(r.ib, impulse));
    }
    int lin_bias = use_bias || r.lin_hz > 0.0f;
    solve_point<JL, JI>(L, j, r, &va, &wa, &vb, &wb, r.lin_spring, lin_bias);
    if (is_dyn_flag(L, r.a)) {
        set_vlin(L, r.a, va);
        set_vang(L, r.a, wa);
    }
    if (is_dyn_flag(L, r.b)) {
        set_vlin(L, r.b, vb);
        set_vang(L, r.b, wb);
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
template <bool JL, bool JI = false>
B3D_FN void solve_revolute(const Lane& L, int j, const JRow& r, float h, float inv_h, int use_bias) {
    V3 va = vlin(L, r.a), wa = vang(L, r.a), vb = vlin(L, r.b), wb = vang(L, r.b);
    V3 axis = r.axis;
    int fixed = r.info & JF_FIXED;
    int en_spring = r.info & JF_SPRING, en_motor = r.info & JF_MOTOR, en_limit = r.info & JF_LIMIT;
    float axial_mass = r.axial_mass;
    float tw = r.tw;
    /* mv(ia, axis), mv(ib, axis) of the step (prepare_joints) */
    const V3 ia_ax = r.ia_ax, ib_ax = r.ib_ax;
    if (en_spring && !fixed) {
        Soft ss = r.spring_soft;
        float c = tw - r.target;
        float bias = ss.bias_rate * c;
        float cdot = dot(sub(wb, wa), axis);
        float old = r.spring_imp;
        float dimp = -ss.mass_scale * axial_mass * (cdot + bias) - ss.impulse_scale * old;
        float nimp = old + dimp;
        if (r.max_torque > 0.0f) {
            float maxp = r.max_torque * h;
            nimp = clampf(nimp, -maxp, maxp);
        }
        dimp = nimp - old;
        jimp_store<JL, JI>(L, j, J_SPRING_IMPULSE, JL_SPRING_IMP, nimp);
        wa = msub(wa, dimp, ia_ax);
        wb = madd(wb, dimp, ib_ax);
    }
    if (en_motor && !fixed) {
        int blocked = 0;
        if (en_limit) {
            if (tw >= r.upper - 0.01f && r.speed > 0.0f) blocked = 1;
            if (tw <= r.lower + 0.01f && r.speed < 0.0f) blocked = 1;
        }
        if (blocked) {
            jimp_store<JL, JI>(L, j, J_MOTOR_IMPULSE, JL_MOTOR_IMP, 0.0f);
        } else {
            float old = r.motor_imp;
            float cdot = dot(sub(wb, wa), axis) - r.speed;
            float dimp = -axial_mass * cdot;
            float nimp = old + dimp;
            float maxp = r.max_torque * h;
            nimp = clampf(nimp, -maxp, maxp);
            dimp = nimp - old;
            jimp_store<JL, JI>(L, j, J_MOTOR_IMPULSE, JL_MOTOR_IMP, nimp);
            wa = msub(wa, dimp, ia_ax);
            wb = madd(wb, dimp, ib_ax);
        }
    }
    if (en_limit && !fixed) {
        float old = r.lower_imp;
        float lo = limit_impulse(tw - r.lower, dot(sub(wb, wa), axis), inv_h, use_bias, r.soft, axial_mass, old);
        jimp_store<JL, JI>(L, j, J_LOWER_IMPULSE, JL_LOWER_IMP, lo);
        float dimp = lo - old;
        wa = msub(wa, dimp, ia_ax);
        wb = madd(wb, dimp, ib_ax);
        old = r.upper_imp;
        float up = limit_impulse(r.upper - tw, dot(sub(wa, wb), axis), inv_h, use_bias, r.soft, axial_mass, old);
        jimp_store<JL, JI>(L, j, J_UPPER_IMPULSE, JL_UPPER_IMP, up);
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
            bias.x = r.soft.bias_rate * r.relx;
            bias.y = r.soft.bias_rate * r.rely;
            mscale = r.soft.mass_scale;
            iscale = r.soft.impulse_scale;
        }
        V3 wrel = sub(wb, wa);
        V2 rhs;
        rhs.x = dot(wrel, r.px) + bias.x;
        rhs.y = dot(wrel, r.py) + bias.y;
        /* b3_solve2 (03_math.inl:347-359) with the matrix and the reciprocal
         * determinant of the delta state (joint_geometry) */
        V2 sol;
        sol.x = 0.0f;
        sol.y = 0.0f;
        if (r.kinv == r.kinv) {
            sol.x = r.kinv * (r.kyy * rhs.x - r.kxy * rhs.y);
            sol.y = r.kinv * (-r.kxy * rhs.x + r.kxx * rhs.y);
        }
        V2 dimp;
        dimp.x = -mscale * sol.x - iscale * r.perp_imp.x;
        dimp.y = -mscale * sol.y - iscale * r.perp_imp.y;
        jimp_store<JL, JI>(L, j, J_PERP_IMPULSE, JL_PERP_IMP, r.perp_imp.x + dimp.x);
        jimp_store<JL, JI>(L, j, J_PERP_IMPULSE + 1, JL_PERP_IMP + 1, r.perp_imp.y + dimp.y);
        V3 ang = add(scale(r.px, dimp.x), scale(r.py, dimp.y));
        wa = sub(wa, mv(r.ia, ang));
        wb = add(wb, mv(r.ib, ang));
    }
    solve_point<JL, JI>(L, j, r, &va, &wa, &vb, &wb, r.soft, use_bias);
    if (is_dyn_flag(L, r.a)) {
        set_vlin(L, r.a, va);
        set_vang(L, r.a, wa);
    }
    if (is_dyn_flag(L, r.b)) {
        set_vlin(L, r.b, vb);
        set_vang(L, r.b, wb);
    }
}

/* b3_solve_joints_global (07_packed.inl:48-81): sweeps in joint order; all
 * of a joint's row is requested before its rows are solved.  The row is
 * loaded right before its solve, with its head (the bodies and flags that
 * select which fields to load) fetched one solve ahead: a second row in
 * flight during a solve costs more in registers than the one round trip it
 * would hide. */
template <bool JI = false>
B3D_FN void solve_joints(const Lane& L, float h, float inv_h, int use_bias) {
    int nj = joint_count(L);
    if (nj <= 0) return;
    int total = (use_bias ? kJointIters : kRelaxIters) * nj;
    JHead head = jhead_load(L, 0);
    int j = 0;
    for (int t = 0; t < total; t++) {
        JRow cur;
        jrow_load<JI>(L, j, head, &cur);
        int jn = j + 1 == nj ? 0 : j + 1;
        if (t + 1 < total) head = jhead_load(L, jn);
        if (cur.info & JF_WELD) solve_weld<false, JI>(L, j, cur, use_bias);
        else solve_revolute<false, JI>(L, j, cur, h, inv_h, use_bias);
        j = jn;
    }
}

/* A joint pass of a shared tile with LDS joint rows, split by joint levels
 * among its waves (every wave calls it, with the tile's level count): each
 * wave solves its share of each level, a barrier after every level, with
 * the geometry of its next solve in flight. */
B3D_FN void solve_joints_leveled(const Lane& L, float h, float inv_h, int use_bias, int nlev) {
    const PairStage& S = L.st;
    int mine = jsch_get(L, 0);
    int lev = 1, i = -1;
    if (mine >= 1) i = S.wave < jsch_get(L, jsch_p(L, 1)) ? S.wave : jlevel_next(L, S.wave - S.waves, &lev, mine);
    JGeo g;
    if (i >= 0) g = jgeo_load(L, jsch_get(L, jsch_entry(L, i)));
    for (int l = 1; l <= nlev; l++) {
        while (i >= 0 && lev == l) {
            int j = jsch_get(L, jsch_entry(L, i));
            JRow cur;
            jrow_lds(L, j, g, &cur);
            int lev1 = lev;
            int i1 = jlevel_next(L, i, &lev1, mine);
            if (i1 >= 0) g = jgeo_load(L, jsch_get(L, jsch_entry(L, i1)));
            if (cur.info & JF_WELD) solve_weld<true>(L, j, cur, use_bias);
            else solve_revolute<true>(L, j, cur, h, inv_h, use_bias);
            i = i1;
            lev = lev1;
        }
        B3D_BARRIER();
    }
}

/* Per-step body records: the velocity increments of gravity and the
 * applied force / torque and the damping factors of 09_step.inl:5-18, whose
 * inputs do not change during a step (BS_*), and the body kind and the
 * step's starting delta pose (BD_*). */
B3D_FN void body_prepass(const Lane& L, float h, int first = 0, int stride = 1) {
    uint32_t* w = L.w;
    V3 g = ld3(w, H_GRAVITY);
    int nb = body_count(L);
    for (int b0 = first * kChunk; b0 < nb; b0 += stride * kChunk) {
        /* the chunk's velocities go to the LDS rows in the same pass (one
         * round trip per chunk for both) */
        float vel[kChunk][6];
        int type[kChunk];
        uint32_t flags[kChunk];
        float inv_mass[kChunk], lin_d[kChunk], ang_d[kChunk], gscale[kChunk];
        V3 force[kChunk], torque[kChunk], dp[kChunk];
        M3 iw[kChunk];
        Q dq[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k;
            if (b >= nb) continue;
#pragma unroll
            for (int c = 0; c < 6; c++) vel[k][c] = ldf(w, bw(L, b, B_LIN_VEL + c));
            dp[k] = ld3(w, bw(L, b, B_DELTA_POS));
            dq[k] = ldq(w, bw(L, b, B_DELTA_ROT));
            type[k] = ldi(w, bw(L, b, B_TYPE));
            flags[k] = ldu(w, bw(L, b, B_FLAGS));
            inv_mass[k] = ldf(w, bw(L, b, B_INV_MASS));
            lin_d[k] = ldf(w, bw(L, b, B_LINEAR_DAMPING));
            ang_d[k] = ldf(w, bw(L, b, B_ANGULAR_DAMPING));
            gscale[k] = ldf(w, bw(L, b, B_GRAVITY_SCALE));
            force[k] = ld3(w, bw(L, b, B_FORCE));
            torque[k] = ld3(w, bw(L, b, B_TORQUE));
            iw[k] = ldm3(w, bw(L, b, B_INV_I_WORLD));
        }
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k;
            if (b >= nb) continue;
            float* row = L.vel + b * kVelWords * kLanes;
#pragma unroll
            for (int c = 0; c < 6; c++) row[c * kLanes] = vel[k][c];
            row[6 * kLanes] = __builtin_bit_cast(float, flags[k]);
            uint32_t* r = body_rec(L, b);
            uint32_t* d = delta_rec(L, b);
            int kind = (int)(flags[k] & 0xffu) | (type[k] == kDynamic ? kKindDynamic : 0)
                | (type[k] == kStatic ? kKindStatic : 0);
            uint32_t dbits = __builtin_bit_cast(uint32_t, dp[k].x) | __builtin_bit_cast(uint32_t, dp[k].y)
                | __builtin_bit_cast(uint32_t, dp[k].z) | __builtin_bit_cast(uint32_t, dq[k].v.x)
                | __builtin_bit_cast(uint32_t, dq[k].v.y) | __builtin_bit_cast(uint32_t, dq[k].v.z)
                | (__builtin_bit_cast(uint32_t, dq[k].s) ^ 0x3f800000u);
            uint32_t fbits = __builtin_bit_cast(uint32_t, force[k].x) | __builtin_bit_cast(uint32_t, force[k].y)
                | __builtin_bit_cast(uint32_t, force[k].z) | __builtin_bit_cast(uint32_t, torque[k].x)
                | __builtin_bit_cast(uint32_t, torque[k].y) | __builtin_bit_cast(uint32_t, torque[k].z);
            kind |= (dbits ? kKindClearDelta : 0) | (fbits ? kKindClearForce : 0);
            rs3(d, BD_DP, dp[k]);
            rsu(d, BD_KIND, (uint32_t)kind);
            rsq(d, BD_DQ, dq[k]);
            if (type[k] != kDynamic) continue;
            float gs = inv_mass[k] > 0.0f ? gscale[k] : 0.0f;
            rs3(r, BS_DV, add(scale(force[k], h * inv_mass[k]), scale(g, h * gs)));
            rsf(r, BS_LD, 1.0f / (1.0f + h * lin_d[k]));
            rs3(r, BS_DW, scale(mv(iw[k], torque[k]), h));
            rsf(r, BS_AD, 1.0f / (1.0f + h * ang_d[k]));
        }
    }
}

/* Gravity, applied force and damping for dynamic bodies (09_step.inl:5-18, 41-53). */
/* Bodies first, first + stride, ... (a shared tile's waves split them). */
B3D_FN void integrate_velocities(const Lane& L, int first = 0, int stride = 1) {
    int nb = body_count(L);
    for (int b0 = first; b0 < nb; b0 += kChunk * stride) {
        int kind[kChunk];
        V3 dv[kChunk], dw[kChunk];
        float ld[kChunk], ad[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k * stride;
            if (b >= nb) continue;
            const uint32_t* r = body_rec(L, b);
            kind[k] = (int)ru(delta_rec(L, b), BD_KIND);
            dv[k] = r3(r, BS_DV);
            dw[k] = r3(r, BS_DW);
            ld[k] = rf(r, BS_LD);
            ad[k] = rf(r, BS_AD);
        }
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k * stride;
            if (b >= nb || !(kind[k] & kKindDynamic)) continue;
            set_vlin(L, b, madd(dv[k], ld[k], vlin(L, b)));
            set_vang(L, b, madd(dw[k], ad[k], vang(L, b)));
        }
    }
}

/* Axis locks, speed clamps and the substep pose update (09_step.inl:55-107). */
B3D_FN void integrate_positions(const Lane& L, float h, float inv_dt, int first = 0, int stride = 1) {
    uint32_t* w = L.w;
    float max_lin = ldf(w, H_MAX_LINEAR_SPEED);
    float max_ang = kMaxRotation * inv_dt;
    float max_lin2 = max_lin * max_lin;
    float max_ang2 = max_ang * max_ang;
    int nb = body_count(L);
    for (int b0 = first; b0 < nb; b0 += kChunk * stride) {
        int kind[kChunk];
        V3 dp[kChunk];
        Q dq[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k * stride;
            if (b >= nb) continue;
            const uint32_t* d = delta_rec(L, b);
            kind[k] = (int)ru(d, BD_KIND);
            dp[k] = r3(d, BD_DP);
            dq[k] = rq4(d, BD_DQ);
        }
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k * stride;
            if (b >= nb || (kind[k] & kKindStatic)) continue;
            uint32_t flags = (uint32_t)kind[k];
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
            uint32_t* d = delta_rec(L, b);
            rs3(d, BD_DP, madd(dp[k], h, v));
            rsu(d, BD_KIND, (uint32_t)kind[k]);
            rsq(d, BD_DQ, qintegrate(dq[k], scale(av, h)));
        }
    }
}

/* Commit the accumulated deltas and clear forces (09_step.inl:109-130);
 * delta pose, force and torque words already zero (identity) are left
 * alone. */
B3D_FN void finalize(const Lane& L, int first = 0, int stride = 1) {
    uint32_t* w = L.w;
    int nb = body_count(L);
    for (int b0 = first * kChunk; b0 < nb; b0 += stride * kChunk) {
        int type[kChunk], kind[kChunk];
        V3 center[kChunk], dp[kChunk], lc[kChunk], inv_i[kChunk];
        Q dq[kChunk], rq[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k;
            if (b >= nb) continue;
            type[k] = ldi(w, bw(L, b, B_TYPE));
            center[k] = ld3(w, bw(L, b, B_CENTER));
            const uint32_t* d = delta_rec(L, b);
            kind[k] = (int)ru(d, BD_KIND);
            dp[k] = r3(d, BD_DP);
            dq[k] = rq4(d, BD_DQ);
            rq[k] = ldq(w, bw(L, b, B_ROTATION));
            lc[k] = ld3(w, bw(L, b, B_LOCAL_CENTER));
            inv_i[k] = ld3(w, bw(L, b, B_INV_INERTIA));
        }
#pragma unroll
        for (int k = 0; k < kChunk; k++) {
            int b = b0 + k;
            if (b >= nb || type[k] == kStatic) continue;
            V3 c = add(center[k], dp[k]);
            Q r = qnorm(qmul(dq[k], rq[k]));
            st3(w, bw(L, b, B_CENTER), c);
            stq(w, bw(L, b, B_ROTATION), r);
            st3(w, bw(L, b, B_POSITION), sub(c, rot(r, lc[k])));
            if (kind[k] & kKindClearDelta) {
                st3(w, bw(L, b, B_DELTA_POS), zero3());
                stq(w, bw(L, b, B_DELTA_ROT), qid());
            }
            if (kind[k] & kKindClearForce) {
                st3(w, bw(L, b, B_FORCE), zero3());
                st3(w, bw(L, b, B_TORQUE), zero3());
            }
            if (type[k] == kDynamic) stm3(w, bw(L, b, B_INV_I_WORLD), world_inv_i(r, inv_i[k]));
        }
    }
}

/* ---- per-substep force laws: the B3_USER_FORCES hook ----
 * 01_config.inl:189-198 and 09_step.inl:20-53: once per substep, before the
 * velocity update, a force law may add to each body's applied force and
 * torque; the velocity update uses the sums, and the applied force and
 * torque are back to their own values for the next substep.  A law here is
 * a type with `static constexpr bool kActive = true` and
 *     B3D_FN void operator()(const ForceView& v) const;
 * built once per world by the kernel that runs it (so it can hold that
 * world's parameters and state).  The view reads the state of the substep
 * as the reference's hook reads the world: start-of-step center, rotation
 * and position with the current delta pose (current center = center +
 * delta_pos, current rotation = delta_rot * rotation), current velocities,
 * and any other world word through `L`. */
struct ForceView {
    Lane L;
    float h;
    B3D_MFN int body_count() const { return b3d::body_count(L); }
    B3D_MFN int type(int b) const { return ldi(L.w, bw(L, b, B_TYPE)); }
    B3D_MFN float inv_mass(int b) const { return ldf(L.w, bw(L, b, B_INV_MASS)); }
    B3D_MFN V3 center(int b) const { return ld3(L.w, bw(L, b, B_CENTER)); }
    B3D_MFN V3 position(int b) const { return ld3(L.w, bw(L, b, B_POSITION)); }
    B3D_MFN Q rotation(int b) const { return ldq(L.w, bw(L, b, B_ROTATION)); }
    B3D_MFN V3 delta_pos(int b) const { return r3(delta_rec(L, b), BD_DP); }
    B3D_MFN Q delta_rot(int b) const { return rq4(delta_rec(L, b), BD_DQ); }
    B3D_MFN V3 lin_vel(int b) const { return vlin(L, b); }
    B3D_MFN V3 ang_vel(int b) const { return vang(L, b); }
    /* The force and torque the velocity update of this substep uses. */
    B3D_MFN V3 force(int b) const { return r3(body_rec(L, b), BS_DV); }
    B3D_MFN V3 torque(int b) const { return r3(body_rec(L, b), BS_DW); }
    B3D_MFN void set_force(int b, V3 f) const { rs3(body_rec(L, b), BS_DV, f); }
    B3D_MFN void set_torque(int b, V3 t) const { rs3(body_rec(L, b), BS_DW, t); }
};

/* The law of a step without a hook (B3_HAS_USER_FORCES 0). */
struct NoForces {
    static constexpr bool kActive = false;
    B3D_MFN void operator()(const ForceView&) const {}
};

/* b3_integrate_velocities with the hook (09_step.inl:5-18, 20-53): the
 * body records' force and torque words take each body's applied force and
 * torque, the law adds to them, and the update of 09_step.inl:5-18 runs on
 * the sums; the world's own force and torque words are never touched. */
template <class Law>
B3D_FN void integrate_velocities_law(const Lane& L, float h, const Law& law) {
    uint32_t* w = L.w;
    int nb = body_count(L);
    for (int b = 0; b < nb; b++) {
        uint32_t* r = body_rec(L, b);
        rs3(r, BS_DV, ld3(w, bw(L, b, B_FORCE)));
        rs3(r, BS_DW, ld3(w, bw(L, b, B_TORQUE)));
    }
    ForceView v;
    v.L = L;
    v.h = h;
    law(v);
    V3 g = ld3(w, H_GRAVITY);
    for (int b = 0; b < nb; b++) {
        if (!(ru(delta_rec(L, b), BD_KIND) & kKindDynamic)) continue;
        const uint32_t* r = body_rec(L, b);
        float inv_mass = ldf(w, bw(L, b, B_INV_MASS));
        float gs = inv_mass > 0.0f ? ldf(w, bw(L, b, B_GRAVITY_SCALE)) : 0.0f;
        V3 dv = add(scale(r3(r, BS_DV), h * inv_mass), scale(g, h * gs));
        V3 dw = scale(mv(ldm3(w, bw(L, b, B_INV_I_WORLD)), r3(r, BS_DW)), h);
        set_vlin(L, b, madd(dv, rf(r, BS_LD), vlin(L, b)));
        set_vang(L, b, madd(dw, rf(r, BS_AD), vang(L, b)));
    }
}

/* One world's b3_step (09_step.inl:148-264, default configuration), with
 * the force law `law` in the B3_USER_FORCES hook.  Body velocities are
 * staged in the velocity rows after contact generation (which uses the
 * same rows for clip polygons) and written back at the end.  JL: the joint
 * rows in LDS (shared tiles); JI: the joint impulses in LDS (one wave per
 * tile, L.ji), staged by the joint warm start and written back at the end.
 * C0: the one-wave step keeps contact 0's row for the step (kept_row;
 * worlds of at most two shapes, whose only contact it is). */
template <bool Masks = false, class Law, bool JL = false, bool JI = false, bool C0 = false>
B3D_FN void step_world(const Lane& L0, float dt, int substeps, const Law& law) {
    static_assert(!(JL && JI), "joint rows and joint impulses are two layouts of the same LDS words");
    if (!(dt > 0.0f)) return;
    Lane L = L0;
    L.sslot = wave_rank(L);
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
    /* Idle lanes (L.active false) run only in a shared tile, where every
     * lane of the workgroup reaches every barrier: the barriers sit outside
     * the `if (L.active)` blocks, in find_pairs and in the levelled warm
     * start and sweeps, which an idle lane enters with no candidates and
     * no contact levels. */
    const bool act = L.active;

    find_contacts<Masks>(L);
    count_bodies_and_joints(L);
    count_contacts(L);
    /* restitution runs in every lane of a wave where some world has it */
    const bool rest_wave = wave_any(L, act && (ldi(L.scr + L.g.scr_flags * kLanes, 0) & kLaneRestitution) != 0);
    /* a shared tile's waves split the body work (sweep_helper does its
     * share before the barrier that follows) */
    const int share = L.staged ? L.st.wave : 0, stride = L.staged ? L.st.waves : 1;
    if (act) body_prepass(L, h, share, stride);   /* with the velocity rows */
    int nlev = 0, njlev = 0;
    if (L.staged) {
        /* the tile's waves prepare the contacts and joints together (and
         * stage the joint rows, JL); wave 0 levels the contacts (and
         * joints); all warm-start the contacts level by level (the helper
         * waves meet wave 0 at each barrier, sweep_helper) */
        B3D_BARRIER();
        if (act) {
            /* wave 0 levels the contacts while the others prepare them
             * (alone, it does both) */
            sched_build(L);
            if (stride == 1) prepare_contacts(L, cs, ss);
            prepare_joints(L, h, share, stride);
        } else {
            sch_set(L, 0, 0);      /* no contact levels */
        }
        B3D_BARRIER();
        if (act) {
            if constexpr (JL) stage_joint_rows(L, share, stride);
            if constexpr (JL) joint_sched_build(L);
        } else {
            if constexpr (JL) jsch_set(L, 0, 0);
        }
        B3D_BARRIER();
        nlev = tile_levels(L);
        if constexpr (JL) njlev = tile_joint_levels(L);
        warm_contacts_leveled(L, nlev);
    } else {
        int warm_done = prepare_contacts(L, cs, ss);
        prepare_joints(L, h);
        if (wave_any(L, !warm_done)) warm_start_contacts(L, warm_done);
    }
    if (act) warm_start_joints<JI>(L);
    CRow row0;
    int have0 = 0;
    if constexpr (C0) have0 = kept_row(L, cs, ss, &row0);
    /* a shared tile's waves split the first joint geometry, after the warm
     * start has read the previous step's hinge rows, which it overwrites */
    if (L.staged) B3D_BARRIER();
    if (act) joint_geometry(L, share, stride);
    /* In a shared tile the waves split the velocity and position updates
     * (bodies) and the joint geometry (joints) of every substep, between
     * barriers: each body and joint is updated by one wave, and the next
     * phase's readers see it after the barrier (sweep_helper runs the same
     * barriers).  Wave 0 alone solves the joints and applies restitution. */
    for (int s = 0; s < subs; s++) {
        if (L.staged) B3D_BARRIER();   /* the last joint and restitution impulses */
        if (act) {
            if constexpr (Law::kActive)   /* one-wave kernels only: no tile sharing */
                integrate_velocities_law(L, h, law);
            else
                integrate_velocities(L, share, stride);
        }
        if (L.staged) solve_contacts_leveled(L, inv_h, contact_speed, 1, cs, ss, nlev);
        else solve_contacts(L, inv_h, contact_speed, 1, cs, ss, C0 ? &row0 : nullptr, have0);
        if constexpr (JL) solve_joints_leveled(L, h, inv_h, 1, njlev);
        else if (act) solve_joints<JI>(L, h, inv_h, 1);
        if (L.staged) B3D_BARRIER();   /* the joints' velocities */
        if (act) integrate_positions(L, h, inv_dt, share, stride);
        if (L.staged) B3D_BARRIER();   /* the delta poses */
        if (act) joint_geometry(L, share, stride);
        if (L.staged) solve_contacts_leveled(L, inv_h, contact_speed, 0, cs, ss, nlev);
        else solve_contacts(L, inv_h, contact_speed, 0, cs, ss, C0 ? &row0 : nullptr, have0, true);
        if constexpr (JL) solve_joints_leveled(L, h, inv_h, 0, njlev);
        if (act) {
            if constexpr (!JL) solve_joints<JI>(L, h, inv_h, 0);
            if (rest_wave) {
                apply_restitution(L, rest_threshold);
                if (have0) kept_row_impulses(L, &row0);
            }
        }
    }
    /* a shared tile's waves split the write-back, after the last
     * restitution and joint impulses (sweep_helper runs the same barrier) */
    if (L.staged) B3D_BARRIER();
    if (act) {
        contact_writeback(L, share, stride);
        if constexpr (JL) joint_writeback(L, share, stride);
        if constexpr (JI) joint_impulse_writeback(L);
        finalize(L, share, stride);
        vel_store(L, share, stride);
    }
}

/* b3_step without a hook; JL: the joint rows in LDS (L.jl, shared tiles);
 * JI: the joint impulses in LDS (L.ji, one wave per tile); C0: contact 0's
 * row kept for the step (one wave per tile). */
template <bool Masks = false, bool JL = false, bool JI = false, bool C0 = false>
B3D_FN void step_world(const Lane& L, float dt, int substeps) {
    step_world<Masks, NoForces, JL, JI, C0>(L, dt, substeps, NoForces());
}

/* A helper wave of a shared-narrowphase tile after its narrowphase share:
 * its share of the contact preparation, of the level-by-level warm start,
 * of the first joint geometry, of every contact sweep, of each substep's
 * velocity and position updates and joint geometry (and joint levels, JL),
 * and of the write-back, in step with wave 0 (the same barriers, in the
 * same order, as step_world's shared path).  Runs in all lanes; its
 * stepping lanes rank as wave 0's, so its body and delta record slots are
 * wave 0's, and its idle lanes have no contact levels (wave 0 set them). */
template <bool JL = false>
B3D_FN void sweep_helper(const Lane& L0, float dt, int substeps) {
    Lane L = L0;
    L.sslot = wave_rank(L);
    int subs = substeps < 1 ? 1 : substeps;
    float h = dt / (float)subs;
    float inv_dt = 1.0f / dt;
    float inv_h = (float)subs * inv_dt;
    float hertz = minf(ldf(L.w, H_CONTACT_HERTZ), 0.25f * inv_h);
    float damping = ldf(L.w, H_CONTACT_DAMPING);
    Soft cs = make_soft(hertz, damping, h);
    Soft ss = make_soft(2.0f * hertz, 0.5f * damping, h);
    float contact_speed = ldf(L.w, H_CONTACT_SPEED);
    count_bodies_and_joints(L);
    if (L.active) body_prepass(L, h, L.st.wave, L.st.waves);   /* with the velocity rows */
    B3D_BARRIER();                 /* the velocities and body records are staged */
    count_contacts(L);             /* wave 0 wrote the count before the barrier */
    if (L.active) {
        /* the contacts split over the waves but wave 0, which levels them */
        prepare_contacts(L, cs, ss, L.st.wave - 1, L.st.waves - 1);
        prepare_joints(L, h, L.st.wave, L.st.waves);
    }
    B3D_BARRIER();                 /* all contacts and joints prepared */
    if constexpr (JL)
        if (L.active) stage_joint_rows(L, L.st.wave, L.st.waves);
    B3D_BARRIER();                 /* wave 0 has levelled them (and the joints, JL) */
    int nlev = tile_levels(L);
    int njlev = 0;
    if constexpr (JL) njlev = tile_joint_levels(L);
    warm_contacts_leveled(L, nlev);
    B3D_BARRIER();                 /* wave 0 has warm-started the joints */
    if (L.active) joint_geometry(L, L.st.wave, L.st.waves);
    for (int s = 0; s < subs; s++) {
        B3D_BARRIER();
        if (L.active) integrate_velocities(L, L.st.wave, L.st.waves);
        solve_contacts_leveled(L, inv_h, contact_speed, 1, cs, ss, nlev);
        if constexpr (JL) solve_joints_leveled(L, h, inv_h, 1, njlev);
        B3D_BARRIER();
        if (L.active) integrate_positions(L, h, inv_dt, L.st.wave, L.st.waves);
        B3D_BARRIER();
        if (L.active) joint_geometry(L, L.st.wave, L.st.waves);
        solve_contacts_leveled(L, inv_h, contact_speed, 0, cs, ss, nlev);
        if constexpr (JL) solve_joints_leveled(L, h, inv_h, 0, njlev);
    }
    B3D_BARRIER();                 /* wave 0's restitution */
    if (L.active) {
        contact_writeback(L, L.st.wave, L.st.waves);
        if constexpr (JL) joint_writeback(L, L.st.wave, L.st.waves);
        finalize(L, L.st.wave, L.st.waves);
        vel_store(L, L.st.wave, L.st.waves);
    }
}

}  // namespace b3d

#endif
