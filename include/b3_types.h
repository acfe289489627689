/*
 * b3_types.h - plain-data world model shared by callers, the MI355X engine
 * and its checkers.
 *
 * Every struct here is byte-for-byte the layout of the reference header so
 * that a caller can hand the engine worlds built by either library:
 *   B3Body     <- src/puffysics/02_types.inl:55-74   (200 B)
 *   B3Shape    <- src/puffysics/02_types.inl:76-89   (88 B)
 *   B3Point    <- src/puffysics/02_types.inl:91-101  (52 B)
 *   B3Contact  <- src/puffysics/02_types.inl:103-131 (476 B)
 *   B3Joint    <- src/puffysics/02_types.inl:144-218 (460 B, default flags)
 *   B3World    <- src/puffysics/02_types.inl:306-332
 *   B3Batch    <- b3_batch.cuh:12-17
 * Capacities are compile-time for the struct (B3_MAX_*), exactly as in the
 * reference (src/puffysics/01_config.inl:53-74).  The engine library itself
 * is capacity-agnostic: it receives B3_CONFIG_SIGNATURE at every boundary
 * call and derives the array offsets at run time (b3_layout_of below).
 */
#ifndef PUFFYSICS_AMD_B3_TYPES_H
#define PUFFYSICS_AMD_B3_TYPES_H

#include <stddef.h>
#include <stdint.h>

#ifndef B3_MAX_BODIES
#define B3_MAX_BODIES 80
#endif
#ifndef B3_MAX_SHAPES
#define B3_MAX_SHAPES 128
#endif
#ifndef B3_MAX_CONTACTS
#define B3_MAX_CONTACTS 128
#endif
#ifndef B3_MAX_JOINTS
#define B3_MAX_JOINTS 32
#endif

/* 16 bits per capacity, bodies in the low word (01_config.inl:70-74). */
#define B3_CONFIG_SIGNATURE ( \
    ((unsigned long long)(B3_MAX_BODIES) & 0xffffull) \
  | (((unsigned long long)(B3_MAX_SHAPES) & 0xffffull) << 16) \
  | (((unsigned long long)(B3_MAX_CONTACTS) & 0xffffull) << 32) \
  | (((unsigned long long)(B3_MAX_JOINTS) & 0xffffull) << 48))

/* Solver constants of the default build (01_config.inl:96-146). */
#define B3_JOINT_ITERS 2
#define B3_RELAX_ITERS 2
#define B3_PI 3.14159265359f
#define B3_LINEAR_SLOP 0.005f
#define B3_SPECULATIVE 0.020f
#define B3_MAX_MANIFOLD 4
#define B3_MAX_ROTATION (0.25f * B3_PI)
#define B3_MIN_FRICTION_W 1.0e-10f

/* Enumerations (02_types.inl:5-22). */
#define B3_STATIC 0
#define B3_KINEMATIC 1
#define B3_DYNAMIC 2
#define B3_SPHERE 0
#define B3_CAPSULE 1
#define B3_BOX 2
#define B3_JOINT_WELD 0
#define B3_JOINT_REVOLUTE 1
#define B3_FLAG_DYNAMIC 0x00001000u
#define B3_LOCK_LIN_X 0x00000001u
#define B3_LOCK_LIN_Y 0x00000002u
#define B3_LOCK_LIN_Z 0x00000004u
#define B3_LOCK_ANG_X 0x00000008u
#define B3_LOCK_ANG_Y 0x00000010u
#define B3_LOCK_ANG_Z 0x00000020u

typedef struct B3Vec3 { float x, y, z; } B3Vec3;
typedef struct B3Vec2 { float x, y; } B3Vec2;
typedef struct B3Quat { B3Vec3 v; float s; } B3Quat;   /* vector first */
typedef struct B3Mat3 { B3Vec3 cx, cy, cz; } B3Mat3;  /* column major */
typedef struct B3Mat2 { B3Vec2 cx, cy; } B3Mat2;
typedef struct B3AABB { B3Vec3 lo, hi; } B3AABB;
typedef struct B3Soft { float bias_rate, mass_scale, impulse_scale; } B3Soft;

typedef struct B3Body {
    B3Vec3 position;
    B3Quat rotation;
    B3Vec3 center;
    B3Vec3 local_center;
    B3Vec3 lin_vel;
    B3Vec3 ang_vel;
    B3Vec3 force;
    B3Vec3 torque;
    B3Vec3 delta_pos;
    B3Quat delta_rot;
    float inv_mass;
    B3Vec3 inv_inertia;
    B3Mat3 inv_i_world;
    float linear_damping;
    float angular_damping;
    float gravity_scale;
    int type;
    uint32_t flags;
} B3Body;

typedef struct B3Shape {
    int body;
    int type;
    B3Vec3 local_pos;
    B3Quat local_rot;
    float radius;
    B3Vec3 half;
    float friction;
    float restitution;
    float rolling;
    float density;
    uint64_t category;
    uint64_t mask;
} B3Shape;

typedef struct B3Point {
    B3Vec3 r_a;
    B3Vec3 r_b;
    float base_sep;
    float rel_vel;
    float normal_impulse;
    float total_normal;
    float normal_mass;
    float lever;
    uint32_t feature;
} B3Point;

typedef struct B3Contact {
    int shape_a;
    int shape_b;
    int body_a;
    int body_b;
    int point_count;
    int static_contact;
    B3Vec3 normal;
    B3Vec3 tangent1;
    B3Vec3 tangent2;
    B3Point points[B3_MAX_MANIFOLD];
    B3Vec3 center_a;
    B3Vec3 center_b;
    float friction;
    float restitution;
    float rolling;
    float twist_mass;
    float twist_impulse;
    B3Vec2 friction_impulse;
    B3Vec3 rolling_impulse;
    B3Mat2 tangent_mass;
    B3Mat3 rolling_mass;
    float inv_mass_a;
    float inv_mass_b;
    B3Mat3 inv_i_a;
    B3Mat3 inv_i_b;
    B3Soft softness;
} B3Contact;

typedef struct B3Joint {
    int type;
    int body_a;
    int body_b;
    int collide_connected;
    int fixed_rotation;
    B3Vec3 local_anchor_a;
    B3Vec3 local_anchor_b;
    B3Quat local_rot_a;
    B3Quat local_rot_b;
    float constraint_hertz;
    float constraint_damping;
    B3Soft softness;
    float inv_mass_a;
    float inv_mass_b;
    B3Mat3 inv_i_a;
    B3Mat3 inv_i_b;
    B3Vec3 frame_p_a;
    B3Vec3 frame_p_b;
    B3Quat frame_q_a;
    B3Quat frame_q_b;
    B3Vec3 delta_center;
    B3Vec3 linear_impulse;
    B3Vec3 angular_impulse;
    B3Mat3 angular_mass;
    float linear_hertz;
    float linear_damping;
    float angular_hertz;
    float angular_damping;
    B3Soft linear_spring;
    B3Soft angular_spring;
    B3Vec2 perp_impulse;
    float spring_impulse;
    float motor_impulse;
    float lower_impulse;
    float upper_impulse;
    float hertz;
    float damping_ratio;
    float max_motor_torque;
    float motor_speed;
    float target_angle;
    float lower_angle;
    float upper_angle;
    int enable_spring;
    int enable_motor;
    int enable_limit;
    B3Vec3 rotation_axis;
    B3Vec3 perp_x;
    B3Vec3 perp_y;
    float axial_mass;
    B3Soft spring_softness;
} B3Joint;

/* World header: everything in B3World before the bodies array. */
typedef struct B3WorldHeader {
    B3Vec3 gravity;
    float contact_hertz;
    float contact_damping;
    float contact_speed;
    float restitution_threshold;
    float max_linear_speed;
    int body_count;
    int shape_count;
    int contact_count;
    int joint_count;
    int body_overflow;
    int shape_overflow;
    int joint_overflow;
    int contact_overflow;
    int contacts_dropped;
} B3WorldHeader;

typedef struct B3World {
    B3Vec3 gravity;
    float contact_hertz;
    float contact_damping;
    float contact_speed;
    float restitution_threshold;
    float max_linear_speed;
    int body_count;
    int shape_count;
    int contact_count;
    int joint_count;
    int body_overflow;
    int shape_overflow;
    int joint_overflow;
    int contact_overflow;
    int contacts_dropped;
    B3Body bodies[B3_MAX_BODIES];
    B3Shape shapes[B3_MAX_SHAPES];
    B3Contact contacts[B3_MAX_CONTACTS];
    B3Joint joints[B3_MAX_JOINTS];
} B3World;

typedef struct B3StepStats {
    int body_count;
    int shape_count;
    int contact_count;
    int joint_count;
    int body_overflow;
    int shape_overflow;
    int joint_overflow;
    int contact_overflow;
    int contacts_dropped;
} B3StepStats;

typedef struct B3BodyDef {
    int type;
    B3Vec3 position;
    B3Quat rotation;
    B3Vec3 lin_vel;
    B3Vec3 ang_vel;
    float linear_damping;
    float angular_damping;
    float gravity_scale;
    uint32_t flags;
} B3BodyDef;

typedef struct B3ShapeDef {
    float density;
    float friction;
    float restitution;
    float rolling;
    uint64_t category;
    uint64_t mask;
} B3ShapeDef;

/* Non-owning strided view of worlds, possibly embedded in a caller struct. */
typedef struct B3Batch {
    void* data;
    size_t stride;       /* sizeof(B3World) or sizeof(enclosing struct) */
    size_t world_offset; /* offsetof(enclosing struct, world) or 0 */
    int count;
} B3Batch;

/* Run-time form of the compile-time capacities: byte offsets of the four
 * arrays inside one B3World of a given signature.  Matches the compiler's
 * layout of B3World: a 68-byte header, 4-aligned bodies, then 8-aligned
 * shapes (B3Shape holds uint64_t), contacts and joints. */
typedef struct B3Layout {
    int max_bodies, max_shapes, max_contacts, max_joints;
    size_t bodies_off, shapes_off, contacts_off, joints_off, world_size;
} B3Layout;

static inline int b3_layout_of(unsigned long long sig, B3Layout* out) {
    int b = (int)(sig & 0xffffull);
    int s = (int)((sig >> 16) & 0xffffull);
    int c = (int)((sig >> 32) & 0xffffull);
    int j = (int)((sig >> 48) & 0xffffull);
    if (b < 1 || s < 1 || c < 1 || j < 1) return 0;
    out->max_bodies = b;
    out->max_shapes = s;
    out->max_contacts = c;
    out->max_joints = j;
    out->bodies_off = sizeof(B3WorldHeader);
    size_t off = out->bodies_off + (size_t)b * sizeof(B3Body);
    off = (off + 7u) & ~(size_t)7u;
    out->shapes_off = off;
    off += (size_t)s * sizeof(B3Shape);
    out->contacts_off = off;
    off += (size_t)c * sizeof(B3Contact);
    out->joints_off = off;
    off += (size_t)j * sizeof(B3Joint);
    out->world_size = (off + 7u) & ~(size_t)7u;
    return 1;
}

#endif /* PUFFYSICS_AMD_B3_TYPES_H */
