/*
 * b3_scene_lib.c - host world builders of the benchmark scenes.
 *
 * Compiled once per scene with that scene's capacities (B3_MAX_*) and
 * B3W_SCENE, like any B3World user: worlds are built by the public
 * creation API (include/b3_setup.h), then handed to the engine.  Exports
 *   b3s_signature_<n>, b3s_world_size_<n>, b3s_build_batch_<n>,
 *   b3s_apply_inputs_batch_<n>
 * Capacity set 0 has no scene; it exports the creation API (b3c_*).
 */
#include <stddef.h>
#include "../../include/b3_setup.h"
#define B3S_WITH_BUILDERS 1
#include "b3_scenes.h"

#define B3L_CAT2(a, b) a##_##b
#define B3L_CAT(a, b) B3L_CAT2(a, b)

unsigned long long B3L_CAT(b3s_signature, B3W_SCENE)(void) { return B3_CONFIG_SIGNATURE; }
size_t B3L_CAT(b3s_world_size, B3W_SCENE)(void) { return sizeof(B3World); }

#if B3W_SCENE > 0
/* Build worlds first .. first + count - 1 into a contiguous array. */
int B3L_CAT(b3s_build_batch, B3W_SCENE)(void* worlds, int count, unsigned long long seed, int first) {
    for (int i = 0; i < count; i++)
        if (!b3s_build(B3W_SCENE, (B3World*)worlds + i, seed, first + i)) return 0;
    return 1;
}

/* Host application of step `step`'s inputs to the selected worlds. */
void B3L_CAT(b3s_apply_inputs_batch, B3W_SCENE)(void* worlds, int count, unsigned long long seed, int first,
        int step, const unsigned char* step_mask) {
    for (int i = 0; i < count; i++)
        if (!step_mask || step_mask[i]) b3s_apply_inputs(B3W_SCENE, (B3World*)worlds + i, seed, first + i, step);
}
#endif

#if B3W_SCENE == 1
/* Reset and step masks of vector step `step` for worlds [first, first +
 * count): the arm scene draws them, every other scene steps all worlds and
 * resets none (the same draws as the device's b3w_masks_gpu). */
void b3s_masks(int scene, unsigned long long seed, int first, int count, int step, unsigned char* reset,
        unsigned char* step_out) {
    for (int i = 0; i < count; i++) {
        if (scene == B3S_ARM) {
            reset[i] = b3s_arm_reset(seed, first + i, step);
            step_out[i] = b3s_arm_step(seed, first + i, step);
        } else {
            reset[i] = 0;
            step_out[i] = 1;
        }
    }
}
#endif

#if B3W_SCENE == 0
/* Capacity set 0 (16 bodies, 16 shapes, 32 contacts, 8 joints) also
 * exports the creation API with plain arguments, so that callers without a
 * C compiler can build arbitrary worlds (include/b3_setup.h, the reference's
 * 04_world.inl and 06_joints.inl). */
void b3c_world_init(void* w, float gx, float gy, float gz) {
    b3_world_init((B3World*)w);
    ((B3World*)w)->gravity = b3_v(gx, gy, gz);
}
int b3c_body(void* w, int type, float px, float py, float pz, float qx, float qy, float qz, float qs, float vx,
        float vy, float vz, float ax, float ay, float az) {
    B3BodyDef d = b3_default_body();
    d.type = type;
    d.position = b3_v(px, py, pz);
    d.rotation = b3_q(qx, qy, qz, qs);
    d.lin_vel = b3_v(vx, vy, vz);
    d.ang_vel = b3_v(ax, ay, az);
    return b3_create_body((B3World*)w, &d);
}
static B3ShapeDef b3c_def(float density, float friction, float restitution) {
    B3ShapeDef d = b3_default_shape();
    d.density = density;
    d.friction = friction;
    d.restitution = restitution;
    return d;
}
int b3c_sphere(void* w, int body, float cx, float cy, float cz, float r, float density, float friction,
        float restitution) {
    B3ShapeDef d = b3c_def(density, friction, restitution);
    return b3_create_sphere((B3World*)w, body, b3_v(cx, cy, cz), r, &d);
}
int b3c_box(void* w, int body, float hx, float hy, float hz, float px, float py, float pz, float density,
        float friction, float restitution) {
    B3ShapeDef d = b3c_def(density, friction, restitution);
    return b3_create_box_local((B3World*)w, body, b3_v(hx, hy, hz), b3_v(px, py, pz), b3_q_id(), &d);
}
int b3c_capsule(void* w, int body, float half_len, float r, float density, float friction, float restitution) {
    B3ShapeDef d = b3c_def(density, friction, restitution);
    return b3_create_capsule((B3World*)w, body, half_len, r, &d);
}
void b3c_finalize_mass(void* w, int body) { b3_finalize_mass((B3World*)w, body); }
void b3c_set_inertial(void* w, int body, float mass, float ix, float iy, float iz) {
    b3_set_inertial((B3World*)w, body, mass, b3_v(0.0f, 0.0f, 0.0f), b3_v(ix, iy, iz));
}
int b3c_revolute(void* w, int a, int b, float ax, float ay, float az, float bx, float by, float bz, float nx,
        float ny, float nz) {
    return b3_create_revolute((B3World*)w, a, b, b3_v(ax, ay, az), b3_v(bx, by, bz), b3_v(nx, ny, nz));
}
int b3c_weld(void* w, int a, int b, float ax, float ay, float az, float bx, float by, float bz) {
    return b3_create_weld((B3World*)w, a, b, b3_v(ax, ay, az), b3_v(bx, by, bz));
}
void b3c_joint_limits(void* w, int j, int enable, float lower, float upper) {
    b3_joint_enable_limit((B3World*)w, j, enable);
    b3_joint_set_limits((B3World*)w, j, lower, upper);
}
void b3c_joint_motor(void* w, int j, int enable, float speed, float max_torque) {
    b3_joint_enable_motor((B3World*)w, j, enable);
    b3_joint_set_motor((B3World*)w, j, speed, max_torque);
}
void b3c_joint_spring(void* w, int j, int enable, float target, float hertz, float damping) {
    b3_joint_enable_spring((B3World*)w, j, enable);
    b3_joint_set_spring((B3World*)w, j, target, hertz, damping);
}
#endif
