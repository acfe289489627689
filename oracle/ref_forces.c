/*
 * ref_forces.c - the reference's own b3_step with a force law in its
 * B3_USER_FORCES hook (01_config.inl:189-198, 09_step.inl:20-53).
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile from the reference
 * sources in place (nbody_rigid.cuh, which pulls puffysics.cuh and
 * nbody.cuh, and ambient.h; nothing is copied), once per capacity set, into
 * oracle/_ref/.  The hook runs one of two of the reference's own force
 * modules:
 *   - b3_nbody_apply_forces (nbody_rigid.cuh:68-73) at the bodies' current
 *     centers: it moves each center to center + delta_pos for the call and
 *     puts it back after;
 *   - b3_fluid_step (ambient.h:361-370) with the caller's B3Fluid and
 *     state.
 * The tests check the oracle's hook and laws against this reference code.
 */
#define _GNU_SOURCE
struct B3World;
static void ref_hook(struct B3World* w, float h);
#define B3_USER_FORCES(w, h) ref_hook((w), (h))
#include "nbody_rigid.cuh"
#include "ambient.h"

static int g_law;   /* 1 gravity, 2 fluid */
static NbodyConfig g_cfg;
static float* g_masses;
static B3Fluid g_fluid;
static B3FluidState g_fstate;

static void ref_gravity_hook(struct B3World* w) {
    B3Vec3 saved[B3_MAX_BODIES];
    for (int i = 0; i < w->body_count; i++) {
        saved[i] = w->bodies[i].center;
        w->bodies[i].center = b3_add(w->bodies[i].center, w->bodies[i].delta_pos);
    }
    b3_nbody_apply_forces(w, g_cfg, g_masses);
    for (int i = 0; i < w->body_count; i++) w->bodies[i].center = saved[i];
}

static void ref_hook(struct B3World* w, float h) {
    if (g_law == 1) ref_gravity_hook(w);
    else if (g_law == 2) b3_fluid_step(&g_fluid, w, &g_fstate, h);
}

unsigned long long refg_sig(void) { return b3_config_signature(); }

/* b3_step on one world with gravity of strength `gravity`, softening
 * `softening`, and gravitational masses `masses` (NULL: 1 / inv_mass). */
void refg_step(void* world, float dt, int substeps, float gravity, float softening, float* masses) {
    g_law = 1;
    g_cfg.gravity = gravity;
    g_cfg.softening = softening;
    g_masses = masses;
    b3_step((B3World*)world, dt, substeps);
    g_law = 0;
}

/* b3_step on one world with b3_fluid_step in the hook.  `fluid` is a
 * B3Fluid; `state` holds, per body, the previous linear and angular
 * velocity (6 floats), then have_prev (int), B3_MAX_BODIES bodies. */
void refg_step_fluid(void* world, float dt, int substeps, const void* fluid, float* state) {
    memcpy(&g_fluid, fluid, sizeof(B3Fluid));
    for (int i = 0; i < B3_MAX_BODIES; i++) {
        g_fstate.prev_lin[i] = b3_v(state[6 * i], state[6 * i + 1], state[6 * i + 2]);
        g_fstate.prev_ang[i] = b3_v(state[6 * i + 3], state[6 * i + 4], state[6 * i + 5]);
    }
    memcpy(&g_fstate.have_prev, state + 6 * B3_MAX_BODIES, sizeof(int));
    g_law = 2;
    b3_step((B3World*)world, dt, substeps);
    g_law = 0;
    for (int i = 0; i < B3_MAX_BODIES; i++) {
        B3Vec3 l = g_fstate.prev_lin[i], a = g_fstate.prev_ang[i];
        float v[6] = {l.x, l.y, l.z, a.x, a.y, a.z};
        memcpy(state + 6 * i, v, sizeof(v));
    }
    memcpy(state + 6 * B3_MAX_BODIES, &g_fstate.have_prev, sizeof(int));
}

size_t refg_fluid_size(void) { return sizeof(B3Fluid); }
