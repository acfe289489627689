/*
 * ref_forces.c - the reference's own b3_step with a force law in its
 * B3_USER_FORCES hook (01_config.inl:189-198, 09_step.inl:20-53).
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile from the reference
 * sources in place (nbody_rigid.cuh, which pulls puffysics.cuh and
 * nbody.cuh; nothing is copied), once per capacity set, into oracle/_ref/.
 * The hook runs the reference's own b3_nbody_apply_forces
 * (nbody_rigid.cuh:68-73) at the bodies' current centers: it moves each
 * center to center + delta_pos for the call and puts it back after.  The
 * tests check the oracle's hook and gravity law against this reference
 * code.
 */
#define _GNU_SOURCE
struct B3World;
static void ref_hook(struct B3World* w, float h);
#define B3_USER_FORCES(w, h) ref_hook((w), (h))
#include "nbody_rigid.cuh"

static int g_law;   /* 1 gravity */
static NbodyConfig g_cfg;
static float* g_masses;

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
    (void)h;
    if (g_law == 1) ref_gravity_hook(w);
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
