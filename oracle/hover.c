/*
 * hover.c - CPU restatement of the reference's PufferLib hover environment.
 *
 * TEST INFRASTRUCTURE ONLY.  Follows examples/pufferlib/puffysics_hover/
 * hover_task.h (task: reset, action, observation, reward, terminal, step)
 * and puffysics_hover.h:38-56 (the environment step: episode return, log,
 * reset on done, observe) and the GPU adapter's per-env seeding
 * (puffysics_hover.cu:32-42), on the oracle's b3_step.  Compiled with the
 * hover capacities (2 bodies, 2 shapes, 4 contacts, 2 joints).  Only the
 * tests load it; the engine's hover adapter never calls it.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "b3_types.h"
#include "b3_setup.h"
#include "b3cpu.h"

typedef struct {
    float target_height, thrust, dt;
    int substeps, horizon;
} OHoverConfig;

typedef struct {
    float perf, score, episode_return, episode_length, n;
} OHoverLog;

typedef struct {
    B3World world;
    OHoverConfig config;
    uint32_t rng;
    int tick;
    int body;
    float episode_return;
    OHoverLog log;
} OHoverEnv;

/* hover_task.h:44-60 */
static void task_reset(OHoverEnv* t) {
    b3_world_init(&t->world);
    t->rng = t->rng * 1664525u + 1013904223u;
    float jitter = (float)(t->rng >> 8) * (1.0f / 16777216.0f) - 0.5f;
    B3BodyDef body = b3_default_body();
    body.type = B3_DYNAMIC;
    body.position = b3_v(0, t->config.target_height + jitter, 0);
    body.linear_damping = 0;
    t->body = b3_create_body(&t->world, &body);
    B3ShapeDef shape = b3_default_shape();
    b3_create_sphere(&t->world, t->body, b3_v(0, 0, 0), 0.25f, &shape);
    b3_finalize_mass(&t->world, t->body);
    t->tick = 0;
    t->episode_return = 0;
}

/* hover_task.h:68-73 */
static void task_action(OHoverEnv* t, float action) {
    float level = action >= 1.5f ? 2.0f : (action >= 0.5f ? 1.0f : 0.0f);
    const B3Body* b = &t->world.bodies[t->body];
    ocpu_apply_force(&t->world, B3_CONFIG_SIGNATURE, t->body, 0.0f, level * t->config.thrust / b->inv_mass, 0.0f);
}

/* hover_task.h:75-92 */
static void task_observe(const OHoverEnv* t, float* obs) {
    const B3Body* b = &t->world.bodies[t->body];
    obs[0] = b->position.y - t->config.target_height;
    obs[1] = b->lin_vel.y;
    obs[2] = (float)t->tick / (float)t->config.horizon;
}
static float task_reward(const OHoverEnv* t) {
    const B3Body* b = &t->world.bodies[t->body];
    float error = fabsf(b->position.y - t->config.target_height);
    float e = error + 0.1f * fabsf(b->lin_vel.y);
    return 1.0f - (e < 2.0f ? e : 2.0f);
}
static int task_terminal(const OHoverEnv* t) {
    float height = t->world.bodies[t->body].position.y;
    return !isfinite(height) || fabsf(height - t->config.target_height) > 3.0f || t->tick >= t->config.horizon;
}

size_t ohover_env_bytes(void) { return sizeof(OHoverEnv); }
unsigned long long ohover_signature(void) { return B3_CONFIG_SIGNATURE; }

/* puffysics_hover.cu:32-42 (seed + i * 747796405) and hover_task.h:62-66 */
void ohover_init(void* envs, int n, float target, float thrust, float dt, int substeps, int horizon, uint32_t seed) {
    OHoverEnv* e = (OHoverEnv*)envs;
    for (int i = 0; i < n; i++) {
        memset(&e[i], 0, sizeof(OHoverEnv));
        e[i].config.target_height = target;
        e[i].config.thrust = thrust;
        e[i].config.dt = dt;
        e[i].config.substeps = substeps;
        e[i].config.horizon = horizon;
        e[i].rng = seed + (uint32_t)i * 747796405u;
        task_reset(&e[i]);
    }
}

/* puffysics_hover.h:31-36 */
void ohover_reset(void* envs, int n, float* obs, float* rewards, float* terminals) {
    OHoverEnv* e = (OHoverEnv*)envs;
    for (int i = 0; i < n; i++) {
        task_reset(&e[i]);
        task_observe(&e[i], obs + (size_t)i * 3);
        rewards[i] = 0;
        terminals[i] = 0;
    }
}

/* puffysics_hover.h:38-56 */
void ohover_step(void* envs, int n, const float* actions, float* obs, float* rewards, float* terminals) {
    OHoverEnv* e = (OHoverEnv*)envs;
    for (int i = 0; i < n; i++) {
        OHoverEnv* t = &e[i];
        task_action(t, actions[i]);
        ocpu_step(&t->world, B3_CONFIG_SIGNATURE, t->config.dt, t->config.substeps);
        t->tick++;
        float reward = task_reward(t);
        int done = task_terminal(t);
        t->episode_return += reward;
        if (done) {
            t->log.perf += t->tick >= t->config.horizon;
            t->log.score += t->episode_return;
            t->log.episode_return += t->episode_return;
            t->log.episode_length += (float)t->tick;
            t->log.n += 1;
            task_reset(t);
        }
        task_observe(t, obs + (size_t)i * 3);
        rewards[i] = reward;
        terminals[i] = (float)done;
    }
}

/* The sum of the per-env logs (perf, score, episode_return, episode_length, n). */
void ohover_log(const void* envs, int n, float* out) {
    const OHoverEnv* e = (const OHoverEnv*)envs;
    for (int k = 0; k < 5; k++) out[k] = 0;
    for (int i = 0; i < n; i++) {
        out[0] += e[i].log.perf;
        out[1] += e[i].log.score;
        out[2] += e[i].log.episode_return;
        out[3] += e[i].log.episode_length;
        out[4] += e[i].log.n;
    }
}

/* A copy of env i's world. */
void ohover_world(const void* envs, int i, void* world) {
    memcpy(world, &((const OHoverEnv*)envs)[i].world, sizeof(B3World));
}
