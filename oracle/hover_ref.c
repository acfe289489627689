/*
 * hover_ref.c - C entry points around the reference's own hover task.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile directly from
 * examples/pufferlib/puffysics_hover/hover_task.h under the reference tree
 * (nothing is copied) into oracle/_ref/.  The environment step of
 * puffysics_hover.h:38-56 (which needs PufferLib's headers) is restated
 * around the reference's task functions.  Writes the hover golden fixtures.
 */
#include "hover_task.h"

typedef struct {
    float perf, score, episode_return, episode_length, n;
} RHoverLog;

typedef struct {
    HoverTask task;
    RHoverLog log;
} RHoverEnv;

size_t rhover_env_bytes(void) { return sizeof(RHoverEnv); }
unsigned long long rhover_signature(void) { return b3_config_signature(); }

void rhover_init(void* envs, int n, float target, float thrust, float dt, int substeps, int horizon, uint32_t seed) {
    RHoverEnv* e = (RHoverEnv*)envs;
    for (int i = 0; i < n; i++) {
        memset(&e[i], 0, sizeof(RHoverEnv));
        HoverConfig c = hover_default_config();
        c.target_height = target;
        c.thrust = thrust;
        c.dt = dt;
        c.substeps = substeps;
        c.horizon = horizon;
        hover_init(&e[i].task, c, seed + (uint32_t)i * 747796405u);
    }
}

void rhover_reset(void* envs, int n, float* obs, float* rewards, float* terminals) {
    RHoverEnv* e = (RHoverEnv*)envs;
    for (int i = 0; i < n; i++) {
        hover_reset(&e[i].task);
        hover_observe(&e[i].task, obs + (size_t)i * 3);
        rewards[i] = 0;
        terminals[i] = 0;
    }
}

void rhover_step(void* envs, int n, const float* actions, float* obs, float* rewards, float* terminals) {
    RHoverEnv* e = (RHoverEnv*)envs;
    for (int i = 0; i < n; i++) {
        HoverTask* task = &e[i].task;
        hover_step(task, actions[i]);
        float reward = hover_reward(task);
        int done = hover_terminal(task);
        task->episode_return += reward;
        if (done) {
            e[i].log.perf += task->tick >= task->config.horizon;
            e[i].log.score += task->episode_return;
            e[i].log.episode_return += task->episode_return;
            e[i].log.episode_length += (float)task->tick;
            e[i].log.n += 1;
            hover_reset(task);
        }
        hover_observe(task, obs + (size_t)i * 3);
        rewards[i] = reward;
        terminals[i] = (float)done;
    }
}

void rhover_log(const void* envs, int n, float* out) {
    const RHoverEnv* e = (const RHoverEnv*)envs;
    for (int k = 0; k < 5; k++) out[k] = 0;
    for (int i = 0; i < n; i++) {
        out[0] += e[i].log.perf;
        out[1] += e[i].log.score;
        out[2] += e[i].log.episode_return;
        out[3] += e[i].log.episode_length;
        out[4] += e[i].log.n;
    }
}

void rhover_world(const void* envs, int i, void* world) {
    memcpy(world, &((const RHoverEnv*)envs)[i].task.world, sizeof(B3World));
}
