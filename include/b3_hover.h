/*
 * b3_hover.h - the PufferLib hover environment on the MI355X engine.
 *
 * The reference ships this task as a CUDA adapter whose single kernel runs
 * action, b3_step, reward / terminal, reset and observation per env
 * (examples/pufferlib/puffysics_hover/puffysics_hover.cu:21-79,
 * puffysics_hover.h:21-94, hover_task.h:45-99).  Here the physics runs in
 * the engine (b3_engine.h) and the task around it in three small kernels
 * on the same stream:
 *   action kernel      level = 0 / 1 / 2 from the action, force on the body
 *   b3_batch_step_gpu  every env
 *   reward kernel      tick, reward, terminal, episode return and log;
 *                      envs that are done draw their next start height
 *   b3_batch_restore_gpu of the done envs to the task's initial world
 *   observe kernel     the new start height of reset envs, observations
 * Results are the reference adapter's, bit for bit (tests/test_hover.py).
 *
 * The entry points mirror the adapter's puf_vec_create / puf_reset /
 * puf_step / puf_close / puf_log (puffysics_hover.cu:44-79,
 * puffysics_hover.h:72-78); buffers are the caller's device arrays of
 * n*3 observations, n actions, n rewards and n terminals.  Conventions are
 * the engine's: hipError_t returns, no abort, hipErrorInvalidValue for bad
 * arguments with nothing launched.
 */
#ifndef PUFFYSICS_AMD_B3_HOVER_H
#define PUFFYSICS_AMD_B3_HOVER_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "b3_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* HoverConfig (hover_task.h:22-28); defaults 2, 10, 1/60, 4, 256
 * (hover_default_config, hover_task.h:39-42). */
typedef struct B3HoverConfig {
    float target_height;
    float thrust;
    float dt;
    int substeps;
    int horizon;
} B3HoverConfig;

/* Log (puffysics_hover.h:13-19), summed over the envs. */
typedef struct B3HoverLog {
    float perf;
    float score;
    float episode_return;
    float episode_length;
    float n;
} B3HoverLog;

typedef struct B3HoverEnvs B3HoverEnvs;

B3HoverConfig b3_hover_default_config(void);

/* puf_vec_create (puffysics_hover.cu:44-60): n envs, env i seeded with
 * seed + i * 747796405 and reset once (hover_init).  The device buffers stay
 * the caller's.  Allocates; synchronises. */
hipError_t b3_hover_create(B3HoverEnvs** out, int n, B3HoverConfig config, uint32_t seed, float* observations,
    float* actions, float* rewards, float* terminals);
/* puf_reset (hover_env_reset, puffysics_hover.h:31-36): every env starts a
 * new episode; observations written, rewards and terminals zeroed. */
hipError_t b3_hover_reset(B3HoverEnvs* envs, hipStream_t stream);
/* puf_step (hover_env_step, puffysics_hover.h:38-56) on every env. */
hipError_t b3_hover_step(B3HoverEnvs* envs, hipStream_t stream);
/* puf_log: the envs' logs summed into *out (synchronises the stream). */
hipError_t b3_hover_log(B3HoverEnvs* envs, B3HoverLog* out, hipStream_t stream);
/* The engine holding the envs' worlds (for downloads and observation
 * kernels); owned by the envs. */
B3Engine* b3_hover_engine(B3HoverEnvs* envs);
/* puf_close (puffysics_hover.cu:71-76).  NULL is a no-op. */
hipError_t b3_hover_destroy(B3HoverEnvs* envs);

#ifdef __cplusplus
}
#endif
#endif
