/*
 * b3_workload.h - host loop that drives a batch of worlds through a scene's
 * per-step inputs, for CPU baselines and fixture generation.
 *
 * One vector step t, in this order (the engine's b3_batch_step_gpu follows
 * the same order on the device):
 *   1. masks: the arm scene draws reset and step masks, other scenes step
 *      every world and reset none;
 *   2. restore worlds whose reset byte is set from their snapshot
 *      (b3_batch_restore semantics);
 *   3. apply the scene inputs of step t to every world that will step;
 *   4. step the worlds selected by the step mask (b3_batch_step).
 * Returns the number of env-steps taken (sum of the step masks).
 *
 * The including translation unit supplies B3World (fixed capacities), the
 * creation-side API used by b3s_apply_inputs, and two functions:
 *   int B3W_STEP(void* worlds, int count, float dt, int substeps, const unsigned char* active);
 *   int B3W_RESTORE(void* worlds, int count, const void* initial, const unsigned char* reset);
 */
#ifndef PUFFYSICS_AMD_B3_WORKLOAD_H
#define PUFFYSICS_AMD_B3_WORKLOAD_H

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define B3S_WITH_BUILDERS 1
#include "b3_scenes.h"

/* Masks of step t for worlds [first, first + count). */
static inline void b3w_masks(int scene, uint64_t seed, int first, int count, int t,
        unsigned char* reset, unsigned char* step, int* any_reset) {
    *any_reset = 0;
    for (int i = 0; i < count; i++) {
        if (scene == B3S_ARM) {
            reset[i] = b3s_arm_reset(seed, first + i, t);
            step[i] = b3s_arm_step(seed, first + i, t);
        } else {
            reset[i] = 0;
            step[i] = 1;
        }
        *any_reset |= reset[i];
    }
}

/* Steps [t0, t0 + nsteps) for worlds [first, first + count).  `initial` holds
 * the snapshots of exactly these worlds. */
static inline long long b3w_run_slice(int scene, B3World* worlds, const B3World* initial, int first,
        int count, uint64_t seed, int t0, int nsteps, float dt, int substeps, pthread_barrier_t* bar) {
    unsigned char* reset = (unsigned char*)malloc((size_t)(count > 0 ? count : 1));
    unsigned char* step = (unsigned char*)malloc((size_t)(count > 0 ? count : 1));
    long long env_steps = 0;
    for (int t = t0; t < t0 + nsteps; t++) {
        int any_reset;
        b3w_masks(scene, seed, first, count, t, reset, step, &any_reset);
        if (any_reset && initial) B3W_RESTORE(worlds, count, initial, reset);
        for (int i = 0; i < count; i++) {
            if (!step[i]) continue;
            b3s_apply_inputs(scene, &worlds[i], seed, first + i, t);
            env_steps++;
        }
        B3W_STEP(worlds, count, dt, substeps, step);
        if (bar) pthread_barrier_wait(bar);
    }
    free(reset);
    free(step);
    return env_steps;
}

typedef struct {
    int scene;
    B3World* worlds;
    const B3World* initial;
    int first, count;
    uint64_t seed;
    int t0, nsteps;
    float dt;
    int substeps;
    pthread_barrier_t* bar;
    long long env_steps;
    int cpu;
} B3wJob;

static void* b3w_thread(void* arg) {
    B3wJob* j = (B3wJob*)arg;
    if (j->cpu >= 0) {
        cpu_set_t set;
        CPU_ZERO(&set);
        CPU_SET(j->cpu, &set);
        pthread_setaffinity_np(pthread_self(), sizeof(set), &set);
    }
    j->env_steps = b3w_run_slice(j->scene, j->worlds + j->first, j->initial ? j->initial + j->first : NULL,
        j->first, j->count, j->seed, j->t0, j->nsteps, j->dt, j->substeps, j->bar);
    return NULL;
}

/* Contiguous slices, one thread each, barrier after every step.  cpus may be
 * NULL (no pinning) or list one logical CPU per thread. */
static inline long long b3w_run(int scene, B3World* worlds, const B3World* initial, int count,
        uint64_t seed, int t0, int nsteps, float dt, int substeps, int nthreads, const int* cpus) {
    if (nthreads <= 1 || count < 2)
        return b3w_run_slice(scene, worlds, initial, 0, count, seed, t0, nsteps, dt, substeps, NULL);
    if (nthreads > count) nthreads = count;
    B3wJob* jobs = (B3wJob*)calloc((size_t)nthreads, sizeof(B3wJob));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    pthread_barrier_t bar;
    pthread_barrier_init(&bar, NULL, (unsigned)nthreads);
    int per = count / nthreads, extra = count % nthreads, first = 0;
    for (int k = 0; k < nthreads; k++) {
        int n = per + (k < extra ? 1 : 0);
        jobs[k].scene = scene;
        jobs[k].worlds = worlds;
        jobs[k].initial = initial;
        jobs[k].first = first;
        jobs[k].count = n;
        jobs[k].seed = seed;
        jobs[k].t0 = t0;
        jobs[k].nsteps = nsteps;
        jobs[k].dt = dt;
        jobs[k].substeps = substeps;
        jobs[k].bar = &bar;
        jobs[k].cpu = cpus ? cpus[k] : -1;
        first += n;
        pthread_create(&th[k], NULL, b3w_thread, &jobs[k]);
    }
    long long total = 0;
    for (int k = 0; k < nthreads; k++) {
        pthread_join(th[k], NULL);
        total += jobs[k].env_steps;
    }
    pthread_barrier_destroy(&bar);
    free(jobs);
    free(th);
    return total;
}

#endif /* PUFFYSICS_AMD_B3_WORKLOAD_H */
