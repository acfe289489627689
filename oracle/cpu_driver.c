/*
 * cpu_driver.c - per-scene CPU workload runner over the oracle.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled once per scene with that scene's
 * capacities (B3_MAX_*) and B3W_SCENE; exports
 *   ocpu_build_<n>, ocpu_apply_inputs_<n>, ocpu_run_<n>
 * used by the tests and by the CPU-baseline leg of the benchmark.  Worlds
 * are built with the engine's public creation header (include/b3_setup.h)
 * and stepped by the oracle (b3cpu.c), one pinned thread per core, with the
 * b3_batch_step / b3_batch_restore semantics of b3_batch.cuh:39-60.
 */
#define _GNU_SOURCE
#include "../include/b3_setup.h"
#include "b3cpu.h"

static int oc_step_batch(void* worlds, int count, float dt, int substeps, const unsigned char* active) {
    return ocpu_batch_step(worlds, sizeof(B3World), 0, count, B3_CONFIG_SIGNATURE, dt, substeps, active);
}
static int oc_restore_batch(void* worlds, int count, const void* initial, const unsigned char* reset) {
    return ocpu_batch_restore(worlds, sizeof(B3World), 0, count, B3_CONFIG_SIGNATURE, initial, reset);
}
#define B3W_STEP oc_step_batch
#define B3W_RESTORE oc_restore_batch
#include "../puffysics_amd/scenes/b3_workload.h"

#define OC_CAT2(a, b) a##_##b
#define OC_CAT(a, b) OC_CAT2(a, b)

int OC_CAT(ocpu_build, B3W_SCENE)(void* world, unsigned long long seed, int index) {
    return b3s_build(B3W_SCENE, (B3World*)world, seed, index);
}
void OC_CAT(ocpu_apply_inputs, B3W_SCENE)(void* world, unsigned long long seed, int index, int step) {
    b3s_apply_inputs(B3W_SCENE, (B3World*)world, seed, index, step);
}
long long OC_CAT(ocpu_run, B3W_SCENE)(void* worlds, const void* initial, int count, unsigned long long seed,
        int t0, int nsteps, float dt, int substeps, int nthreads, const int* cpus) {
    return b3w_run(B3W_SCENE, (B3World*)worlds, (const B3World*)initial, count, seed, t0, nsteps, dt,
        substeps, nthreads, cpus);
}
