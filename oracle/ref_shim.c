/*
 * ref_shim.c - C entry points around the reference's own CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile directly from the
 * reference sources (b3_batch.cuh, puffysics.cuh under the reference tree;
 * nothing is copied) once per capacity set, into oracle/_ref/.  It lets the
 * tests check the C restatement in b3cpu.c bit for bit against the real
 * b3_step, b3_batch_step and b3_batch_restore, and writes golden fixtures.
 * Scenes are built through the reference's creation API by the same
 * scene code the engine's scene library uses.
 */
#define _GNU_SOURCE
#include "b3_batch.cuh"

static int ref_step_batch(void* worlds, int count, float dt, int substeps, const unsigned char* active) {
    B3Batch b = {worlds, sizeof(B3World), 0, count};
    return b3_batch_step(b, dt, substeps, active);
}
static int ref_restore_batch(void* worlds, int count, const void* initial, const unsigned char* reset) {
    B3Batch b = {worlds, sizeof(B3World), 0, count};
    return b3_batch_restore(b, (const B3World*)initial, reset);
}
#define B3W_STEP ref_step_batch
#define B3W_RESTORE ref_restore_batch
#include "b3_workload.h"

unsigned long long ref_sig(void) { return b3_config_signature(); }
size_t ref_world_size(void) { return sizeof(B3World); }
int ref_build(int scene, void* world, unsigned long long seed, int index) {
    return b3s_build(scene, (B3World*)world, seed, index);
}
void ref_apply_inputs(int scene, void* world, unsigned long long seed, int index, int step) {
    b3s_apply_inputs(scene, (B3World*)world, seed, index, step);
}
void ref_step(void* world, float dt, int substeps) { b3_step((B3World*)world, dt, substeps); }
void ref_find_contacts(void* world) { b3_find_contacts((B3World*)world); }
int ref_batch_step(void* worlds, int count, float dt, int substeps, const unsigned char* active) {
    return ref_step_batch(worlds, count, dt, substeps, active);
}
int ref_batch_restore(void* worlds, int count, const void* initial, const unsigned char* reset) {
    return ref_restore_batch(worlds, count, initial, reset);
}
long long ref_run(int scene, void* worlds, const void* initial, int count, unsigned long long seed,
        int t0, int nsteps, float dt, int substeps, int nthreads, const int* cpus) {
    return b3w_run(scene, (B3World*)worlds, (const B3World*)initial, count, seed, t0, nsteps, dt,
        substeps, nthreads, cpus);
}
int ref_build_batch(int scene, void* worlds, int count, unsigned long long seed, int first) {
    for (int i = 0; i < count; i++)
        if (!b3s_build(scene, (B3World*)worlds + i, seed, first + i)) return 0;
    return 1;
}
